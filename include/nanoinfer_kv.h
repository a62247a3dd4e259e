/*
 * nanoinfer_kv.h -- C ABI of the MI355X (gfx950) paged f16 KV-cache hot path.
 *
 * A drop-in for the KV part of nanoinfer's batched engine: the page allocator
 * and block tables of `Batch` (crates/metal/src/batch.rs:129-254), the f16
 * append (crates/metal/src/shaders/batch.metal:329-344), the block-table
 * gather (batch.metal:24-26) and paged flash-decoding attention with split-K
 * partitions and a log-sum-exp merge (batch.metal:349-424, dispatched from
 * batch.rs:577-616).  Paths are relative to the reference repository.
 *
 * Conventions
 *  - Every call returns an int status (NI_OK or an NI_ERR_* code); the text
 *    of the last failure is ni_kv_last_error().  Where the reference returns
 *    Err(String) the text is the reference's.
 *  - The handle owns the device page pools and its staging buffers.  The
 *    caller owns every q/k/v/out buffer it passes (device memory).
 *  - One host thread per handle.  Data-path calls enqueue work on the
 *    caller's HIP stream (`ni_stream`, a hipStream_t; NULL = null stream) and
 *    return without waiting; ni_kv_sync() waits.
 *  - A handle's data-path calls run on the device in the order they are
 *    made, whatever streams they are made on (they share the handle's split
 *    partials, and a page that truncate or free_seq returns may go to the
 *    very next append).  A call on a stream other than the one that holds
 *    the handle's previous work makes its stream wait for that work first
 *    (an event recorded on the previous stream, then hipStreamWaitEvent).
 *    So a stream the handle's last call used must stay alive until the next
 *    call on another stream, or until ni_kv_sync(kv, that stream).  Calls on
 *    a stream that is capturing a graph are not ordered against other
 *    streams: the captured work runs when the caller replays the graph, and
 *    ordering replays is the caller's part.
 *  - Bookkeeping calls (add/free/truncate/reserve/commit) act on host state
 *    at once.  A data-path call snapshots the block tables it needs when it
 *    is made, so later bookkeeping never changes work already enqueued.
 *  - f32 arguments (q/k/v/out) must be 16-byte aligned with row and layer
 *    strides that are multiples of 4 floats.  Strides count elements.
 */
#ifndef NANOINFER_KV_H
#define NANOINFER_KV_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ni_kv ni_kv;
typedef void* ni_stream; /* hipStream_t */

/* Positions per page (crates/metal/src/batch.rs:33, KV_BLOCK). */
#define NI_KV_BLOCK 16
/* `layer` argument: every layer in each launch of the call (inputs at
 * base + l * layer_stride for l in 0..n_layer). */
#define NI_ALL_LAYERS (-1)

enum ni_status {
    NI_OK = 0,
    NI_ERR_NO_SLOT = 1,         /* add_seq: every sequence slot is live (batch.rs:201-202 -> None) */
    NI_ERR_CONTEXT_FULL = 2,    /* "sequence {s}: context full ({len} > {n_ctx})" (batch.rs:244-246) */
    NI_ERR_POOL_EXHAUSTED = 3,  /* "KV cache pool exhausted" (batch.rs:248) */
    NI_ERR_NOT_LIVE = 4,        /* "sequence {s} is not live" (batch.rs:281-283) */
    NI_ERR_BAD_LEN = 5,         /* truncate past seq_len: the reference's assert (batch.rs:221) */
    NI_ERR_HIP = 6,             /* a HIP runtime call failed */
    NI_ERR_BAD_ARG = 7,         /* bad sequence index, shape, alignment or option */
    NI_ERR_EMPTY_WORK = 8,      /* "empty work item" (batch.rs:284-286) */
    NI_ERR_TOO_MANY_ROWS = 9,   /* "{n} rows > max_rows {max}" (batch.rs:300-302) */
    NI_ERR_NOT_RESERVED = 10,   /* a row's position has no page yet (reserve first) */
    NI_ERR_NO_DEVICE = 11       /* data-path call on a NI_KV_HOST_ONLY handle */
};

/* ni_kv_opts.flags: keep only the host bookkeeping (no device memory); the
 * data-path calls then fail with NI_ERR_NO_DEVICE.  For tests without a GPU. */
#define NI_KV_HOST_ONLY 1u
/* ni_kv_opts.flags: the Q8 cache (crates/metal/src/shaders/kv8.metal:1-95):
 * each (position, head) of K and V is stored as head_dim int8 values and one
 * f32 scale = amax / 127 (68 bytes per 64 values instead of 128).  Appends
 * quantise (kv_quant8, :15-48; inputs must be finite), attention dequantises
 * (attn_decode_split_q8, :50-95); ni_kv_gather and ni_kv_qkv_append are
 * refused (ni_kv_gather_q8 returns the stored bytes). */
#define NI_KV_Q8 2u

/* Sizes and policies (the KV fields of BatchOpts, batch.rs:44-76, plus the
 * model shape the reference takes from Config, crates/core/src/config.rs:23). */
typedef struct ni_kv_opts {
    uint32_t n_layer;   /* layers sharing each page id (batch.rs:166,390) */
    uint32_t n_head;
    uint32_t head_dim;  /* 64 or 128 on the device path */
    uint32_t kv_pages;  /* pages in the pool (BatchOpts::kv_blocks) */
    uint32_t max_seqs;  /* sequence slots (BatchOpts::max_seqs) */
    uint32_t max_ctx;   /* most positions per sequence (Config::n_ctx) */
    uint32_t max_rows;  /* most rows per data-path call (BatchOpts::max_rows) */
    uint32_t flags;     /* NI_KV_HOST_ONLY */
    /* Optional (NULL = the reference's order 0, 1, 2, ...): a permutation of
     * 0..kv_pages-1 giving the order in which free pages are handed out. */
    const uint32_t* page_order;
} ni_kv_opts;

/* One row: token `pos` of sequence `seq` (batch.rs:112-117; sent to the
 * reference's kernels as uint4(seq, pos, 0, 0), batch.rs:306). */
typedef struct ni_row {
    uint32_t seq;
    uint32_t pos;
} ni_row;

/* One work item of ni_kv_step: append n_new rows to `seq` (positions
 * seq_len .. seq_len+n_new-1) and run attention for the last n_query of them
 * (batch.rs:259-315; n_query = n_new is the reference's all_logits). */
typedef struct ni_work {
    uint32_t seq;
    uint32_t n_new;
    uint32_t n_query;
} ni_work;

/* ---- lifecycle (BatchEngine::new + BatchEngine::batch, batch.rs:95-104,159-194) ---- */
int ni_kv_create(const ni_kv_opts* opts, ni_kv** out);
void ni_kv_destroy(ni_kv* kv);
/* Text of the last failure on this handle; with kv == NULL, of the last
 * failed ni_kv_create or ni_attention on this thread. */
const char* ni_kv_last_error(const ni_kv* kv);
/* Bytes of one page over all layers, K and V (BatchEngine::kv_block_bytes, batch.rs:107-109). */
size_t ni_kv_page_bytes(const ni_kv* kv);

/* ---- bookkeeping (batch.rs:200-254, 270) ---- */
int ni_kv_add_seq(ni_kv* kv, uint32_t* seq);                    /* Batch::add_seq, :201-206 */
int ni_kv_free_seq(ni_kv* kv, uint32_t seq);                    /* Batch::free_seq, :209-212 */
int ni_kv_seq_len(const ni_kv* kv, uint32_t seq, uint32_t* len); /* Batch::seq_len, :214-216 */
int ni_kv_is_live(const ni_kv* kv, uint32_t seq, int* live);     /* Batch::seq_live, :134 */
int ni_kv_truncate(ni_kv* kv, uint32_t seq, uint32_t len);       /* Batch::truncate, :220-227 */
int ni_kv_reserve(ni_kv* kv, uint32_t seq, uint32_t len);        /* Batch::ensure_blocks, :243-254 */
int ni_kv_commit(ni_kv* kv, uint32_t seq, uint32_t n);           /* seq_len += n, :270 */
/* Batch::block_table, :230-232.  *pages stays valid until the next
 * bookkeeping call on this handle. */
int ni_kv_block_table(const ni_kv* kv, uint32_t seq, const uint32_t** pages, uint32_t* n);
uint32_t ni_kv_blocks_used(const ni_kv* kv);      /* Batch::blocks_used, :235-237 */
uint32_t ni_kv_free_block_count(const ni_kv* kv); /* Batch::free_block_count, :238-240 */

/* ---- data path (device) ---- */

/* f32 K/V rows -> f16 (round to nearest even, quant.rs:25-54) into each
 * row's page slot (b_kv_write, batch.metal:329-344).  Row i of k/v is
 * rows[i]; layer l reads k + l*layer_stride (+ i*row_stride) when
 * layer == NI_ALL_LAYERS, else `layer` is the only layer written and k/v
 * point at its rows.  Positions must be reserved. */
int ni_kv_append(ni_kv* kv, int32_t layer, const ni_row* rows, uint32_t n, const float* k, const float* v,
                 int64_t row_stride, int64_t layer_stride, ni_stream stream);

/* The QKV projection with the append in its epilogue (the reference's
 * matvec_batch<..., BEPI_QKV>, batch.metal:94-165, dispatched per layer at
 * batch.rs:396-415): for row i, y = x_i W^T + bias with W [3C][d_in] f32
 * row-major (the reference's weight layout) and bias [3C] (NULL = none);
 * q = y[0, C) goes to q_out row i (f32), k = y[C, 2C) and v = y[2C, 3C) are
 * stored as f16 (round to nearest even) in rows[i]'s page slot of `layer`
 * (0 <= layer < n_layer) without passing through memory as f32.  Positions
 * must be reserved; d_in must be a multiple of 16; x, w and q_out 16-byte
 * aligned with strides that are multiples of 4 floats. */
int ni_kv_qkv_append(ni_kv* kv, int32_t layer, const ni_row* rows, uint32_t n, const float* x,
                     int64_t x_row_stride, uint32_t d_in, const float* w, const float* bias, float* q_out,
                     int64_t q_row_stride, ni_stream stream);

/* The same projection with every output to `out` ([n][3C] f32; the
 * reference's BEPI_PLAIN epilogue): the same kernel and arithmetic, so the
 * K/V bits ni_kv_qkv_append stores equal f32->f16 of out[:, C:3C]. */
int ni_kv_qkv_project(ni_kv* kv, const float* x, int64_t x_row_stride, uint32_t n, uint32_t d_in, const float* w,
                      const float* bias, float* out, int64_t out_row_stride, ni_stream stream);

/* The same two calls with W in one of the reference's weight formats (DType,
 * crates/metal/src/lib.rs:36-43, laid out as crates/metal/src/weights.rs:12-86
 * stores the row-major [3C][d_in] matrix; the BEPI_QKV matvec and GEMM
 * paths load them through BF32/BF16/BQ8/BQ4, batch.metal:45-90).  Each
 * weight is dequantised exactly into f32 (f16 widened, q * d, (q - 8) * d),
 * so the result has the bits of the f32 call on the dequantised matrix.
 * Block formats need d_in a multiple of 32; w 16-byte aligned. */
#define NI_W_F32 0u  /* [3C][d_in] f32 */
#define NI_W_F16 1u  /* [3C][d_in] f16 */
#define NI_W_Q8_0 2u /* [3C*d_in] int8, then [3C*d_in/32] f16 scales (quantize_q8_0) */
#define NI_W_Q4_0 3u /* [3C*d_in/2] bytes (byte i of a 32-block: element i in the low nibble, i+16 in the high),
                        then [3C*d_in/32] f16 scales (quantize_q4_0) */
int ni_kv_qkv_append_w(ni_kv* kv, int32_t layer, const ni_row* rows, uint32_t n, const float* x,
                       int64_t x_row_stride, uint32_t d_in, const void* w, uint32_t w_format, const float* bias,
                       float* q_out, int64_t q_row_stride, ni_stream stream);
int ni_kv_qkv_project_w(ni_kv* kv, const float* x, int64_t x_row_stride, uint32_t n, uint32_t d_in, const void* w,
                        uint32_t w_format, const float* bias, float* out, int64_t out_row_stride, ni_stream stream);

/* Block-table gather: f16 bits of K and V at (seq, pos) for each row, in the
 * reference's row layout [C] = [head][head_dim] (the reads of b_attn_split,
 * batch.metal:377,392, through kv_slot, :24-26).  Strides in halves. */
int ni_kv_gather(ni_kv* kv, int32_t layer, const ni_row* rows, uint32_t n, uint16_t* k_out, uint16_t* v_out,
                 int64_t row_stride, int64_t layer_stride, ni_stream stream);

/* Q8 handles: the stored int8 values [n_lay][n][C] (n_lay = n_layer for
 * NI_ALL_LAYERS, else 1) and scales [n_lay][n][n_head] of each row, dense;
 * k_out/v_out 16-byte aligned. */
int ni_kv_gather_q8(ni_kv* kv, int32_t layer, const ni_row* rows, uint32_t n, int8_t* k_out, int8_t* v_out,
                    float* k_scale, float* v_scale, ni_stream stream);

/* Paged decode attention (b_attn_split + b_attn_merge, batch.metal:349-424;
 * math of kv16.rs:144-164): row i attends causally to keys 0..rows[i].pos
 * of rows[i].seq; out row i = softmax(q.K^T / sqrt(head_dim)) V.  Keys are
 * split into partitions of `split_tokens` (a multiple of 16; 0 = automatic)
 * and merged by log-sum-exp.  Consecutive rows of one sequence at
 * consecutive positions (speculative verify, prefill chunks) share their
 * K/V reads. */
int ni_paged_decode_attention(ni_kv* kv, int32_t layer, const float* q, int64_t q_row_stride,
                              int64_t q_layer_stride, const ni_row* rows, uint32_t n, float* out,
                              int64_t out_row_stride, int64_t out_layer_stride, uint32_t split_tokens,
                              ni_stream stream);

/* One step of the hot path over every layer (Batch::step, batch.rs:259-315,
 * the KV part): for each work item in order check it (not live / empty /
 * context full / pool exhausted, the reference's errors and texts), reserve
 * pages, then append all rows and run attention for the queried rows, and
 * finally commit seq_len += n_new.  Rows are numbered in work order; row r
 * of layer l is at base + l*layer_stride + r*row_stride in q/k/v and out. */
int ni_kv_step(ni_kv* kv, const ni_work* work, uint32_t n_work, const float* q, const float* k, const float* v,
               int64_t row_stride, int64_t layer_stride, float* out, int64_t out_row_stride,
               int64_t out_layer_stride, uint32_t split_tokens, ni_stream stream);

/* ni_kv_step that allocates nothing.  No counterpart in the reference: it is
 * for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  Same
 * arguments, checks, errors and results as ni_kv_step (the same kernels over
 * the same plan), but no hipMalloc, hipFree, staging upload or event
 * creation: the split-K partials live in a file-scope device array of
 * 32 MiB, one per GPU, held until the process ends, and the plan travels in
 * the launch arguments.  A step whose plan exceeds 32 KB or whose partials
 * exceed 32 MiB returns NI_ERR_BAD_ARG with the limit in the message (its
 * pages stay reserved, as after any failed launch; nothing is launched).
 * The first handle to call it on a GPU holds that GPU's array until
 * ni_kv_destroy (which first waits for the handle's work); calls through
 * any other handle on that GPU meanwhile return NI_ERR_BAD_ARG.  The
 * holder's calls are ordered (see the conventions above), but replays of
 * graphs captured from them that overlap on the GPU race.  ni_kv_profile
 * does not time the launches of this call (timing would take events from
 * the handle's pool, which may create them). */
int ni_kv_step_noalloc(ni_kv* kv, const ni_work* work, uint32_t n_work, const float* q, const float* k,
                       const float* v, int64_t row_stride, int64_t layer_stride, float* out, int64_t out_row_stride,
                       int64_t out_layer_stride, uint32_t split_tokens, ni_stream stream);

/* The same step one layer at a time, as a model's forward runs it: the
 * reference encodes a step once (Batch::encode_step, batch.rs:280-306: check,
 * reserve, lay out the rows) and then dispatches each layer's KV write and
 * attention between that layer's other kernels (batch.rs:390-416).
 * ni_kv_step_begin checks the work items and reserves pages exactly as
 * ni_kv_step (same errors; nothing is open after an error) and plans the step
 * once; ni_kv_step_layer(layer) then appends that layer's new rows and runs
 * its attention over that plan, in one launch (a step of prompt chunks that
 * are queried at every row: an append launch, then the prefill launch)
 * (q/k/v/out hold the layer's rows
 * only, row r at base + r*row_stride); ni_kv_step_end commits seq_len +=
 * n_new.  Layers may come in any order, each once, all on the stream of
 * the first layer's call (the layers share the step's plan and split
 * partials; another stream returns NI_ERR_BAD_ARG and nothing is
 * launched).  While a step is open, ni_kv_step, ni_kv_decode_steps,
 * ni_kv_truncate, ni_kv_free_seq and ni_kv_commit return NI_ERR_BAD_ARG. */
int ni_kv_step_begin(ni_kv* kv, const ni_work* work, uint32_t n_work, uint32_t split_tokens);
int ni_kv_step_layer(ni_kv* kv, int32_t layer, const float* q, const float* k, const float* v, int64_t row_stride,
                     float* out, int64_t out_row_stride, ni_stream stream);
int ni_kv_step_end(ni_kv* kv);

/* Batch::decode_resident's KV part (batch.rs:322-363): `steps` decode steps
 * of the sequences seqs[0..n), enqueued at once with no host wait.  Pages
 * for every step are reserved first (each sequence to seq_len + steps; the
 * reference's errors, nothing enqueued on error); step t then appends one
 * row per sequence at position seq_len + t and runs its attention, and
 * seq_len += 1 after each step.  Row i of step t, layer l is at
 * base + t*step_stride + l*layer_stride + i*row_stride in q/k/v (out with
 * the out_ strides).  In a model, step t's q/k/v come from step t-1's
 * output; here the caller provides them. */
int ni_kv_decode_steps(ni_kv* kv, const uint32_t* seqs, uint32_t n, uint32_t steps, const float* q, const float* k,
                       const float* v, int64_t row_stride, int64_t layer_stride, int64_t step_stride, float* out,
                       int64_t out_row_stride, int64_t out_layer_stride, int64_t out_step_stride,
                       uint32_t split_tokens, ni_stream stream);

/* Wait for all work this handle enqueued on `stream`; afterwards no call of
 * the handle waits for that work, and `stream` may be destroyed. */
int ni_kv_sync(ni_kv* kv, ni_stream stream);

/* The device pool, for inspection: one allocation of `bytes`, laid out
 * [n_layer][kv_pages][n_head][K block][V block]; *k_pool is its start and
 * *v_pool the first V block.  f16: a block is [16][head_dim] f16.  Q8: a
 * block is [16][head_dim] int8 then 16 f32 scales. */
int ni_kv_pools(const ni_kv* kv, void** k_pool, void** v_pool, size_t* bytes);

/* Contiguous causal attention over f32 K/V rows, the CPU engine's op
 * Kernels::attention(out, q: Rows, k: Rows, v: Rows, n_q, q_pos0, n_head,
 * head_dim, scores) (crates/core/src/kernels/mod.rs:86-98; what it computes:
 * reference::attention, kernels/reference.rs:109-142): query i at position
 * q_pos0 + i attends to rows 0 .. q_pos0 + i;
 * out[i][h*hd + d] = softmax(q_i,h . K_h^T / sqrt(hd)) V_h.  Row j of head h
 * of K is at k + j*k_stride + h*head_dim (a Rows{data, stride}); q, v and
 * out alike.  No scores buffer: the device keeps a running softmax.  Keys
 * past q_pos0 + n_q - 1 are never read.  head_dim 64 or 128; pointers
 * 16-byte aligned, strides multiples of 4 floats.  Enqueued on `stream`;
 * failures are reported by ni_kv_last_error(NULL). */
int ni_attention(float* out, int64_t out_stride, const float* q, int64_t q_stride, const float* k, int64_t k_stride,
                 const float* v, int64_t v_stride, uint32_t n_q, uint32_t q_pos0, uint32_t n_head, uint32_t head_dim,
                 ni_stream stream);

/* quant.rs:25-54 on the device, elementwise (the conversion the append uses). */
int ni_f32_to_f16(const float* in, uint16_t* out, size_t n, ni_stream stream);

/* ---- measurement ---- */
/* The streaming rate the hot path is held against (no counterpart in the
 * reference): `blocks` workgroups of 256 threads walk `bytes` (a multiple of
 * 16, at least blocks * 4096) of src in 16-byte non-temporal loads.
 * mode & NI_PROBE_COPY: each unit is also stored to dst (bytes long); else a
 * read only (dst, at least bytes long, is in practice not written).
 * mode & NI_PROBE_SPAN: each workgroup walks one contiguous span of the
 * buffer; else a grid stride.  Enqueued on `stream`; time it with events. */
#define NI_PROBE_COPY 1u
#define NI_PROBE_SPAN 2u
int ni_stream_probe(uint32_t mode, const void* src, void* dst, size_t bytes, uint32_t blocks, ni_stream stream);

/* HIP event timestamps of this handle's kernel launches. */
enum ni_kernel_id { NI_K_APPEND = 0, NI_K_ATTN = 1, NI_K_MERGE = 2, NI_K_QKV = 3, NI_K_COUNT = 4 };
/* Bit k of kernel_mask times every launch of kernel k (ni_kernel_id): the
 * dispatch itself records the kernel's start and end into a pair of HIP
 * events (hipExtLaunchKernelGGL), so the time is the kernel's own, with no
 * extra commands in the stream; 0 stops.  NI_K_ATTN is the attention launch
 * (with the append fused into it when ni_kv_step fuses). */
int ni_kv_profile(ni_kv* kv, uint32_t kernel_mask);
/* Total milliseconds and launches of one kernel since the last read (waits). */
int ni_kv_profile_read(ni_kv* kv, int kernel, double* total_ms, uint64_t* launches);

const char* ni_version(void);

#ifdef __cplusplus
}
#endif
#endif /* NANOINFER_KV_H */
