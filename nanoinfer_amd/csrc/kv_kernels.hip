// kv_kernels.hip -- gfx950 (MI355X) kernels of the paged f16 KV-cache path.
//
// Pool layout (device): one allocation [n_layer][kv_pages][n_head][K|V][16][D]
// f16.  One (page, head) block of K is 16*D halves contiguous (2 KB at D = 64)
// and its V block follows it, so a wave64 reading a block with 16-byte lanes
// moves 1 KB per load instruction with every lane on consecutive bytes.  The
// reference keeps [page][16][C] (crates/metal/src/batch.rs:166); values are
// identical per (seq, pos, head, d), only the placement differs.
//
// Kernels:
//   kv_append_kernel   f32 K/V rows -> f16 page slots (b_kv_write, batch.metal:329-344)
//   kv_gather_kernel   page slots -> f16 rows in the reference layout (kv_slot reads, :24-26)
//   attn_split_kernel  paged flash-decoding of single query rows, one workgroup
//                      per (item, layer, head) (b_attn_split, batch.metal:349-400),
//                      with the step's append fused in (head_dim 64: the new
//                      rows taken from the input as their pages stream)
//   attn_mfma_kernel   the same for groups of 2..16 causal query rows of one
//                      sequence, on the matrix cores
//   attn_prefill_kernel  groups of 17..64 rows (prompt chunks), K/V tiles DMA'd
//                      into an LDS ring shared by four waves (attn.metal:100-222)
//   attn_prefill_q8_kernel  the same on the Q8 cache; in a step of prompt
//                      chunks only, a workgroup runs one sequence's groups,
//                      appending the rows each needs first
//   attn_q8_kernel     single rows on the int8 + scale (Q8) cache (kv8.metal)
//   attn_merge_kernel  log-sum-exp merge of partitions (b_attn_merge, :403-424)
//   qkv_kernel         the QKV projection with the append in its epilogue
//                      (matvec_batch<..., BEPI_QKV>, batch.metal:94-165); with
//                      qkv_small_kernel (up to 16 rows) and qkv_mid_kernel
//                      (17..64 rows), the same arithmetic at every row count
//   attn_rows_kernel   contiguous f32 attention (Kernels::attention)
//
// Decode is HBM-bound streaming of f16 (or int8) K/V.  Arithmetic is f32 (the
// matrix-core kernels carry f32 operands as f16 hi + lo parts); softmax runs
// in the base-2 domain (scores pre-scaled by log2(e)/sqrt(D)).
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <cstring>
#include <mutex>
#include <vector>

#include "kv_plan.h"

namespace ni {
namespace {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));

// f32 -> f16 bits with round to nearest even (the hardware conversion under
// the default rounding mode keeps f16 subnormals and overflows to inf), NaN
// made canonical sign|0x7e00 -- the rules of crates/core/src/quant.rs:25-54.
__device__ __forceinline__ uint32_t f16_bits(float x) {
    uint32_t h = __builtin_bit_cast(uint16_t, static_cast<_Float16>(x));
    const uint32_t b = __float_as_uint(x);
    if ((b & 0x7fffffffu) > 0x7f800000u) h = ((b >> 16) & 0x8000u) | 0x7e00u;
    return h;
}

__device__ __forceinline__ uint4 pack8(const float4 a, const float4 b) {
    uint4 r;
    r.x = f16_bits(a.x) | (f16_bits(a.y) << 16);
    r.y = f16_bits(a.z) | (f16_bits(a.w) << 16);
    r.z = f16_bits(b.x) | (f16_bits(b.y) << 16);
    r.w = f16_bits(b.z) | (f16_bits(b.w) << 16);
    return r;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Cross-lane move inside a row of 16 lanes (DPP; no LDS traffic).
template <int CTRL>
__device__ __forceinline__ float dpp_move(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}

// Sum over the LPK consecutive lanes that hold one key row (LPK = 8 or 16).
template <int LPK>
__device__ __forceinline__ float key_sum(float x) {
    x += dpp_move<0xb1>(x);                            // quad_perm(1,0,3,2): lane ^ 1
    x += dpp_move<0x4e>(x);                            // quad_perm(2,3,0,1): lane ^ 2
    if constexpr (LPK >= 8) x += dpp_move<0x141>(x);   // row_half_mirror: the other quad of 8
    if constexpr (LPK >= 16) x += dpp_move<0x140>(x);  // row_mirror: the other 8 of 16
    return x;
}

// (m, l, o) <- (m, l, o) (+) (m2, l2, o2): the log-sum-exp merge of two
// partial softmax states (batch.metal:415-423), base 2.
template <int N>
__device__ __forceinline__ void merge_state(float& m, float& l, float (&o)[N], float m2, float l2,
                                            const float (&o2)[N]) {
    const float mn = fmaxf(m, m2);
    const float a1 = fast_exp2(m - mn), a2 = fast_exp2(m2 - mn);
    l = l * a1 + l2 * a2;
#pragma unroll
    for (int e = 0; e < N; e++) o[e] = o[e] * a1 + o2[e] * a2;
    m = mn;
}

// Running max starts at a finite sentinel so that exp2(m - m_new) of two
// empty states is 1 (not NaN); masked scores are -inf and weigh 0.
constexpr float kMinScore = -1e30f;

// A plan passed with the kernel arguments (N > 0) or left in device memory
// (N == 0: the launch struct's `plan` pointer).  Arguments live in the
// read-only kernarg segment; the kernels index it in place.
template <int N>
struct PlanArg {
    uint8_t b[N > 0 ? N : 4];
};

template <int N>
__device__ __forceinline__ const uint8_t* plan_base(const PlanArg<N>& pa, const uint8_t* dev) {
    if constexpr (N > 0)
        return pa.b;
    else
        return dev;
}

// ------------------------------------------------------------------ append

// One thread's share of an append: 8 elements (two float4 loads, one 16-byte
// store) of K or V of one row of one layer.  `gid` enumerates
// [layer][row][K then V][C/8] over the n_rows entries.
template <bool IDX_SRC = false>
__device__ __forceinline__ void append_chunk(const PoolGeom& pool, const float* k, const float* v, int64_t row_stride,
                                             int64_t layer_stride, const AppendEntry* entries, uint32_t n_rows,
                                             uint32_t layer0, uint32_t n_lay, uint32_t gid) {
    const uint32_t D = pool.head_dim;
    const uint32_t chunks = (pool.n_head * D) >> 3;  // 8 elements per thread
    const uint32_t per_row = 2 * chunks;               // K then V
    const uint32_t per_layer = per_row * n_rows;
    if (gid >= per_layer * n_lay) return;
    const uint32_t lay = gid / per_layer;
    uint32_t r = gid - lay * per_layer;
    const uint32_t row = r / per_row;
    r -= row * per_row;
    const uint32_t is_v = r >= chunks;
    const uint32_t c8 = (r - is_v * chunks) * 8;
    const AppendEntry e = entries[row];
    // IDX_SRC: entry i reads input row i (a step's own append list), so the
    // input load need not wait for the entry's.
    const float* src =
        (is_v ? v : k) + (int64_t)lay * layer_stride + (int64_t)(IDX_SRC ? row : e.src_row) * row_stride + c8;
    const float4 x0 = reinterpret_cast<const float4*>(src)[0];
    const float4 x1 = reinterpret_cast<const float4*>(src)[1];
    const uint32_t head = c8 / D, d0 = c8 - head * D;
    uint16_t* dst = (is_v ? pool.v : pool.k) + (uint64_t)(layer0 + lay) * pool.layer_halves +
                    (uint64_t)e.page * pool.page_halves + (uint64_t)head * pool.head_halves + e.slot * D + d0;
    *reinterpret_cast<uint4*>(dst) = pack8(x0, x1);
}

// ----------------------------------------------------------- Q8 cache
//
// kv_quant8 (crates/metal/src/shaders/kv8.metal:15-48): each (position,
// head) of K or V is stored as int8 with one f32 scale, scale = amax / 127,
// q = clamp(rint(x * (1 / scale)), -127, 127) (inverse 0 when amax is 0);
// both divisions correctly rounded, rint to nearest even.  Inputs must be
// finite.

// A (page, head) block of a Q8 pool as bytes: [16][D] int8, then 16 scales.
__device__ __forceinline__ uint8_t* q8_block(const PoolGeom& pool, bool is_v, uint64_t off_halves) {
    return reinterpret_cast<uint8_t*>((is_v ? pool.v : pool.k) + off_halves);
}

__device__ __forceinline__ uint32_t q8_byte(float x, float inv) {
    return (uint32_t)(int32_t)fminf(fmaxf(rintf(x * inv), -127.f), 127.f) & 0xffu;
}

// Quantise 8 values of one (position, head) held by a lane whose aligned
// group of g = D/8 neighbouring lanes holds the rest; stores the 8 bytes at
// blk + slot*D + d0 and (lane d0 == 0) the scale.
__device__ __forceinline__ void q8_store8(uint8_t* blk, uint32_t D, uint32_t slot, uint32_t d0, const float4 x0,
                                          const float4 x1) {
    float a = fmaxf(fmaxf(fmaxf(fabsf(x0.x), fabsf(x0.y)), fmaxf(fabsf(x0.z), fabsf(x0.w))),
                    fmaxf(fmaxf(fabsf(x1.x), fabsf(x1.y)), fmaxf(fabsf(x1.z), fabsf(x1.w))));
    for (uint32_t off = 1; off < D / 8; off <<= 1) a = fmaxf(a, __shfl_xor(a, off));
    const float scale = a / 127.f;
    const float inv = scale > 0.f ? 1.f / scale : 0.f;
    uint2 q;
    q.x = q8_byte(x0.x, inv) | q8_byte(x0.y, inv) << 8 | q8_byte(x0.z, inv) << 16 | q8_byte(x0.w, inv) << 24;
    q.y = q8_byte(x1.x, inv) | q8_byte(x1.y, inv) << 8 | q8_byte(x1.z, inv) << 16 | q8_byte(x1.w, inv) << 24;
    *reinterpret_cast<uint2*>(blk + slot * D + d0) = q;
    if (d0 == 0) reinterpret_cast<float*>(blk + kPage * D)[slot] = scale;
}

// append_chunk for a Q8 pool: the same enumeration; the D/8 lanes of one
// (layer, row, K|V, head) are consecutive and aligned, and whole groups
// leave together at the end of the grid.
template <bool IDX_SRC = false>
__device__ __forceinline__ void append_chunk_q8(const PoolGeom& pool, const float* k, const float* v, int64_t row_stride,
                                                int64_t layer_stride, const AppendEntry* entries, uint32_t n_rows,
                                                uint32_t layer0, uint32_t n_lay, uint32_t gid) {
    const uint32_t D = pool.head_dim;
    const uint32_t chunks = (pool.n_head * D) >> 3;
    const uint32_t per_row = 2 * chunks;
    const uint32_t per_layer = per_row * n_rows;
    if (gid >= per_layer * n_lay) return;
    const uint32_t lay = gid / per_layer;
    uint32_t r = gid - lay * per_layer;
    const uint32_t row = r / per_row;
    r -= row * per_row;
    const uint32_t is_v = r >= chunks;
    const uint32_t c8 = (r - is_v * chunks) * 8;
    const AppendEntry e = entries[row];
    // IDX_SRC: entry i reads input row i (a step's own append list), so the
    // input load need not wait for the entry's.
    const float* src =
        (is_v ? v : k) + (int64_t)lay * layer_stride + (int64_t)(IDX_SRC ? row : e.src_row) * row_stride + c8;
    const float4 x0 = reinterpret_cast<const float4*>(src)[0];
    const float4 x1 = reinterpret_cast<const float4*>(src)[1];
    const uint32_t head = c8 / D, d0 = c8 - head * D;
    uint8_t* blk = q8_block(pool, is_v, (uint64_t)(layer0 + lay) * pool.layer_halves +
                                            (uint64_t)e.page * pool.page_halves + (uint64_t)head * pool.head_halves);
    q8_store8(blk, D, e.slot, d0, x0, x1);
}

template <int INL>
__global__ __launch_bounds__(256) void kv_append_kernel(const AppendLaunch a, const PlanArg<INL> pa) {
    const AppendEntry* entries = reinterpret_cast<const AppendEntry*>(plan_base(pa, a.plan) + a.off_entries);
    if (a.pool.q8)
        append_chunk_q8<true>(a.pool, a.k, a.v, a.row_stride, a.layer_stride, entries, a.n_rows, a.layer0, a.n_lay,
                              blockIdx.x * 256u + threadIdx.x);
    else
        append_chunk<true>(a.pool, a.k, a.v, a.row_stride, a.layer_stride, entries, a.n_rows, a.layer0, a.n_lay,
                     blockIdx.x * 256u + threadIdx.x);
}

// One thread per (layer, row, K|V, head): D int8 values and the scale.
template <int INL>
__global__ __launch_bounds__(256) void kv_gather_q8_kernel(const GatherQ8Launch a, const PlanArg<INL> pa) {
    const uint32_t D = a.pool.head_dim, H = a.pool.n_head;
    const uint32_t gid = blockIdx.x * 256u + threadIdx.x;
    const uint32_t per_layer = a.n_rows * 2 * H;
    if (gid >= per_layer * a.n_lay) return;
    const uint32_t lay = gid / per_layer;
    uint32_t r = gid - lay * per_layer;
    const uint32_t row = r / (2 * H);
    r -= row * 2 * H;
    const uint32_t is_v = r >= H;
    const uint32_t head = r - is_v * H;
    const AppendEntry e = reinterpret_cast<const AppendEntry*>(plan_base(pa, a.plan) + a.off_entries)[row];
    const uint8_t* blk = q8_block(a.pool, is_v, (uint64_t)(a.layer0 + lay) * a.pool.layer_halves +
                                                    (uint64_t)e.page * a.pool.page_halves +
                                                    (uint64_t)head * a.pool.head_halves);
    const uint64_t orow = ((uint64_t)lay * a.n_rows + e.src_row);
    int8_t* dst = (is_v ? a.v_out : a.k_out) + orow * H * D + head * D;
    for (uint32_t c = 0; c < D; c += 16)
        *reinterpret_cast<uint4*>(dst + c) = *reinterpret_cast<const uint4*>(blk + e.slot * D + c);
    (is_v ? a.v_scale : a.k_scale)[orow * H + head] = reinterpret_cast<const float*>(blk + kPage * D)[e.slot];
}

template <int INL>
__global__ __launch_bounds__(256) void kv_gather_kernel(const GatherLaunch a, const PlanArg<INL> pa) {
    const uint32_t D = a.pool.head_dim;
    const uint32_t chunks = (a.pool.n_head * D) >> 3;
    const uint32_t per_row = 2 * chunks;
    const uint32_t per_layer = per_row * a.n_rows;
    const uint32_t gid = blockIdx.x * 256u + threadIdx.x;
    if (gid >= per_layer * a.n_lay) return;
    const uint32_t lay = gid / per_layer;
    uint32_t r = gid - lay * per_layer;
    const uint32_t row = r / per_row;
    r -= row * per_row;
    const uint32_t is_v = r >= chunks;
    const uint32_t c8 = (r - is_v * chunks) * 8;
    const AppendEntry e = reinterpret_cast<const AppendEntry*>(plan_base(pa, a.plan) + a.off_entries)[row];
    const uint32_t head = c8 / D, d0 = c8 - head * D;
    const uint16_t* src = (is_v ? a.pool.v : a.pool.k) + (uint64_t)(a.layer0 + lay) * a.pool.layer_halves +
                          (uint64_t)e.page * a.pool.page_halves + (uint64_t)head * a.pool.head_halves + e.slot * D + d0;
    uint16_t* dst = (is_v ? a.v_out : a.k_out) + (int64_t)lay * a.layer_stride + (int64_t)e.src_row * a.row_stride + c8;
    *reinterpret_cast<uint4*>(dst) = *reinterpret_cast<const uint4*>(src);
}

__global__ __launch_bounds__(256) void f32_to_f16_kernel(const float* __restrict__ in, uint16_t* __restrict__ out,
                                                         size_t n) {
    const size_t i = (size_t)blockIdx.x * 256u + threadIdx.x;
    if (i < n) out[i] = static_cast<uint16_t>(f16_bits(in[i]));
}

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// ------------------------------------------------------- bandwidth probe

// The memory system's streaming rate, beside which the hot path's roofline
// fraction is read.  Threads move 16-byte units with non-temporal loads, 4
// independent ones in flight per iteration.  SPAN = false: a grid stride
// (unit i, i + G, ... for G threads in the grid); SPAN = true: workgroup b
// walks its own contiguous 1/gridDim of the buffer, 16 KB per iteration
// (the kind of run the attention kernel reads: whole blocks).  COPY stores
// each unit to dst; otherwise the units are folded and the fold is stored
// only if it equals a value it cannot reach in practice (the loads stay,
// nothing is written).
template <bool COPY, bool SPAN>
__global__ __launch_bounds__(256) void stream_kernel(const u32x4* __restrict__ src, u32x4* __restrict__ dst,
                                                     uint64_t n16) {
    uint64_t i, end, stride;
    if (SPAN) {
        const uint64_t span = (n16 + gridDim.x - 1) / gridDim.x;
        i = (uint64_t)blockIdx.x * span + threadIdx.x;
        end = min((uint64_t)(blockIdx.x + 1) * span, n16);
        stride = 256;
    } else {
        i = (uint64_t)blockIdx.x * 256u + threadIdx.x;
        end = n16;
        stride = (uint64_t)gridDim.x * 256u;
    }
    u32x4 acc = {0u, 0u, 0u, 0u};
    for (; i + 3 * stride < end; i += 4 * stride) {
        u32x4 a = __builtin_nontemporal_load(src + i);
        u32x4 b = __builtin_nontemporal_load(src + i + stride);
        u32x4 c = __builtin_nontemporal_load(src + i + 2 * stride);
        u32x4 d = __builtin_nontemporal_load(src + i + 3 * stride);
        if (COPY) {
            __builtin_nontemporal_store(a, dst + i);
            __builtin_nontemporal_store(b, dst + i + stride);
            __builtin_nontemporal_store(c, dst + i + 2 * stride);
            __builtin_nontemporal_store(d, dst + i + 3 * stride);
        } else {
            acc ^= a ^ b ^ c ^ d;
        }
    }
    for (; i < end; i += stride) {
        u32x4 a = __builtin_nontemporal_load(src + i);
        if (COPY)
            __builtin_nontemporal_store(a, dst + i);
        else
            acc ^= a;
    }
    if (!COPY && acc.x == 0x9e3779b9u && acc.y == 0x7f4a7c15u && acc.z == 0x85ebca6bu && acc.w == 0xc2b2ae35u)
        dst[(uint64_t)blockIdx.x * 256u + threadIdx.x] = acc;
}

// --------------------------------------------------------------- attention

// Shape of the split kernel's launches (measured best on MI355X for the
// GPT-2 and long-context shapes).
constexpr int kWaves = 4;         // waves per workgroup sharing one item's pages
constexpr int kPagesPerIter = 2;  // pages per wave per loop iteration (head_dim 64)
constexpr int kPagesD128 = 2;     // the same at head_dim 128

// K/V loads are non-temporal: each byte is streamed once per step (156 -> 140
// us per config-3 launch against ordinary loads).
__device__ __forceinline__ u32x4 load16(const u32x4* p) { return __builtin_nontemporal_load(p); }

// The (item, layer, head) unit workgroup b of an attention launch runs:
// unit b itself (item-major, b = (item * n_lay + layer) * n_head + head), or
// in a balanced wide launch the plan's block -> unit table (the blocks a CU
// receives then carry an even share of the launch's pages).
struct AttnUnit {
    uint32_t item, lay, head;
};
__device__ __forceinline__ AttnUnit attn_unit(const AttnLaunch& a, const uint8_t* plan, uint32_t b) {
    const uint32_t H = a.pool.n_head;
    const uint32_t lh = a.n_lay * H;
    const uint32_t u = a.ordered ? (uint32_t)reinterpret_cast<const uint16_t*>(plan + a.off_order)[b] : b;
    AttnUnit r;
    r.item = u / lh;
    const uint32_t rem = u - r.item * lh;
    r.lay = rem / H;
    r.head = rem - r.lay * H;
    return r;
}

// Fused append of one item: this step's new rows in [kv_begin, kv_end),
// this (layer, head)'s slice.  No other workgroup of the launch reads or
// writes these blocks and the vector L1 starts the kernel clean, so after a
// barrier the workgroup's loads see its own stores.
template <int D>
__device__ __forceinline__ void item_append(const AttnLaunch& a, const uint8_t* plan, const AttnItem& it, uint32_t lay,
                                            uint32_t head, uint64_t layer_off, uint64_t page_stride, uint32_t nthreads) {
    constexpr uint32_t CH = D / 8;  // 16-byte chunks per row of one head
    for (uint32_t t = threadIdx.x; t < it.napp * 2 * CH; t += nthreads) {
        const uint32_t row = t / (2 * CH);
        const uint32_t rem2 = t - row * (2 * CH);
        const uint32_t is_v = rem2 >= CH;
        const uint32_t c = (rem2 - is_v * CH) * 8;
        const AppendEntry e = reinterpret_cast<const AppendEntry*>(plan + a.off_app)[it.app0 + row];
        // (append entry i reads input row i: the load need not wait for e)
        const float* src = (is_v ? a.v : a.k) + (int64_t)lay * a.kv_layer_stride +
                           (int64_t)(it.app0 + row) * a.kv_row_stride + head * D + c;
        const float4 x0 = reinterpret_cast<const float4*>(src)[0];
        const float4 x1 = reinterpret_cast<const float4*>(src)[1];
        uint16_t* dst = (is_v ? a.pool.v : a.pool.k) + layer_off + (uint64_t)e.page * page_stride + e.slot * D + c;
        *reinterpret_cast<uint4*>(dst) = pack8(x0, x1);
    }
}

// K and V chunks of PB pages for one lane: page pg+b, load i covers key rows
// i*KPL .. i*KPL+KPL-1 of the page.  Pages past pg_end read as zeros.
template <int PB, int LPP>
struct PageRegs {
    u32x4 k[PB][LPP];
    u32x4 v[PB][LPP];
};

// A fused launch's new rows of one item, (layer, head): positions pos ..
// pos+n-1, K/V input rows k/v + (p - pos) * row_stride (already offset to the
// lane's 8 dims).  The wave that streams their page takes them from the input
// (converted as the append converts them), stores them to the pool and uses
// them: no separate append before the attention, no barrier.
struct NewRows {
    const float* k;
    const float* v;
    int64_t row_stride;
    uint32_t pos, n;
};

template <int PB, int LPP>
__device__ __forceinline__ void load_pages(PageRegs<PB, LPP>& r, const uint32_t* __restrict__ tab, uint32_t pg,
                                           uint32_t pg_end, const uint16_t* __restrict__ kbase,
                                           const uint16_t* __restrict__ vbase, uint64_t page_stride, int lane,
                                           const NewRows& nr, int kl) {
    constexpr uint32_t KPL = kPage / LPP;  // key rows per load
#pragma unroll
    for (int b = 0; b < PB; b++) {
        if (pg + b < pg_end) {
            const uint64_t phys = tab[pg + b];
            const u32x4* kp = reinterpret_cast<const u32x4*>(kbase + phys * page_stride) + lane;
            const u32x4* vp = reinterpret_cast<const u32x4*>(vbase + phys * page_stride) + lane;
            const uint32_t p0 = (pg + b) * kPage;
            if (nr.n && p0 < nr.pos + nr.n && p0 + kPage > nr.pos) {  // wave-uniform: the page holds new rows
#pragma unroll
                for (int i = 0; i < LPP; i++) {
                    const uint32_t d = p0 + i * KPL + kl - nr.pos;  // unsigned: >= n unless new
                    if (d < nr.n) {
                        const float4* ks = reinterpret_cast<const float4*>(nr.k + (int64_t)d * nr.row_stride);
                        const float4* vs = reinterpret_cast<const float4*>(nr.v + (int64_t)d * nr.row_stride);
                        const uint4 kw = pack8(ks[0], ks[1]), vw = pack8(vs[0], vs[1]);
                        *const_cast<uint4*>(reinterpret_cast<const uint4*>(kp + i * 64)) = kw;
                        *const_cast<uint4*>(reinterpret_cast<const uint4*>(vp + i * 64)) = vw;
                        r.k[b][i] = u32x4{kw.x, kw.y, kw.z, kw.w};
                        r.v[b][i] = u32x4{vw.x, vw.y, vw.z, vw.w};
                    } else {
                        r.k[b][i] = load16(kp + i * 64);
                        r.v[b][i] = load16(vp + i * 64);
                    }
                }
                continue;
            }
#pragma unroll
            for (int i = 0; i < LPP; i++) {
                r.k[b][i] = load16(kp + i * 64);
                r.v[b][i] = load16(vp + i * 64);
            }
        } else {
#pragma unroll
            for (int i = 0; i < LPP; i++) {
                r.k[b][i] = u32x4{0, 0, 0, 0};
                r.v[b][i] = u32x4{0, 0, 0, 0};
            }
        }
    }
}

// One workgroup = W waves = one (item, layer, head).  Waves take the item's
// pages round-robin, PB pages per iteration.  Inside a wave, lane l reads 16
// bytes (8 halves) of key row kl = l / LPK, dims ds*8 .. ds*8+7 (ds = l % LPK):
// one load instruction covers KPL = 64 / LPK key rows, a page LPP = 16 / KPL
// loads.  Each lane keeps its own flash state (m, l, o[8]) per query over the
// keys its key-row group sees; the groups are merged once at the end (wave
// shuffles, then LDS across waves).
// Waves per SIMD the wide (8-wave, one-layer) workgroups' registers must allow:
// with one page per iteration (kWidePages) the fused kernel fits 80 VGPRs
// without spilling, so a layer's 768 workgroups of config 3 (64 sequences x
// 12 heads) are all resident at once instead of 512 and then a tail of 256:
// one launch per layer 3711 -> 4183 GB/s (two pages per iteration, 119
// VGPRs, 4 waves per SIMD, before).
constexpr int kWideMinWaves = 6;
// Pages per wave iteration of the wide launches (two, at 119 VGPRs and 4
// waves per SIMD: 3711 against 4183 GB/s; separate append + attention calls
// per layer 3501 against 3780).
constexpr int kWidePages = 1;
template <int D, int NQ, int W, int PB, bool FUSED, int INL>
__global__ __launch_bounds__(64 * W, W == 8 ? kWideMinWaves : 1) void attn_split_kernel(const AttnLaunch a,
                                                                                            const PlanArg<INL> pa) {
    constexpr int LPK = D / 8;
    constexpr int KPL = 64 / LPK;
    constexpr int LPP = kPage / KPL;
    __shared__ float red[W][NQ][D + 2];

    const int lane = threadIdx.x & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t H = a.pool.n_head;
    const uint32_t lh = a.n_lay * H;
    const uint8_t* plan = plan_base(pa, a.plan);
    if constexpr (FUSED) {
        // Blocks past the items' append the rows of sequences without queries.
        const uint32_t n_attn = a.n_items * lh;
        if (blockIdx.x >= n_attn) {
            const uint32_t base = (blockIdx.x - n_attn) * (64u * W);
            append_chunk(a.pool, a.k, a.v, a.kv_row_stride, a.kv_layer_stride,
                         reinterpret_cast<const AppendEntry*>(plan + a.off_orphans), a.n_orphans, a.layer0,
                         a.n_lay, base + threadIdx.x);
            return;
        }
    }
    const AttnUnit un = attn_unit(a, plan, blockIdx.x);
    const uint32_t item_i = un.item, lay = un.lay, head = un.head;
    const AttnItem it = reinterpret_cast<const AttnItem*>(plan + a.off_items)[item_i];
    const int kl = lane / LPK;
    const int ds = lane % LPK;

    const uint64_t layer_off = (uint64_t)(a.layer0 + lay) * a.pool.layer_halves + (uint64_t)head * a.pool.head_halves;
    const uint16_t* kbase = a.pool.k + layer_off;
    const uint16_t* vbase = a.pool.v + layer_off;
    const uint64_t page_stride = a.pool.page_halves;
    const uint32_t* __restrict__ tab = reinterpret_cast<const uint32_t*>(plan + a.off_table) + it.tab;
    const uint32_t pg_begin = it.kv_begin / kPage;
    const uint32_t pg_end = (it.kv_end + kPage - 1) / kPage;
    // Keys below full_end are visible to every query of the item.
    const uint32_t full_end = min(it.pos0 + 1, it.kv_end);
    constexpr uint32_t STRIDE = W * PB;

    // Fused, head_dim 64: the item's new rows come from the k/v input as
    // their pages stream.  head_dim 128 appends them first (streaming them
    // costs 37 registers there, a wave per SIMD).
    NewRows nr{};
    if constexpr (FUSED) {
        if (it.napp) {
            if constexpr (D == 64) {
                const int64_t off =
                    (int64_t)lay * a.kv_layer_stride + (int64_t)it.app_src * a.kv_row_stride + head * D + ds * 8;
                nr = NewRows{a.k + off, a.v + off, a.kv_row_stride, it.app_pos, it.napp};
            } else {
                item_append<D>(a, plan, it, lay, head, layer_off, page_stride, 64 * W);
                __syncthreads();
            }
        }
    }

    // First pages in flight before the query loads.
    PageRegs<PB, LPP> cur;
    uint32_t pg = pg_begin + wave * PB;
    if (pg < pg_end) load_pages(cur, tab, pg, pg_end, kbase, vbase, page_stride, lane, nr, kl);

    float q[NQ][8];
    {
        const float* qb = a.q + (int64_t)lay * a.q_layer_stride + (int64_t)it.row0 * a.q_row_stride + head * D + ds * 8;
#pragma unroll
        for (int r = 0; r < NQ; r++) {
            if (r < (int)it.nq) {
                const float4 x0 = reinterpret_cast<const float4*>(qb + (int64_t)r * a.q_row_stride)[0];
                const float4 x1 = reinterpret_cast<const float4*>(qb + (int64_t)r * a.q_row_stride)[1];
                q[r][0] = x0.x * a.qscale; q[r][1] = x0.y * a.qscale;
                q[r][2] = x0.z * a.qscale; q[r][3] = x0.w * a.qscale;
                q[r][4] = x1.x * a.qscale; q[r][5] = x1.y * a.qscale;
                q[r][6] = x1.z * a.qscale; q[r][7] = x1.w * a.qscale;
            } else {
#pragma unroll
                for (int e = 0; e < 8; e++) q[r][e] = 0.f;
            }
        }
    }
    float m[NQ], l[NQ], o[NQ][8];
#pragma unroll
    for (int r = 0; r < NQ; r++) {
        m[r] = kMinScore;
        l[r] = 0.f;
#pragma unroll
        for (int e = 0; e < 8; e++) o[r][e] = 0.f;
    }

    for (; pg < pg_end; pg += STRIDE) {
        // the next iteration's pages in flight while this one computes
        PageRegs<PB, LPP> nxt;
        if (pg + STRIDE < pg_end) load_pages(nxt, tab, pg + STRIDE, pg_end, kbase, vbase, page_stride, lane, nr, kl);
        float s[NQ][PB][LPP];
#pragma unroll
        for (int b = 0; b < PB; b++) {
#pragma unroll
            for (int i = 0; i < LPP; i++) {
                const half8_t kh = __builtin_bit_cast(half8_t, cur.k[b][i]);
#pragma unroll
                for (int r = 0; r < NQ; r++) {
                    float acc = 0.f;
                    if (r < (int)it.nq) {
#pragma unroll
                        for (int e = 0; e < 8; e++) acc = fmaf(q[r][e], static_cast<float>(kh[e]), acc);
                    }
                    s[r][b][i] = key_sum<LPK>(acc);
                }
            }
        }
        if ((pg + PB) * kPage > full_end) {  // a page past the first query's position: mask
#pragma unroll
            for (int b = 0; b < PB; b++) {
#pragma unroll
                for (int i = 0; i < LPP; i++) {
                    const uint32_t j = (pg + b) * kPage + i * KPL + kl;
                    if (j >= it.kv_end) cur.v[b][i] = u32x4{0, 0, 0, 0};
#pragma unroll
                    for (int r = 0; r < NQ; r++)
                        if (j > it.pos0 + r || j >= it.kv_end) s[r][b][i] = -INFINITY;
                }
            }
        }
#pragma unroll
        for (int r = 0; r < NQ; r++) {
            if (r >= (int)it.nq) continue;
            float mb = s[r][0][0];
#pragma unroll
            for (int b = 0; b < PB; b++)
#pragma unroll
                for (int i = 0; i < LPP; i++) mb = fmaxf(mb, s[r][b][i]);
            const float mn = fmaxf(m[r], mb);
            const float alpha = fast_exp2(m[r] - mn);
            m[r] = mn;
            l[r] *= alpha;
#pragma unroll
            for (int e = 0; e < 8; e++) o[r][e] *= alpha;
#pragma unroll
            for (int b = 0; b < PB; b++) {
#pragma unroll
                for (int i = 0; i < LPP; i++) {
                    const float p = fast_exp2(s[r][b][i] - mn);
                    l[r] += p;
                    const half8_t vh = __builtin_bit_cast(half8_t, cur.v[b][i]);
#pragma unroll
                    for (int e = 0; e < 8; e++) o[r][e] = fmaf(p, static_cast<float>(vh[e]), o[r][e]);
                }
            }
        }
        cur = nxt;
    }

    // Merge the KPL key-row groups of the wave (lanes ds, ds+LPK, ...).
#pragma unroll
    for (int r = 0; r < NQ; r++) {
        if (r >= (int)it.nq) continue;
#pragma unroll
        for (int off = LPK; off < 64; off <<= 1) {
            const float m2 = __shfl_xor(m[r], off);
            const float l2 = __shfl_xor(l[r], off);
            float o2[8];
#pragma unroll
            for (int e = 0; e < 8; e++) o2[e] = __shfl_xor(o[r][e], off);
            merge_state(m[r], l[r], o[r], m2, l2, o2);
        }
    }
    if (kl == 0) {
#pragma unroll
        for (int r = 0; r < NQ; r++) {
            if (r >= (int)it.nq) continue;
#pragma unroll
            for (int e = 0; e < 8; e++) red[wave][r][2 + ds * 8 + e] = o[r][e];
            if (ds == 0) {
                red[wave][r][0] = m[r];
                red[wave][r][1] = l[r];
            }
        }
    }
    __syncthreads();
    // Merge the W waves and write: the output itself when the item is its
    // group's only partition, else the partial (m, l, o) for the merge kernel.
    for (uint32_t t = threadIdx.x; t < it.nq * D; t += 64 * W) {
        const uint32_t r = t / D, d = t - r * D;
        float M = red[0][r][0];
#pragma unroll
        for (int w = 1; w < W; w++) M = fmaxf(M, red[w][r][0]);
        float L = 0.f, O = 0.f;
#pragma unroll
        for (int w = 0; w < W; w++) {
            const float wt = fast_exp2(red[w][r][0] - M);
            L += red[w][r][1] * wt;
            O += red[w][r][2 + d] * wt;
        }
        if (it.part_slot == kNoSlot) {
            a.out[(int64_t)lay * a.out_layer_stride + (int64_t)(it.row0 + r) * a.out_row_stride + head * D + d] = O / L;
        } else {
            float* p = a.partials + ((((uint64_t)it.part_slot * a.n_lay + lay) * H + head) * NQ + r) * (D + 2);
            if (d == 0) {
                p[0] = M;
                p[1] = L;
            }
            p[2 + d] = O;
        }
    }
}

// --------------------------------------------- contiguous f32 attention

// Kernels::attention (crates/core/src/kernels/mod.rs:86-98; the math of
// reference::attention, reference.rs:109-142): query i at position q_pos0 + i
// attends to f32 K/V rows 0 .. q_pos0 + i held contiguously with a row
// stride.  One workgroup of W waves per (query, head); wave w takes key
// blocks w, w + W, ... of U * 4 keys.  Lane l reads D/16 floats of key row
// l / 16 of a load (16 lanes per row, 4 rows per load), keeps its own flash
// state over the rows it sees, and the lanes' and waves' states are merged
// once at the end, as in attn_split_kernel.  Rows past the query's last key
// are never read (their loads repeat the last key and weigh 0).
template <int D, int W>
__global__ __launch_bounds__(64 * W) void attn_rows_kernel(const RowsLaunch a) {
    constexpr int F = D / 16;  // floats per lane
    constexpr int KPL = 4;     // key rows per load
    constexpr int U = 4;       // loads per wave iteration
    constexpr uint32_t KPI = KPL * U;
    __shared__ float red[W][D + 2];
    const int lane = threadIdx.x & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t i = blockIdx.x / a.n_head, h = blockIdx.x - i * a.n_head;
    const uint32_t n_kv = a.q_pos0 + i + 1;
    const int kl = lane >> 4, ds = lane & 15;
    float q[F];
    {
        const float4* qp = reinterpret_cast<const float4*>(a.q + (int64_t)i * a.q_stride + h * D + F * ds);
#pragma unroll
        for (int c = 0; c < F / 4; c++) {
            const float4 x = qp[c];
            q[4 * c] = x.x * a.qscale;
            q[4 * c + 1] = x.y * a.qscale;
            q[4 * c + 2] = x.z * a.qscale;
            q[4 * c + 3] = x.w * a.qscale;
        }
    }
    const float* kb = a.k + h * D + F * ds;
    const float* vb = a.v + h * D + F * ds;
    float m = kMinScore, l = 0.f, o[F];
#pragma unroll
    for (int e = 0; e < F; e++) o[e] = 0.f;
    for (uint32_t j0 = wave * KPI; j0 < n_kv; j0 += W * KPI) {
        float4 kr[U][F / 4], vr[U][F / 4];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const uint32_t j = min(j0 + u * KPL + kl, n_kv - 1);
            const float4* kp = reinterpret_cast<const float4*>(kb + (int64_t)j * a.k_stride);
            const float4* vp = reinterpret_cast<const float4*>(vb + (int64_t)j * a.v_stride);
#pragma unroll
            for (int c = 0; c < F / 4; c++) {
                kr[u][c] = kp[c];
                vr[u][c] = vp[c];
            }
        }
        float s[U];
        float mb = -INFINITY;
#pragma unroll
        for (int u = 0; u < U; u++) {
            float acc = 0.f;
#pragma unroll
            for (int c = 0; c < F / 4; c++) {
                acc = fmaf(q[4 * c], kr[u][c].x, acc);
                acc = fmaf(q[4 * c + 1], kr[u][c].y, acc);
                acc = fmaf(q[4 * c + 2], kr[u][c].z, acc);
                acc = fmaf(q[4 * c + 3], kr[u][c].w, acc);
            }
            s[u] = key_sum<16>(acc);
            if (j0 + u * KPL + kl >= n_kv) s[u] = -INFINITY;
            mb = fmaxf(mb, s[u]);
        }
        const float mn = fmaxf(m, mb);
        const float alpha = fast_exp2(m - mn);
        m = mn;
        l *= alpha;
#pragma unroll
        for (int e = 0; e < F; e++) o[e] *= alpha;
#pragma unroll
        for (int u = 0; u < U; u++) {
            const float p = fast_exp2(s[u] - mn);
            l += p;
#pragma unroll
            for (int c = 0; c < F / 4; c++) {
                o[4 * c] = fmaf(p, vr[u][c].x, o[4 * c]);
                o[4 * c + 1] = fmaf(p, vr[u][c].y, o[4 * c + 1]);
                o[4 * c + 2] = fmaf(p, vr[u][c].z, o[4 * c + 2]);
                o[4 * c + 3] = fmaf(p, vr[u][c].w, o[4 * c + 3]);
            }
        }
    }
    // The wave's 4 key-row groups (lanes ds, ds + 16, ds + 32, ds + 48).
#pragma unroll
    for (int off = 16; off < 64; off <<= 1) {
        const float m2 = __shfl_xor(m, off);
        const float l2 = __shfl_xor(l, off);
        float o2[F];
#pragma unroll
        for (int e = 0; e < F; e++) o2[e] = __shfl_xor(o[e], off);
        merge_state(m, l, o, m2, l2, o2);
    }
    if (kl == 0) {
#pragma unroll
        for (int e = 0; e < F; e++) red[wave][2 + F * ds + e] = o[e];
        if (ds == 0) {
            red[wave][0] = m;
            red[wave][1] = l;
        }
    }
    __syncthreads();
    for (uint32_t d = threadIdx.x; d < (uint32_t)D; d += 64 * W) {
        float M = red[0][0];
#pragma unroll
        for (int w = 1; w < W; w++) M = fmaxf(M, red[w][0]);
        float L = 0.f, O = 0.f;
#pragma unroll
        for (int w = 0; w < W; w++) {
            const float wt = fast_exp2(red[w][0] - M);
            L += red[w][1] * wt;
            O += red[w][2 + d] * wt;
        }
        a.out[(int64_t)i * a.out_stride + h * D + d] = O / L;
    }
}

// ------------------------------------------------------- Q8 attention

// Byte j of w as a signed integer, in f32.
__device__ __forceinline__ float i8f(uint32_t w, int j) { return (float)((int32_t)(w << (24 - 8 * j)) >> 24); }

// Pages per wave iteration of attn_q8_kernel: 1 measured 1% faster than 2
// and 6% faster than 4 on config 3.
constexpr int kQ8Pages = 1;

// item_append for a Q8 pool: each aligned group of D/8 threads quantises one
// (row, K|V) of the head.
template <int D>
__device__ __forceinline__ void item_append_q8(const AttnLaunch& a, const uint8_t* plan, const AttnItem& it,
                                               uint32_t lay, uint32_t head, uint64_t layer_off, uint64_t page_stride,
                                               uint32_t nthreads) {
    constexpr uint32_t CH = D / 8;
    for (uint32_t t = threadIdx.x; t < it.napp * 2 * CH; t += nthreads) {
        const uint32_t row = t / (2 * CH);
        const uint32_t rem2 = t - row * (2 * CH);
        const uint32_t is_v = rem2 >= CH;
        const uint32_t c = (rem2 - is_v * CH) * 8;
        const AppendEntry e = reinterpret_cast<const AppendEntry*>(plan + a.off_app)[it.app0 + row];
        // (append entry i reads input row i: the load need not wait for e)
        const float* src = (is_v ? a.v : a.k) + (int64_t)lay * a.kv_layer_stride +
                           (int64_t)(it.app0 + row) * a.kv_row_stride + head * D + c;
        const float4 x0 = reinterpret_cast<const float4*>(src)[0];
        const float4 x1 = reinterpret_cast<const float4*>(src)[1];
        q8_store8(q8_block(a.pool, is_v, layer_off + (uint64_t)e.page * page_stride), D, e.slot, c, x0, x1);
    }
}

// Paged decode attention over a Q8 pool (attn_decode_split_q8,
// kv8.metal:50-95, over pages): score_j = (q . k_j) * ks_j / sqrt(D) with
// k_j the int8 values, out = sum_j p_j vs_j v_j / sum_j p_j.  One workgroup
// of W waves per (item, layer, head), one query row per item; lane l reads
// 16 int8 of key row l / LPK (LPK = D/16 lanes per key) and that key's
// scale, as attn_split_kernel reads 8 halves.
template <int D, int W, int PB, bool FUSED, int INL>
__global__ __launch_bounds__(64 * W) void attn_q8_kernel(const AttnLaunch a, const PlanArg<INL> pa) {
    constexpr int LPK = D / 16;
    constexpr int KPL = 64 / LPK;
    constexpr int LPP = kPage / KPL;
    __shared__ float red[W][D + 2];

    const int lane = threadIdx.x & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t H = a.pool.n_head;
    const uint32_t lh = a.n_lay * H;
    const uint8_t* plan = plan_base(pa, a.plan);
    if constexpr (FUSED) {
        const uint32_t n_attn = a.n_items * lh;
        if (blockIdx.x >= n_attn) {
            const uint32_t base = (blockIdx.x - n_attn) * (64u * W);
            append_chunk_q8(a.pool, a.k, a.v, a.kv_row_stride, a.kv_layer_stride,
                            reinterpret_cast<const AppendEntry*>(plan + a.off_orphans), a.n_orphans, a.layer0,
                            a.n_lay, base + threadIdx.x);
            return;
        }
    }
    const AttnUnit un = attn_unit(a, plan, blockIdx.x);
    const uint32_t item_i = un.item, lay = un.lay, head = un.head;
    const AttnItem it = reinterpret_cast<const AttnItem*>(plan + a.off_items)[item_i];
    const int kl = lane / LPK;
    const int ds = lane % LPK;

    const uint64_t layer_off = (uint64_t)(a.layer0 + lay) * a.pool.layer_halves + (uint64_t)head * a.pool.head_halves;
    const uint8_t* kbase = reinterpret_cast<const uint8_t*>(a.pool.k + layer_off);
    const uint8_t* vbase = reinterpret_cast<const uint8_t*>(a.pool.v + layer_off);
    const uint64_t page_bytes = a.pool.page_halves * 2;
    const uint32_t* __restrict__ tab = reinterpret_cast<const uint32_t*>(plan + a.off_table) + it.tab;
    const uint32_t pg_begin = it.kv_begin / kPage;
    const uint32_t pg_end = (it.kv_end + kPage - 1) / kPage;
    constexpr uint32_t STRIDE = W * PB;

    // Fused, in the wide (one layer per launch) workgroups: the item's new
    // rows come from the k/v input as their pages stream, quantised as the
    // append quantises them (the row's amax reduced over its LPK lanes; a max
    // does not depend on the order).  Otherwise they are appended first
    // (streaming them costs ~24 registers, 7 -> 5 waves per SIMD, which all
    // layers in one launch lose: 5202 against 4638 GB/s; one layer per
    // launch gains, 2641 -> 2823).
    constexpr bool STREAM = D == 64 && W == (int)kWideWavesQ8 && (int)kWideWavesQ8 != kWaves;
    NewRows nr{};
    if constexpr (FUSED) {
        if (it.napp) {
            if constexpr (STREAM) {
                const int64_t off =
                    (int64_t)lay * a.kv_layer_stride + (int64_t)it.app_src * a.kv_row_stride + head * D + ds * 16;
                nr = NewRows{a.k + off, a.v + off, a.kv_row_stride, it.app_pos, it.napp};
            } else {
                item_append_q8<D>(a, plan, it, lay, head, layer_off, a.pool.page_halves, 64 * W);
                __syncthreads();
            }
        }
    }

    struct Regs {
        u32x4 k[PB][LPP], v[PB][LPP];
        float ks[PB][LPP], vs[PB][LPP];
    };
    // A new row's 16 values of this lane (all lanes take part: the amax
    // crosses lanes), its int8 bytes and scale; stored to the pool when new.
    auto quant16 = [&](const float* src, bool isnew, uint8_t* blk, uint32_t key, u32x4& w, float& scale) {
        float4 x[4];
#pragma unroll
        for (int m = 0; m < 4; m++)
            x[m] = isnew ? reinterpret_cast<const float4*>(src)[m] : float4{0.f, 0.f, 0.f, 0.f};
        float am = 0.f;
#pragma unroll
        for (int m = 0; m < 4; m++)
            am = fmaxf(am, fmaxf(fmaxf(fabsf(x[m].x), fabsf(x[m].y)), fmaxf(fabsf(x[m].z), fabsf(x[m].w))));
#pragma unroll
        for (int off = 1; off < LPK; off <<= 1) am = fmaxf(am, __shfl_xor(am, off));
        scale = am / 127.f;
        const float inv = scale > 0.f ? 1.f / scale : 0.f;
#pragma unroll
        for (int m = 0; m < 4; m++)
            w[m] = q8_byte(x[m].x, inv) | q8_byte(x[m].y, inv) << 8 | q8_byte(x[m].z, inv) << 16 |
                   q8_byte(x[m].w, inv) << 24;
        if (isnew) {
            *reinterpret_cast<u32x4*>(blk + key * D + ds * 16) = w;
            if (ds == 0) reinterpret_cast<float*>(blk + kPage * D)[key] = scale;
        }
    };
    auto load = [&](uint32_t pg, Regs& r) {
#pragma unroll
        for (int b = 0; b < PB; b++) {
            if (pg + b < pg_end) {
                const uint64_t phys = tab[pg + b];
                const uint8_t* kb = kbase + phys * page_bytes;
                const uint8_t* vb = vbase + phys * page_bytes;
                const uint32_t p0 = (pg + b) * kPage;
                if (nr.n && p0 < nr.pos + nr.n && p0 + kPage > nr.pos) {  // wave-uniform: new rows in the page
#pragma unroll
                    for (int i = 0; i < LPP; i++) {
                        const uint32_t key = i * KPL + kl;
                        const uint32_t d = p0 + key - nr.pos;  // unsigned: >= n unless new
                        const bool isnew = d < nr.n;
                        const int64_t ro = (int64_t)(isnew ? d : 0u) * nr.row_stride;
                        u32x4 wk, wv;
                        float sk, sv;
                        quant16(nr.k + ro, isnew, const_cast<uint8_t*>(kb), key, wk, sk);
                        quant16(nr.v + ro, isnew, const_cast<uint8_t*>(vb), key, wv, sv);
                        if (isnew) {
                            r.k[b][i] = wk;
                            r.v[b][i] = wv;
                            r.ks[b][i] = sk;
                            r.vs[b][i] = sv;
                        } else {
                            r.k[b][i] = load16(reinterpret_cast<const u32x4*>(kb) + lane + i * 64);
                            r.v[b][i] = load16(reinterpret_cast<const u32x4*>(vb) + lane + i * 64);
                            r.ks[b][i] = reinterpret_cast<const float*>(kb + kPage * D)[key];
                            r.vs[b][i] = reinterpret_cast<const float*>(vb + kPage * D)[key];
                        }
                    }
                    continue;
                }
#pragma unroll
                for (int i = 0; i < LPP; i++) {
                    r.k[b][i] = load16(reinterpret_cast<const u32x4*>(kb) + lane + i * 64);
                    r.v[b][i] = load16(reinterpret_cast<const u32x4*>(vb) + lane + i * 64);
                    r.ks[b][i] = reinterpret_cast<const float*>(kb + kPage * D)[i * KPL + kl];
                    r.vs[b][i] = reinterpret_cast<const float*>(vb + kPage * D)[i * KPL + kl];
                }
            } else {
#pragma unroll
                for (int i = 0; i < LPP; i++) {
                    r.k[b][i] = r.v[b][i] = u32x4{0, 0, 0, 0};
                    r.ks[b][i] = r.vs[b][i] = 0.f;
                }
            }
        }
    };
    Regs cur;
    uint32_t pg = pg_begin + wave * PB;
    if (pg < pg_end) load(pg, cur);

    float q[16];
    {
        const float* qb = a.q + (int64_t)lay * a.q_layer_stride + (int64_t)it.row0 * a.q_row_stride + head * D + ds * 16;
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const float4 x = reinterpret_cast<const float4*>(qb)[c];
            q[4 * c] = x.x * a.qscale;
            q[4 * c + 1] = x.y * a.qscale;
            q[4 * c + 2] = x.z * a.qscale;
            q[4 * c + 3] = x.w * a.qscale;
        }
    }
    float m = kMinScore, l = 0.f, o[16];
#pragma unroll
    for (int e = 0; e < 16; e++) o[e] = 0.f;

    for (; pg < pg_end; pg += STRIDE) {
        Regs nxt;
        if (pg + STRIDE < pg_end) load(pg + STRIDE, nxt);
        float s[PB][LPP];
#pragma unroll
        for (int b = 0; b < PB; b++) {
#pragma unroll
            for (int i = 0; i < LPP; i++) {
                float acc = 0.f;
#pragma unroll
                for (int w = 0; w < 4; w++)
#pragma unroll
                    for (int j = 0; j < 4; j++) acc = fmaf(q[4 * w + j], i8f(cur.k[b][i][w], j), acc);
                s[b][i] = key_sum<LPK>(acc) * cur.ks[b][i];
                const uint32_t key = (pg + b) * kPage + i * KPL + kl;
                if (key > it.pos0 || key >= it.kv_end) {
                    s[b][i] = -INFINITY;
                    cur.vs[b][i] = 0.f;
                }
            }
        }
        float mb = s[0][0];
#pragma unroll
        for (int b = 0; b < PB; b++)
#pragma unroll
            for (int i = 0; i < LPP; i++) mb = fmaxf(mb, s[b][i]);
        const float mn = fmaxf(m, mb);
        const float alpha = fast_exp2(m - mn);
        m = mn;
        l *= alpha;
#pragma unroll
        for (int e = 0; e < 16; e++) o[e] *= alpha;
#pragma unroll
        for (int b = 0; b < PB; b++) {
#pragma unroll
            for (int i = 0; i < LPP; i++) {
                const float p = fast_exp2(s[b][i] - mn);
                l += p;
                const float pv = p * cur.vs[b][i];
#pragma unroll
                for (int w = 0; w < 4; w++)
#pragma unroll
                    for (int j = 0; j < 4; j++) o[4 * w + j] = fmaf(pv, i8f(cur.v[b][i][w], j), o[4 * w + j]);
            }
        }
        cur = nxt;
    }

    // Merge the KPL key-row groups of the wave (lanes ds, ds+LPK, ...).
#pragma unroll
    for (int off = LPK; off < 64; off <<= 1) {
        const float m2 = __shfl_xor(m, off);
        const float l2 = __shfl_xor(l, off);
        float o2[16];
#pragma unroll
        for (int e = 0; e < 16; e++) o2[e] = __shfl_xor(o[e], off);
        merge_state(m, l, o, m2, l2, o2);
    }
    if (kl == 0) {
#pragma unroll
        for (int e = 0; e < 16; e++) red[wave][2 + ds * 16 + e] = o[e];
        if (ds == 0) {
            red[wave][0] = m;
            red[wave][1] = l;
        }
    }
    __syncthreads();
    for (uint32_t d = threadIdx.x; d < D; d += 64 * W) {
        float M = red[0][0];
#pragma unroll
        for (int w = 1; w < W; w++) M = fmaxf(M, red[w][0]);
        float L = 0.f, O = 0.f;
#pragma unroll
        for (int w = 0; w < W; w++) {
            const float wt = fast_exp2(red[w][0] - M);
            L += red[w][1] * wt;
            O += red[w][2 + d] * wt;
        }
        if (it.part_slot == kNoSlot) {
            a.out[(int64_t)lay * a.out_layer_stride + (int64_t)it.row0 * a.out_row_stride + head * D + d] = O / L;
        } else {
            float* p = a.partials + (((uint64_t)it.part_slot * a.n_lay + lay) * H + head) * (D + 2);
            if (d == 0) {
                p[0] = M;
                p[1] = L;
            }
            p[2 + d] = O;
        }
    }
}

// ------------------------------------------------------- QKV projection

// y = x W^T + b on the matrix cores in f32 (v_mfma_f32_16x16x4f32), the
// reference's QKV matvec with its epilogue
// (matvec_batch<..., BEPI_QKV>, batch.metal:94-165): q to `out`, k/v as f16
// straight into the rows' page slots, so f32 K/V never travel through HBM.
//
// In a 16-wide slice of d_in, lane l holds 4 consecutive x values of row
// l%16 and 4 of W's feature l%16 at offset 4*(l/16); product c of the slice
// uses component c of both, so lane group g supplies k = 4g + c to A and B
// alike.
//
// Summation order, the same for every row count and both kernels below (so
// a row's bits never depend on the batch it is projected in): slice s of
// d_in belongs to part s % 8; part p's accumulator takes the 4 products of
// each of its slices in increasing s (components x, y, z, w in turn), and
// y = (((P0 + P1) + (P2 + P3)) + ((P4 + P5) + (P6 + P7))) + bias.
constexpr int kQkvParts = 8;
// Rows up to which qkv_small_kernel runs (kernel time per layer, GPT-2
// 768 -> 2304: 1 row 4.66 against 7.11 us, 16 rows 6.15 against 7.61 us; from
// 24 rows its 64-byte row pieces per load lose to the LDS-staged kernel's
// whole-row reads: 24 rows 8.98 against 7.65 us, 64 rows 11.9 against 9.5).
constexpr uint32_t kQkvSmallRows = 16;
// 16-row blocks per workgroup of the small-batch kernel (2 and 4 measured
// 154 and 141 us per 12 layers of 64 rows).
constexpr int kQkvSmallRb = 1;

// Large row counts: the tile is 32 rows x 16*FB features.  x and W arrive
// through LDS in chunks of kQkvChunk values of d_in (8 slices, one per
// part), each row segment loaded contiguously (a wave-wide load covers 1 KB
// of one or two rows); the next chunk is in registers while the current one
// is multiplied.  Wave w owns row block w & 1 and parts 4 (w >> 1) ..
// 4 (w >> 1) + 3, i.e. half (w >> 1) of every chunk.
constexpr int kQkvChunk = 128;
constexpr int kQkvPad = kQkvChunk + 4;  // LDS row stride (floats): conflict-free 16-byte reads
static_assert(kQkvChunk == 16 * kQkvParts, "one slice per part per chunk");

// W[f][k .. k+3] (k a multiple of 4) as f32, dequantised as the reference's
// weight loaders do (batch.metal:45-90: BF32, BF16, BQ8, BQ4 over the layouts
// of crates/metal/src/weights.rs:12-86): f16 widened; Q8_0 q * d and Q4_0
// (q - 8) * d with d the block's f16 scale -- every value exact in f32, so a
// projection with quantised weights has the bits of the same projection
// with the dequantised matrix in f32.  Blocks of 32 follow the row-major
// element index f * d_in + k (d_in a multiple of 32); Q4_0 byte i of a
// block holds element i (low nibble) and element i + 16 (high nibble).
typedef float qkv_f4 __attribute__((ext_vector_type(4)));
template <int WF>
__device__ __forceinline__ qkv_f4 qkv_w4(const QkvLaunch& a, uint32_t f, uint32_t k) {
    const uint64_t i = (uint64_t)f * a.d_in + k;
    if constexpr (WF == kWF32) {
        return *reinterpret_cast<const qkv_f4*>(static_cast<const float*>(a.w) + i);
    } else if constexpr (WF == kWF16) {
        typedef _Float16 h4 __attribute__((ext_vector_type(4)));
        const h4 h = *reinterpret_cast<const h4*>(static_cast<const uint16_t*>(a.w) + i);
        return qkv_f4{(float)h[0], (float)h[1], (float)h[2], (float)h[3]};
    } else {
        const uint8_t* wb = static_cast<const uint8_t*>(a.w);
        const uint64_t n = (uint64_t)a.n_feat * a.d_in;
        const uint16_t* scales = reinterpret_cast<const uint16_t*>(wb + (WF == kWQ8 ? n : n / 2));
        const float d = (float)__builtin_bit_cast(_Float16, scales[i / 32]);
        if constexpr (WF == kWQ8) {
            const uint32_t q = *reinterpret_cast<const uint32_t*>(wb + i);
            return qkv_f4{(float)(int8_t)(q & 0xffu) * d, (float)(int8_t)((q >> 8) & 0xffu) * d,
                          (float)(int8_t)((q >> 16) & 0xffu) * d, (float)(int8_t)(q >> 24) * d};
        } else {
            const uint32_t j = (uint32_t)(i % 32);
            const uint32_t q = *reinterpret_cast<const uint32_t*>(wb + (i / 32) * 16 + (j % 16));
            const uint32_t sh = j < 16 ? 0u : 4u;
            return qkv_f4{(float)((int)((q >> sh) & 15u) - 8) * d, (float)((int)((q >> (8 + sh)) & 15u) - 8) * d,
                          (float)((int)((q >> (16 + sh)) & 15u) - 8) * d,
                          (float)((int)((q >> (24 + sh)) & 15u) - 8) * d};
        }
    }
}

// Output y of (row, feature f): q columns (or every column when not fused)
// to `out`, k/v as f16 (the append's rounding) into the row's page slot.
__device__ __forceinline__ void qkv_store(const QkvLaunch& a, const AppendEntry* entries, uint32_t row, uint32_t f,
                                          float y) {
    const uint32_t C = a.n_feat / 3, D = a.pool.head_dim;
    if (!a.fused || f < C) {
        a.out[(int64_t)row * a.out_row_stride + f] = y;
    } else {
        const AppendEntry en = entries[row];
        const uint32_t is_v = f >= 2 * C;
        const uint32_t c = f - C - is_v * C, head = c / D, d = c - head * D;
        uint16_t* dst = (is_v ? a.pool.v : a.pool.k) + (uint64_t)a.layer * a.pool.layer_halves +
                        (uint64_t)en.page * a.pool.page_halves + (uint64_t)head * a.pool.head_halves + en.slot * D + d;
        *dst = (uint16_t)f16_bits(y);
    }
}

// qkv_store with the row's append entry already in hand.
__device__ __forceinline__ void qkv_store_en(const QkvLaunch& a, const AppendEntry& en, uint32_t row, uint32_t f,
                                             float y) {
    const uint32_t C = a.n_feat / 3, D = a.pool.head_dim;
    if (!a.fused || f < C) {
        a.out[(int64_t)row * a.out_row_stride + f] = y;
    } else {
        const uint32_t is_v = f >= 2 * C;
        const uint32_t c = f - C - is_v * C, head = c / D, d = c - head * D;
        uint16_t* dst = (is_v ? a.pool.v : a.pool.k) + (uint64_t)a.layer * a.pool.layer_halves +
                        (uint64_t)en.page * a.pool.page_halves + (uint64_t)head * a.pool.head_halves + en.slot * D + d;
        *dst = (uint16_t)f16_bits(y);
    }
}

template <int FB, int INL, int WF>
__global__ __launch_bounds__(256) void qkv_kernel(const QkvLaunch a, const PlanArg<INL> pa) {
    typedef float f4 __attribute__((ext_vector_type(4)));
    constexpr int TM = kQkvTileRows, TF = 16 * FB, KC = kQkvChunk, KP = kQkvPad;
    constexpr int XV = TM * KC / 4 / 256, WV = TF * KC / 4 / 256;  // float4 per thread per chunk
    __shared__ __attribute__((aligned(16))) float xs[TM][KP];
    __shared__ __attribute__((aligned(16))) float ws[TF][KP];
    __shared__ float red[2][FB][4][64];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int rb = wave & 1, kh = wave >> 1;
    const uint32_t m0 = blockIdx.x * TM, n0 = blockIdx.y * TF;
    const int i = lane & 15, g = lane >> 4;

    // Staging: float4 u = threadIdx.x + 256 * j of a chunk is row u / (KC/4),
    // column 4 * (u % (KC/4)).  Rows past n_rows repeat the last row; values
    // past d_in (the last, partial chunk) are zeros.
    float4 xr[XV], wr[WV];
    auto fetch = [&](uint32_t k0) {
#pragma unroll
        for (int j = 0; j < XV; j++) {
            const uint32_t u = threadIdx.x + 256 * j, row = u / (KC / 4), col = 4 * (u % (KC / 4));
            const uint32_t r = min(m0 + row, a.n_rows - 1);
            xr[j] = k0 + col < a.d_in ? *reinterpret_cast<const float4*>(a.x + (int64_t)r * a.x_row_stride + k0 + col)
                                      : float4{0.f, 0.f, 0.f, 0.f};
        }
#pragma unroll
        for (int j = 0; j < WV; j++) {
            const uint32_t u = threadIdx.x + 256 * j, row = u / (KC / 4), col = 4 * (u % (KC / 4));
            if (k0 + col < a.d_in) {
                const qkv_f4 v = qkv_w4<WF>(a, n0 + row, k0 + col);
                wr[j] = float4{v[0], v[1], v[2], v[3]};
            } else {
                wr[j] = float4{0.f, 0.f, 0.f, 0.f};
            }
        }
    };
    f4 acc[FB][4];  // the wave's 4 parts
#pragma unroll
    for (int fb = 0; fb < FB; fb++)
#pragma unroll
        for (int pp = 0; pp < 4; pp++) acc[fb][pp] = f4{0.f, 0.f, 0.f, 0.f};
    const uint32_t n_slices = a.d_in / 16;
    fetch(0);
    for (uint32_t k0 = 0; k0 < a.d_in; k0 += KC) {
        __syncthreads();  // the previous chunk's products are done with LDS
#pragma unroll
        for (int j = 0; j < XV; j++) {
            const uint32_t u = threadIdx.x + 256 * j;
            *reinterpret_cast<float4*>(&xs[u / (KC / 4)][4 * (u % (KC / 4))]) = xr[j];
        }
#pragma unroll
        for (int j = 0; j < WV; j++) {
            const uint32_t u = threadIdx.x + 256 * j;
            *reinterpret_cast<float4*>(&ws[u / (KC / 4)][4 * (u % (KC / 4))]) = wr[j];
        }
        __syncthreads();
        if (k0 + KC < a.d_in) fetch(k0 + KC);
        // This wave's half of the chunk: slices of 16, slice sl of the half
        // is part 4 kh + sl; lane (i, g) holds k = 4g .. 4g+3 of the slice
        // for row 16rb + i and for feature 16fb + i.  Slices past d_in (the
        // last chunk's zeros) are skipped, as the small-batch kernel does.
#pragma unroll
        for (int sl = 0; sl < KC / 32; sl++) {
            const uint32_t slice = k0 / 16 + kh * (KC / 32) + sl;
            if (slice >= n_slices) break;
            const int kk = (kh * (KC / 32) + sl) * 16 + 4 * g;
            const float4 xv = *reinterpret_cast<const float4*>(&xs[16 * rb + i][kk]);
#pragma unroll
            for (int fb = 0; fb < FB; fb++) {
                const float4 wv = *reinterpret_cast<const float4*>(&ws[16 * fb + i][kk]);
                acc[fb][sl] = __builtin_amdgcn_mfma_f32_16x16x4f32(xv.x, wv.x, acc[fb][sl], 0, 0, 0);
                acc[fb][sl] = __builtin_amdgcn_mfma_f32_16x16x4f32(xv.y, wv.y, acc[fb][sl], 0, 0, 0);
                acc[fb][sl] = __builtin_amdgcn_mfma_f32_16x16x4f32(xv.z, wv.z, acc[fb][sl], 0, 0, 0);
                acc[fb][sl] = __builtin_amdgcn_mfma_f32_16x16x4f32(xv.w, wv.w, acc[fb][sl], 0, 0, 0);
            }
        }
    }
    // Each wave's parts summed as (Pa + Pb) + (Pc + Pd); half 1's sum goes
    // to LDS for half 0's waves.
    f4 half[FB];
#pragma unroll
    for (int fb = 0; fb < FB; fb++) half[fb] = (acc[fb][0] + acc[fb][1]) + (acc[fb][2] + acc[fb][3]);
    if (kh == 1) {
#pragma unroll
        for (int fb = 0; fb < FB; fb++)
#pragma unroll
            for (int e = 0; e < 4; e++) red[rb][fb][e][lane] = half[fb][e];
    }
    __syncthreads();
    if (kh == 1) return;
    // Output (row 16rb + 4g + e, feature 16fb + i) is element e of lane
    // i + 16g's block fb (the matrix-core output layout).
    const AppendEntry* entries = reinterpret_cast<const AppendEntry*>(plan_base(pa, a.plan) + a.off_entries);
#pragma unroll
    for (int fb = 0; fb < FB; fb++) {
        const uint32_t f = n0 + 16 * fb + i;
        const float b = a.bias ? a.bias[f] : 0.f;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const uint32_t row = m0 + 16 * rb + 4 * g + e;
            if (row >= a.n_rows) break;
            qkv_store(a, entries, row, f, (half[fb][e] + red[rb][fb][e][lane]) + b);
        }
    }
}

// Small row counts (single-sequence and small-batch decode): a workgroup of
// 8 waves owns a 16*RB-row x 16-feature tile, wave p computes part p over
// all of d_in with its operands loaded straight from memory into the
// matrix-core layout (up to kQkvBatch slices of x and W in flight per wave,
// so d_in 768 is one round of loads instead of qkv_kernel's six chunks),
// and the 8 parts meet in LDS.  The same products in the same order as
// qkv_kernel, so the bits are the same at every row count.
constexpr int kQkvBatch = 6;

template <int RB, int INL, int WF>
__global__ __launch_bounds__(64 * kQkvParts) void qkv_small_kernel(const QkvLaunch a, const PlanArg<INL> pa) {
    typedef float f4 __attribute__((ext_vector_type(4)));
    __shared__ f4 red[kQkvParts][RB][64];
    const int lane = threadIdx.x & 63;
    const uint32_t p = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int i = lane & 15, g = lane >> 4;
    const uint32_t m0 = blockIdx.x * 16 * RB, n0 = blockIdx.y * 16;
    const uint32_t n_slices = a.d_in / 16;
    const float* xr[RB];
#pragma unroll
    for (int rb = 0; rb < RB; rb++)  // rows past n_rows repeat the last row (their results are dropped)
        xr[rb] = a.x + (int64_t)min(m0 + 16 * rb + i, a.n_rows - 1) * a.x_row_stride + 4 * g;

    // What wave p < RB stores at the end (rows m0 + 16p + 4g .. +3, feature
    // n0 + i): the rows' pages and slots and the bias, loaded with the
    // operands instead of after the sum.
    const AppendEntry* entries = reinterpret_cast<const AppendEntry*>(plan_base(pa, a.plan) + a.off_entries);
    AppendEntry en[4] = {};
    float bias = 0.f;
    if (p < (uint32_t)RB) {
        if (a.fused && n0 >= a.n_feat / 3) {
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const AppendEntry& r = entries[min(m0 + 16 * p + 4 * g + e, a.n_rows - 1)];
                en[e].page = r.page;
                en[e].slot = r.slot;
            }
        }
        if (a.bias) bias = a.bias[n0 + i];
    }

    f4 acc[RB];
#pragma unroll
    for (int rb = 0; rb < RB; rb++) acc[rb] = f4{0.f, 0.f, 0.f, 0.f};
    for (uint32_t s0 = p; s0 < n_slices; s0 += kQkvParts * kQkvBatch) {
        float4 xv[kQkvBatch][RB], wv[kQkvBatch];
#pragma unroll
        for (int j = 0; j < kQkvBatch; j++) {
            const uint32_t sl = s0 + kQkvParts * j;
            if (sl < n_slices) {
#pragma unroll
                for (int rb = 0; rb < RB; rb++) xv[j][rb] = *reinterpret_cast<const float4*>(xr[rb] + 16 * sl);
                const qkv_f4 w = qkv_w4<WF>(a, n0 + i, 16 * sl + 4 * g);
                wv[j] = float4{w[0], w[1], w[2], w[3]};
            }
        }
#pragma unroll
        for (int j = 0; j < kQkvBatch; j++) {
            if (s0 + kQkvParts * j >= n_slices) break;
#pragma unroll
            for (int rb = 0; rb < RB; rb++) {
                acc[rb] = __builtin_amdgcn_mfma_f32_16x16x4f32(xv[j][rb].x, wv[j].x, acc[rb], 0, 0, 0);
                acc[rb] = __builtin_amdgcn_mfma_f32_16x16x4f32(xv[j][rb].y, wv[j].y, acc[rb], 0, 0, 0);
                acc[rb] = __builtin_amdgcn_mfma_f32_16x16x4f32(xv[j][rb].z, wv[j].z, acc[rb], 0, 0, 0);
                acc[rb] = __builtin_amdgcn_mfma_f32_16x16x4f32(xv[j][rb].w, wv[j].w, acc[rb], 0, 0, 0);
            }
        }
    }
#pragma unroll
    for (int rb = 0; rb < RB; rb++) red[p][rb][lane] = acc[rb];
    __syncthreads();
    if (p >= (uint32_t)RB) return;
    // Wave rb finishes row block rb: the same tree as qkv_kernel.
    const int rb = (int)p;
    const f4 y = ((red[0][rb][lane] + red[1][rb][lane]) + (red[2][rb][lane] + red[3][rb][lane])) +
                 ((red[4][rb][lane] + red[5][rb][lane]) + (red[6][rb][lane] + red[7][rb][lane]));
    const uint32_t f = n0 + i;
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const uint32_t row = m0 + 16 * rb + 4 * g + e;
        if (row >= a.n_rows) break;
        qkv_store_en(a, en[e], row, f, y[e] + bias);
    }
}

// ------------------------------------------------ attention, several queries

typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef float float4_t __attribute__((ext_vector_type(4)));

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

// Four signed int8 values (bytes 0..3 of w) as f16, exactly and bit for bit
// as static_cast<_Float16>: the f16 bit pattern 0x6400 | (b ^ 0x80) is 1024 +
// (b + 128), and subtracting 1152 leaves b (operands and result exactly
// representable, so the subtraction does not round).  Two values per byte
// permute (a byte to the low byte of each 16-bit half, zeros above), XOR and
// packed f16 subtract, against a bit extract and two conversions per value.
__device__ __forceinline__ half4_t i8x4_f16(uint32_t w) {
    const uint32_t lo = __builtin_amdgcn_perm(w, w, 0x0c010c00u) ^ 0x64806480u;  // bytes 0, 1
    const uint32_t hi = __builtin_amdgcn_perm(w, w, 0x0c030c02u) ^ 0x64806480u;  // bytes 2, 3
    const half2_t k1152 = {static_cast<_Float16>(1152.f), static_cast<_Float16>(1152.f)};
    const half2_t a = __builtin_bit_cast(half2_t, lo) - k1152;
    const half2_t b = __builtin_bit_cast(half2_t, hi) - k1152;
    return half4_t{a[0], a[1], b[0], b[1]};
}

// f32 -> f16 hi plus the residual scaled by 2^11 (kept in the normal range
// of f16, where the residual itself would often be subnormal): x ~= hi +
// lo * 2^-11 to ~2^-22 relative.  Products of hi and of lo are accumulated
// separately on the matrix cores and combined in f32.  gfx950's f16 matrix
// products take subnormal operands exactly (both operands, 16x16x16 and
// 16x16x32, down to 2^-24), so a subnormal hi needs no special case.
constexpr float kLoScale = 2048.f, kLoUnscale = 1.f / 2048.f;
__device__ __forceinline__ void split_f16(float x, _Float16& hi, _Float16& lo) {
    // x as one f32 register: otherwise the compiler may fold the caller's
    // product into the conversions (a mixed-precision FMA rounding the exact
    // product to f16 once) for one use of hi and not the other, and the two
    // disagree by an f16 ulp in double-rounding cases (q off by 2^-10).
    asm("" : "+v"(x));
    hi = static_cast<_Float16>(x);
    lo = static_cast<_Float16>((x - static_cast<float>(hi)) * kLoScale);
}
// The same split for two softmax weights already scaled up (x in [0,
// 2^15]), packed: hi = f16(x), lo = f16(x - hi) unscaled, ~2^-22 relative
// where lo is normal and within 2^-25 absolute where it is subnormal.  One
// packed convert and one mixed-precision FMA per weight (x * 1 - hi, hi
// read as the f16 half of the packed register) instead of convert, convert
// back, subtract and convert; the same bits (checked on gfx950 against the
// plain formula over 2^21 pairs from 2^-40 to 2^16, zeros included).
__device__ __forceinline__ void split_w16x2(float x0, float x1, uint32_t& hi, uint32_t& lo) {
    const half2_t h = {static_cast<_Float16>(x0), static_cast<_Float16>(x1)};
    hi = __builtin_bit_cast(uint32_t, h);
    asm("v_fma_mixlo_f16 %0, %1, 1.0, -%2 op_sel_hi:[0,0,1]" : "=v"(lo) : "v"(x0), "v"(hi));
    asm("v_fma_mixhi_f16 %0, %1, 1.0, -%2 op_sel:[0,0,1] op_sel_hi:[0,0,1]" : "+v"(lo) : "v"(x1), "v"(hi));
}
// Max and sum over lanes l, l ^ 16, l ^ 32, l ^ 48 (the four lanes holding
// one query column of an MFMA 16x16 output): v_permlane16_swap and
// v_permlane32_swap of a value with itself leave the two halves of each
// lane pair in the two results, so combining them is the pair's max or sum
// in both lanes.  No LDS round trip; the same bits as __shfl_xor.
__device__ __forceinline__ float rows4_max(float v) {
    u32x2_t s = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = fmaxf(__uint_as_float(s[0]), __uint_as_float(s[1]));
    s = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(s[0]), __uint_as_float(s[1]));
}
__device__ __forceinline__ float rows4_sum(float v) {
    u32x2_t s = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(s[0]) + __uint_as_float(s[1]);
    s = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(s[0]) + __uint_as_float(s[1]);
}
// Position, in 16-byte chunks, of chunk q of row `key` in an LDS tile of
// CH-chunk rows: row major, the chunk index XORed with a permutation of the
// row's 256-byte window index, so that the 16 lanes reading one chunk of 16
// consecutive rows (the K operand) and the 32 lanes reading 4 dims of 8 rows
// for the transposed V operand each hit distinct banks.
template <int CH>
__device__ __forceinline__ uint32_t tile_chunk(uint32_t key, uint32_t q) {
    const uint32_t i = (key * CH / 16) % CH;
    const uint32_t sw = ((i & (CH / 2 - 1)) << 1) | (i / (CH / 2));
    return key * CH + (q ^ sw);
}
typedef __fp16 v4fp16_t __attribute__((__vector_size__(4 * sizeof(__fp16))));
#define NI_LDS(p) ((__attribute__((address_space(3))) void*)(p))
// p in [0, 1] enters PV scaled by 2^14 (through the exponent reference:
// exp2(s - (m - 14))), so that p down to ~4e-9 is a normal f16.
constexpr float kPUnscale = 1.f / 16384.f, kLog2PScale = 14.f;

// Groups of 2..16 queries of one sequence (speculative verify, prefill
// chunks) on matrix cores: one wave per page walks S^T = K Q^T (16 keys x 16
// query slots, v_mfma_f32_16x16x32_f16, q split into f16 hi + lo), the
// online softmax on S^T's columns, and O^T += V^T P^T (v_mfma_f32_16x16x16_f16,
// p split hi + lo), V rows through a per-wave LDS tile read back transposed
// (ds_read_b64_tr_b16), and on f16 pools K rows through another, loaded
// coalesced and read back as the A operand.  Lane l owns
// query column l % 16 of S^T and O^T, rows 4*(l/16) .. +3 (MFMA output
// layout), so the softmax state of a query lives in lanes q, q+16, q+32, q+48.
// Waves take the item's pages round-robin and merge through LDS at the end,
// as in attn_split_kernel.
// Waves per SIMD the register allocation must allow at head_dim 64: 4 (<= 128
// registers, no spills) measured 3.9% faster on config 5 than the
// unconstrained 3.  (head_dim 128 needs ~250 registers: 2 waves.)
constexpr int kMfmaMinWaves = 4;
// Q8: the pool holds int8 values with a scale per (position, head); K
// values enter the products as f16 (int8 converts exactly), the key scale
// multiplies the scores and the value scale multiplies p before its split.
template <int D, int W, int PB, bool FUSED, int INL, bool Q8>
__global__ __launch_bounds__(64 * W, D == 64 ? kMfmaMinWaves : 1) void attn_mfma_kernel(const AttnLaunch a,
                                                                                            const PlanArg<INL> pa) {
    constexpr int QC = D / 32;      // 32-dim chunks of the QK product
    constexpr int VC = D / 16;      // 16-dim chunks of the PV product
    constexpr int VE = Q8 ? 16 : 8; // V values per 16-byte lane load
    constexpr int LPK = D / VE;     // lanes per key row in a coalesced V load
    constexpr int KPL = 64 / LPK;   // key rows per V load
    constexpr int LPP = kPage / KPL;
    constexpr int CH = D / 8;       // 16-byte chunks per V row
    constexpr int NQ = 16;
    // Per-wave V tile, row major with tile_chunk's chunk swizzle: rows go in
    // with 16-byte writes, V^T comes out through transposing reads.
    // f16: K rows load coalesced (as V) and reach the A operand through a
    // per-wave tile of the same layout (config 5 5684 -> 5852 GB/s against
    // each lane loading its operand chunk directly; Q8 keeps its direct
    // 8-byte loads: an int8 tile measured 12% slower).  The waves' merge
    // buffer `red`, used after the loop, shares the tiles' LDS: 16.9 KB per
    // 4-wave workgroup instead of 33, and with one PV accumulator (92 VGPRs)
    // 5 waves per SIMD (config 5 6053-6057 -> 6069-6077 GB/s, on the Q8
    // cache 5361-5372 -> 5432-5478).
    constexpr bool KT = !Q8;
    constexpr size_t kTileBytes = (size_t)W * PB * kPage * D * 2;
    constexpr size_t kRedBytes = (size_t)W * NQ * (D + 2) * 4;
    constexpr size_t kLds = (KT ? 2 : 1) * kTileBytes > kRedBytes ? (KT ? 2 : 1) * kTileBytes : kRedBytes;
    __shared__ __attribute__((aligned(16))) uint8_t lds[kLds];
    auto& vt = *reinterpret_cast<_Float16(*)[W][PB * kPage * D]>(lds);
    auto& kt = *reinterpret_cast<_Float16(*)[KT ? W : 1][KT ? PB * kPage * D : 8]>(lds + (KT ? kTileBytes : 0));
    auto& red = *reinterpret_cast<float(*)[W][NQ][D + 2]>(lds);

    const int lane = threadIdx.x & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t H = a.pool.n_head;
    const uint32_t lh = a.n_lay * H;
    const uint8_t* plan = plan_base(pa, a.plan);
    if constexpr (FUSED) {
        const uint32_t n_attn = a.n_items * lh;
        if (blockIdx.x >= n_attn) {
            const uint32_t base = (blockIdx.x - n_attn) * (64u * W);
            const AppendEntry* orphans = reinterpret_cast<const AppendEntry*>(plan + a.off_orphans);
            if constexpr (Q8)
                append_chunk_q8(a.pool, a.k, a.v, a.kv_row_stride, a.kv_layer_stride, orphans, a.n_orphans, a.layer0,
                                a.n_lay, base + threadIdx.x);
            else
                append_chunk(a.pool, a.k, a.v, a.kv_row_stride, a.kv_layer_stride, orphans, a.n_orphans, a.layer0,
                             a.n_lay, base + threadIdx.x);
            return;
        }
    }
    const AttnUnit un = attn_unit(a, plan, blockIdx.x);
    const uint32_t item_i = un.item, lay = un.lay, head = un.head;
    const AttnItem it = reinterpret_cast<const AttnItem*>(plan + a.off_items)[item_i];
    const int col = lane & 15;  // query slot of S^T / O^T columns
    const int rg = lane >> 4;   // row group: keys (or dims) 4*rg .. 4*rg+3

    const uint64_t layer_off = (uint64_t)(a.layer0 + lay) * a.pool.layer_halves + (uint64_t)head * a.pool.head_halves;
    const uint16_t* kbase = a.pool.k + layer_off;
    const uint16_t* vbase = a.pool.v + layer_off;
    const uint64_t page_stride = a.pool.page_halves;
    const uint32_t* __restrict__ tab = reinterpret_cast<const uint32_t*>(plan + a.off_table) + it.tab;
    const uint32_t pg_begin = it.kv_begin / kPage;
    const uint32_t pg_end = (it.kv_end + kPage - 1) / kPage;
    constexpr uint32_t STRIDE = W * PB;

    if constexpr (FUSED) {
        if (it.napp) {
            if constexpr (Q8)
                item_append_q8<D>(a, plan, it, lay, head, layer_off, page_stride, 64 * W);
            else
                item_append<D>(a, plan, it, lay, head, layer_off, page_stride, 64 * W);
            __syncthreads();
        }
    }

    // Page registers: K as the A operand (key col, dims c*32 + 8*rg ..), V
    // as coalesced rows (key i*KPL + lane/LPK, dims (lane%LPK)*8 ..).  Pages
    // past pg_end (possible only with PB > 1) are not loaded: their keys are
    // masked, and their registers are zeroed so that, Q8, p = 0 meets a
    // scale of 0, not whatever the registers held.
    // Q8: K as 8 int8 per (key, chunk), the scales of keys 4*rg .. 4*rg+3
    // (the rows of S^T and P^T this lane holds).
    struct Regs {
        u32x4 k[PB][QC];  // Q8: .x, .y hold 8 int8
        u32x4 v[PB][LPP];
        float4 ks[Q8 ? PB : 1], vs[Q8 ? PB : 1];
    };
    auto load = [&](uint32_t pg, Regs& r) {
#pragma unroll
        for (int b = 0; b < PB; b++) {
            if (pg + b >= pg_end) {
#pragma unroll
                for (int c = 0; c < QC; c++) r.k[b][c] = u32x4{0, 0, 0, 0};
#pragma unroll
                for (int i = 0; i < LPP; i++) r.v[b][i] = u32x4{0, 0, 0, 0};
                if constexpr (Q8) r.ks[b] = r.vs[b] = float4{0.f, 0.f, 0.f, 0.f};
                continue;
            }
            const uint64_t phys = tab[pg + b];
            if constexpr (Q8) {
                const uint8_t* kb = reinterpret_cast<const uint8_t*>(kbase + phys * page_stride);
                const uint8_t* vb = reinterpret_cast<const uint8_t*>(vbase + phys * page_stride);
#pragma unroll
                for (int c = 0; c < QC; c++) {
                    const uint2 w = *reinterpret_cast<const uint2*>(kb + col * D + c * 32 + 8 * rg);
                    r.k[b][c] = u32x4{w.x, w.y, 0u, 0u};
                }
#pragma unroll
                for (int i = 0; i < LPP; i++) r.v[b][i] = load16(reinterpret_cast<const u32x4*>(vb) + lane + i * 64);
                r.ks[b] = *reinterpret_cast<const float4*>(kb + kPage * D + 16 * rg);
                r.vs[b] = *reinterpret_cast<const float4*>(vb + kPage * D + 16 * rg);
            } else {
                const uint16_t* kp = kbase + phys * page_stride + col * D + 8 * rg;
                if constexpr (KT) {  // key i*KPL + lane/LPK, dims (lane%LPK)*8 (QC == LPP)
                    const u32x4* kq = reinterpret_cast<const u32x4*>(kbase + phys * page_stride) + lane;
#pragma unroll
                    for (int c = 0; c < QC; c++) r.k[b][c] = load16(kq + c * 64);
                } else {
#pragma unroll
                    for (int c = 0; c < QC; c++) r.k[b][c] = load16(reinterpret_cast<const u32x4*>(kp + c * 32));
                }
                const u32x4* vp = reinterpret_cast<const u32x4*>(vbase + phys * page_stride) + lane;
#pragma unroll
                for (int i = 0; i < LPP; i++) r.v[b][i] = load16(vp + i * 64);
            }
        }
    };
    Regs cur;
    uint32_t pg = pg_begin + wave * PB;
    if (pg < pg_end) load(pg, cur);

    // Q^T as the B operand: query col, dims c*32 + 8*rg .. +7, f16 hi + lo.
    half8_t qh[QC], ql[QC];
    {
        const bool has = col < (int)it.nq;
        const float* qb = a.q + (int64_t)lay * a.q_layer_stride + (int64_t)(it.row0 + (has ? col : 0)) * a.q_row_stride +
                          head * D + 8 * rg;
#pragma unroll
        for (int c = 0; c < QC; c++) {
            float x[8] = {0, 0, 0, 0, 0, 0, 0, 0};
            if (has) {
                const float4 x0 = reinterpret_cast<const float4*>(qb + c * 32)[0];
                const float4 x1 = reinterpret_cast<const float4*>(qb + c * 32)[1];
                x[0] = x0.x; x[1] = x0.y; x[2] = x0.z; x[3] = x0.w;
                x[4] = x1.x; x[5] = x1.y; x[6] = x1.z; x[7] = x1.w;
            }
#pragma unroll
            for (int e = 0; e < 8; e++) {
                _Float16 h, l;
                split_f16(x[e] * a.qscale, h, l);
                qh[c][e] = h;
                ql[c][e] = l;
            }
        }
    }
    float m = kMinScore, lsum = 0.f;
    float4_t o[VC];  // PV products of p's hi and lo parts, into one accumulator
#pragma unroll
    for (int c = 0; c < VC; c++) o[c] = float4_t{0.f, 0.f, 0.f, 0.f};
    // Q8: p enters PV as p * vs / vref (at most 2^14 after scaling, so its
    // f16 hi never overflows) and the accumulators hold the sum in units of
    // vref: vref starts at 1 (scales up to 1, values up to 127 in magnitude,
    // leave it there, and the products match p * vs * 2^14 bit for bit)
    // and follows the largest scale seen beyond that.
    float vref = 1.f, vinv = 1.f;  // vinv = 1 / vref
    _Float16* my_vt = vt[wave];
    const uint32_t qpos = it.pos0 + col;  // this lane's query position
    const bool qok = col < (int)it.nq;

    for (; pg < pg_end; pg += STRIDE) {
        Regs nxt;
        if (pg + STRIDE < pg_end) load(pg + STRIDE, nxt);
        // V rows to LDS; rows past kv_end as zeros (stale halves must not
        // reach the product even with p = 0).
#pragma unroll
        for (int b = 0; b < PB; b++) {
#pragma unroll
            for (int i = 0; i < LPP; i++) {
                const uint32_t key = b * kPage + i * KPL + lane / LPK;
                const u32x4 val = pg * kPage + key < it.kv_end ? cur.v[b][i] : u32x4{0, 0, 0, 0};
                if constexpr (Q8) {  // 16 values: chunks 2q, 2q+1 of the row
                    const uint32_t q = 2 * (lane % LPK);
                    const half4_t v0 = i8x4_f16(val[0]), v1 = i8x4_f16(val[1]);
                    const half4_t v2 = i8x4_f16(val[2]), v3 = i8x4_f16(val[3]);
                    *reinterpret_cast<half8_t*>(my_vt + tile_chunk<CH>(key, q) * 8) =
                        __builtin_shufflevector(v0, v1, 0, 1, 2, 3, 4, 5, 6, 7);
                    *reinterpret_cast<half8_t*>(my_vt + tile_chunk<CH>(key, q + 1) * 8) =
                        __builtin_shufflevector(v2, v3, 0, 1, 2, 3, 4, 5, 6, 7);
                } else {
                    *reinterpret_cast<u32x4*>(my_vt + tile_chunk<CH>(key, lane % LPK) * 8) = val;
                    if constexpr (KT) {
                        const u32x4 kv = pg * kPage + key < it.kv_end ? cur.k[b][i] : u32x4{0, 0, 0, 0};
                        *reinterpret_cast<u32x4*>(kt[wave] + tile_chunk<CH>(key, lane % LPK) * 8) = kv;
                    }
                }
            }
        }
        if constexpr (KT) {  // the K tile is read back by other lanes
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        }
        // S^T = K Q^T per page; scores of keys 4*rg+j of each page.
        float s[PB][4];
        float mx = -INFINITY;
#pragma unroll
        for (int b = 0; b < PB; b++) {
            float4_t st = {0.f, 0.f, 0.f, 0.f}, sl = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int c = 0; c < QC; c++) {
                half8_t kh;
                if constexpr (Q8) {
                    const half4_t k0 = i8x4_f16(cur.k[b][c][0]), k1 = i8x4_f16(cur.k[b][c][1]);
                    kh = half8_t{k0[0], k0[1], k0[2], k0[3], k1[0], k1[1], k1[2], k1[3]};
                } else if constexpr (KT) {  // key col, dims c*32 + 8*rg .. +7
                    kh = *reinterpret_cast<const half8_t*>(kt[wave] + tile_chunk<CH>(b * kPage + col, 4 * c + rg) * 8);
                } else {
                    kh = __builtin_bit_cast(half8_t, cur.k[b][c]);
                }
                st = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh, qh[c], st, 0, 0, 0);
                sl = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh, ql[c], sl, 0, 0, 0);
            }
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const uint32_t kp = (pg + b) * kPage + 4 * rg + j;
                const bool ok = qok && kp < it.kv_end && kp <= qpos;
                float sv = st[j] + sl[j] * kLoUnscale;
                if constexpr (Q8) sv *= cur.ks[b][j];
                s[b][j] = ok ? sv : -INFINITY;
                mx = fmaxf(mx, s[b][j]);
            }
        }
        mx = rows4_max(mx);
        const float mn = fmaxf(m, mx);
        const float alpha = fast_exp2(m - mn);
        float oalpha = alpha;  // the accumulators' factor
        m = mn;
        if constexpr (Q8) {
            // Past the reference vref, move it to the tile's largest value
            // scale (a scale belongs to its key, so the same for every lane
            // once reduced over the lane rows) and shrink the accumulators
            // with it. Scales past kv_end are stale: only the item's last
            // tile masks them.
            float vm = 0.f;
            if ((pg + PB) * kPage <= it.kv_end) {
#pragma unroll
                for (int b = 0; b < PB; b++)
#pragma unroll
                    for (int j = 0; j < 4; j++) vm = fmaxf(vm, cur.vs[b][j]);
            } else {
#pragma unroll
                for (int b = 0; b < PB; b++)
#pragma unroll
                    for (int j = 0; j < 4; j++)
                        if ((pg + b) * kPage + 4 * rg + j < it.kv_end) vm = fmaxf(vm, cur.vs[b][j]);
            }
            if (__any(vm > vref)) {
                vm = rows4_max(vm);
                oalpha *= vref / vm;
                vref = vm;
                vinv = 1.f / vm;
            }
        }
        // Weights scaled by 2^14 through the exponent reference, so lsum
        // is in those units too; Q8 weighs p by vs / vref before the split.
        const float mref = mn - kLog2PScale;
        half4_t ph[PB], pl[PB];
        float ps = 0.f;
#pragma unroll
        for (int b = 0; b < PB; b++) {
            float p[4];
#pragma unroll
            for (int j = 0; j < 4; j++) p[j] = fast_exp2(s[b][j] - mref);
            ps += (p[0] + p[1]) + (p[2] + p[3]);
            if constexpr (Q8) {
#pragma unroll
                for (int j = 0; j < 4; j++) p[j] *= cur.vs[b][j] * vinv;
            }
            uint32_t h0, l0, h1, l1;
            split_w16x2(p[0], p[1], h0, l0);
            split_w16x2(p[2], p[3], h1, l1);
            ph[b] = __builtin_bit_cast(half4_t, u32x2_t{h0, h1});
            pl[b] = __builtin_bit_cast(half4_t, u32x2_t{l0, l1});
        }
        lsum = lsum * alpha + ps;
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        // Rescale only when some query's running max (or, Q8, the value
        // scale reference) moved: otherwise every alpha is exactly 1 and the
        // multiplies change nothing.
        if (__any(oalpha != 1.f)) {
#pragma unroll
            for (int c = 0; c < VC; c++) o[c] *= oalpha;
        }
        // O^T += V^T P^T, 16 dims per product; V^T (dim c*16 + col of keys
        // 4*rg .. 4*rg+3) by a transposing read of the row-major tile, as in
        // attn_prefill_kernel, and pages in pairs through the 32-key product
        // when PB is even.
        auto vread = [&](int b, int c) {
            const int t = (lane >> 2) & 3, av = lane & 3;
            const _Float16* vp = my_vt + tile_chunk<CH>(b * kPage + 4 * rg + t, 2 * c + (av >> 1)) * 8 + (av & 1) * 4;
            return __builtin_bit_cast(
                half4_t, __builtin_amdgcn_ds_read_tr16_b64_v4f16((__attribute__((address_space(3))) v4fp16_t*)(vp)));
        };
        if constexpr (PB % 2 == 0) {
#pragma unroll
            for (int b = 0; b < PB; b += 2) {
                const half8_t p8h = __builtin_shufflevector(ph[b], ph[b + 1], 0, 1, 2, 3, 4, 5, 6, 7);
                const half8_t p8l = __builtin_shufflevector(pl[b], pl[b + 1], 0, 1, 2, 3, 4, 5, 6, 7);
#pragma unroll
                for (int c = 0; c < VC; c++) {
                    const half8_t v8 = __builtin_shufflevector(vread(b, c), vread(b + 1, c), 0, 1, 2, 3, 4, 5, 6, 7);
                    o[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(v8, p8h, o[c], 0, 0, 0);
                    o[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(v8, p8l, o[c], 0, 0, 0);
                }
            }
        } else {
#pragma unroll
            for (int c = 0; c < VC; c++) {
#pragma unroll
                for (int b = 0; b < PB; b++) {
                    const half4_t vt4 = vread(b, c);
                    o[c] = __builtin_amdgcn_mfma_f32_16x16x16f16(vt4, ph[b], o[c], 0, 0, 0);
                    o[c] = __builtin_amdgcn_mfma_f32_16x16x16f16(vt4, pl[b], o[c], 0, 0, 0);
                }
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        if (pg + STRIDE < pg_end) cur = nxt;
    }
    // Lanes q, q+16, q+32, q+48 hold partial sums of query q's softmax.
    lsum = rows4_sum(lsum);
    __syncthreads();  // every wave is done with its tiles, which `red` overwrites
    if (qok) {
        if (rg == 0) {
            red[wave][col][0] = m;
            red[wave][col][1] = lsum * kPUnscale;
        }
#pragma unroll
        for (int c = 0; c < VC; c++)
#pragma unroll
            for (int j = 0; j < 4; j++)
                red[wave][col][2 + c * 16 + 4 * rg + j] = o[c][j] * (kPUnscale * vref);
    }
    __syncthreads();
    for (uint32_t t = threadIdx.x; t < it.nq * D; t += 64 * W) {
        const uint32_t r = t / D, d = t - r * D;
        float M = red[0][r][0];
#pragma unroll
        for (int w = 1; w < W; w++) M = fmaxf(M, red[w][r][0]);
        float L = 0.f, O = 0.f;
#pragma unroll
        for (int w = 0; w < W; w++) {
            const float wt = fast_exp2(red[w][r][0] - M);
            L += red[w][r][1] * wt;
            O += red[w][r][2 + d] * wt;
        }
        if (it.part_slot == kNoSlot) {
            a.out[(int64_t)lay * a.out_layer_stride + (int64_t)(it.row0 + r) * a.out_row_stride + head * D + d] = O / L;
        } else {
            float* p = a.partials + ((((uint64_t)it.part_slot * a.n_lay + lay) * H + head) * NQ + r) * (D + 2);
            if (d == 0) {
                p[0] = M;
                p[1] = L;
            }
            p[2 + d] = O;
        }
    }
}

// ------------------------------------------------- attention, prefill groups
//
// Groups of kMfmaTile+1 .. kPrefillRows consecutive query rows of one
// sequence (a prompt chunk with every row queried).  Wave w owns rows
// 16w .. 16w+15 of the group and runs attn_mfma_kernel's per-page arithmetic
// for them (S^T = K Q^T with q split into f16 hi + scaled lo, the online
// softmax on S^T's columns, O^T += V^T P^T with p split likewise), but the
// workgroup's 256 threads copy each tile of PT pages of K and V once into LDS
// and all four waves read it there: each K/V byte leaves memory once per 64
// queries instead of once per 16.  Tiles travel by DMA
// (global_load_lds_dwordx4: lane l's 16 bytes land at the wave's LDS base +
// 16 l, whatever address the lane loads) through a ring of kPrefillStages
// tiles: two tiles in flight while one is computed, one barrier per tile, no
// registers held for them.  Rows past the item's end load the item's first
// key instead (finite data; their weights are 0), and a wave skips pages
// past its own last query.  No cross-wave merge: each wave writes its own
// rows (or their partials when the group is split into partitions).
// Pages per LDS tile (4: 383 against 364 us) and tiles in the ring (a
// 4-tile ring measured within 2%).
constexpr int kPrefillPages = 2;
constexpr int kPrefillStages = 3;
static_assert(kPrefillStages == 3 || kPrefillStages == 4, "ring of 3 or 4 tiles");

// 16 bytes per lane from g to LDS at the wave-uniform dst + 16 * lane
// (global_load_lds_dwordx4, M0 = dst's LDS address).  Written as assembly
// so that the compiler does not add a wait for every DMA in flight before
// each LDS read it cannot prove disjoint from them: the caller waits
// (vmcnt) and synchronises itself.  The "memory" clobber and dst as an
// operand tell the compiler that LDS may change here.  The s_nop is the one
// wait state CDNA requires between a scalar write of M0 and an LDS-DMA load
// reading it; the compiler inserts it for its own code but cannot see into
// the asm.
__device__ __forceinline__ void lds_dma16(const void* g, void* dst) {
    const uint32_t m0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)NI_LDS(dst));
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" : : "v"(g), "s"(m0) : "memory", "m0");
}
// The same from a wave-uniform base plus a per-lane 32-bit byte offset (the
// SADDR form: no 64-bit address per lane), to the LDS byte address lds.
__device__ __forceinline__ void lds_dma16_sbase(const void* base, uint32_t off, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" : : "v"(off), "s"(base), "s"(lds)
                 : "memory", "m0");
}
// The prefill kernel keeps its exponent reference m until some query's max
// exceeds it by more than kRefSlack (log2 units): weights are then up to
// 2^kRefSlack, so p enters PV scaled by 2^(15 - kRefSlack) (at most 2^15 in
// f16; weights down to 2^-31 of the reference stay nonzero as f16
// subnormals, which the matrix cores take exactly), and the accumulators
// are rescaled only when the reference moves.
constexpr float kRefSlack = 8.f;
constexpr float kLog2PScalePre = 7.f, kPUnscalePre = 1.f / 128.f;

// Q8 tiles (head_dim 64): int8 rows of 64 bytes, 16-byte chunk q of row key
// at key * 4 + (q ^ sw), sw = ((key >> 2) & 3) ^ (((key >> 4) & 1) << 1):
// the 16 lanes reading one chunk of 16 rows (the K operand) and the 32 lanes
// of a transposing read of 8 rows of two pages (the V operand) both hit
// distinct banks.
__device__ __forceinline__ uint32_t tile_chunk_q8(uint32_t key, uint32_t q) {
    return key * 4 + (q ^ (((key >> 2) & 3) ^ (((key >> 4) & 1) << 1)));
}
typedef int v2i32_t __attribute__((ext_vector_type(2)));

// Wait until at most `ahead` tiles of N DMA loads each are outstanding (vmcnt
// counts this wave's loads in order).
template <int N>
__device__ __forceinline__ void wait_tiles(uint32_t ahead) {
    if (ahead >= 2)
        __builtin_amdgcn_s_waitcnt(0x0f70 | (2 * N));
    else if (ahead == 1)
        __builtin_amdgcn_s_waitcnt(0x0f70 | N);
    else
        __builtin_amdgcn_s_waitcnt(0x0f70);
}

// QKV projection of mid-size batches (kQkvSmallRows < n <= kQkvMidRows):
// a workgroup of 8 waves owns a 16-row x 16-feature tile, as
// qkv_small_kernel with one row block, but x and W reach the matrix cores
// through LDS.  Loading operands straight into the matrix-core layout reads
// 16 rows x 64 bytes per instruction, half of each 128-byte line; x is read
// by every feature tile, and those half-line reads cost ~4 us per layer more
// than whole-line ones at 64 rows (measured).  Here every thread issues all
// its loads of the tile at once, whole lines (wave p: rows 2p and 2p+1 of x
// and of W, 512 contiguous bytes each per chunk of 128 values of d_in), NC
// chunks in registers (6 up to d_in 768, else 8: d_in <= 1024); then chunk by chunk the tile goes
// through a double-buffered LDS chunk (one barrier per chunk) into the
// matrix-core layout.  Row r's 16-byte piece q sits in slot q ^ (r & 15) of
// its 512-byte LDS row, so the 16 lanes reading piece q of 16 rows hit
// distinct banks.  Wave p multiplies slice p of every chunk -- part p, in
// increasing slice order: the same products in the same order as the other
// two kernels -- and the parts meet in LDS, so the bits are the same at
// every row count.  (A 3-stage DMA ring of chunks instead, two in flight:
// 103 us per 12 layers at 64 rows, latency-bound.)
constexpr uint32_t kQkvMidRows = 64;
constexpr int kQkvMidChunks = 8;  // chunks of d_in held in registers: d_in up to 1024 on this kernel

template <int INL, int WF, int NC>
__global__ __launch_bounds__(64 * kQkvParts) void qkv_mid_kernel(const QkvLaunch a, const PlanArg<INL> pa) {
    typedef float f4 __attribute__((ext_vector_type(4)));
    constexpr int KC = kQkvChunk;       // d_in values per chunk (8 slices of 16)
    constexpr uint32_t RB = KC * 4;     // bytes of one row's chunk (512)
    constexpr uint32_t CB = 16 * RB;    // bytes of 16 rows' chunk (8 KB)
    static_assert(NC <= kQkvMidChunks, "chunks held in registers");
    static_assert(KC == 128 && kQkvParts == 8, "two rows of 32 pieces per wave and chunk, 8 waves");
    __shared__ __attribute__((aligned(16))) uint8_t buf[2][2 * CB];  // [x rows | W rows], double-buffered
    const int lane = threadIdx.x & 63;
    const uint32_t p = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int i = lane & 15, g = lane >> 4;
    // Workgroups go to the 8 XCDs in turn (w % 8), each XCD with its own L2.
    // The nx row tiles of feature tile f are dealt to one XCD back to back,
    // so W's tile leaves HBM once and the other row tiles read it from that
    // L2 (the row tiles of a feature tile on different XCDs made half of all
    // L2 requests misses at 64 rows).  Needs the feature-tile count to be a
    // multiple of 8; otherwise the plain order.
    const uint32_t nx = gridDim.x / (a.n_feat / 16), w = blockIdx.x;
    uint32_t rt = w % nx, ft = w / nx;
    if ((a.n_feat / 16) % 8 == 0) {
        const uint32_t k = w / 8;
        rt = k % nx;
        ft = 8 * (k / nx) + w % 8;
    }
    const uint32_t m0 = rt * 16, n0 = ft * 16;
    const uint32_t n_slices = a.d_in / 16;
    const uint32_t n_chunks = (a.d_in + KC - 1) / KC;
    // This thread's share of every chunk: piece `pc` of row `dr` (x and W).
    // Rows past n_rows repeat the last row; pieces past d_in (the last,
    // partial chunk) load the row's first piece (their slices are skipped).
    const uint32_t dr = 2 * p + (lane >> 5), pc = lane & 31;
    const float* xsrc = a.x + (int64_t)min(m0 + dr, a.n_rows - 1) * a.x_row_stride;

    const uint32_t wo = dr * RB + 16u * (pc ^ (dr & 15));
    // Lane (i, g) reads piece 4p + g of x row i and of W row i.
    const uint32_t rd = (uint32_t)i * RB + 16u * ((4u * p + (uint32_t)g) ^ (uint32_t)i);
    // Every load at once (d_in <= NC chunks; chunks past the end repeat the
    // last one, unused): branches or a loop here put xr/wr on the stack.
    f4 xr[NC], wr[NC];  // native vectors: HIP's float4 struct copied into LDS kept them on the stack
#pragma clang loop unroll(full)
    for (int j = 0; j < NC; j++) {
        uint32_t col = min((uint32_t)j, n_chunks - 1) * KC + 4 * pc;
        col = col < a.d_in ? col : 0;
        xr[j] = *reinterpret_cast<const f4*>(xsrc + col);
        wr[j] = qkv_w4<WF>(a, n0 + dr, col);
    }
    // What the store at the end needs (wave 0: rows m0 + 4g .. +3, feature
    // n0 + i): the rows' append entries and the bias, loaded with the
    // operands instead of after the sum.
    const AppendEntry* entries = reinterpret_cast<const AppendEntry*>(plan_base(pa, a.plan) + a.off_entries);
    AppendEntry en[4] = {};
    float bias = 0.f;
    if (p == 0) {
        if (a.fused && n0 >= a.n_feat / 3) {
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const AppendEntry& r = entries[min(m0 + 4 * g + e, a.n_rows - 1)];
                en[e].page = r.page;  // (the store needs page and slot only)
                en[e].slot = r.slot;
            }
        }
        if (a.bias) bias = a.bias[n0 + i];
    }
    f4 acc = f4{0.f, 0.f, 0.f, 0.f};
#pragma clang loop unroll(full)
    for (int j = 0; j < NC; j++) {
        if ((uint32_t)j < n_chunks) {  // uniform
            uint8_t* b = buf[j & 1];
            // buf[j & 1] was last read for chunk j - 2, before every wave
            // passed the barrier of chunk j - 1.
            *reinterpret_cast<f4*>(b + wo) = xr[j];
            *reinterpret_cast<f4*>(b + CB + wo) = wr[j];
            __syncthreads();
            if (8 * (uint32_t)j + p < n_slices) {
                const float4 xv = *reinterpret_cast<const float4*>(b + rd);
                const float4 wv = *reinterpret_cast<const float4*>(b + CB + rd);
                acc = __builtin_amdgcn_mfma_f32_16x16x4f32(xv.x, wv.x, acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_16x16x4f32(xv.y, wv.y, acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_16x16x4f32(xv.z, wv.z, acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_16x16x4f32(xv.w, wv.w, acc, 0, 0, 0);
            }
        }
    }
    __syncthreads();  // every wave is done with the buffers: reuse them for the parts
    f4* red = reinterpret_cast<f4*>(&buf[0][0]);
    red[p * 64 + lane] = acc;
    __syncthreads();
    if (p != 0) return;
    // The same tree as qkv_kernel and qkv_small_kernel.
    const f4 y = ((red[0 * 64 + lane] + red[1 * 64 + lane]) + (red[2 * 64 + lane] + red[3 * 64 + lane])) +
                 ((red[4 * 64 + lane] + red[5 * 64 + lane]) + (red[6 * 64 + lane] + red[7 * 64 + lane]));
    const uint32_t f = n0 + i;
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const uint32_t row = m0 + 4 * g + e;
        if (row >= a.n_rows) break;
        qkv_store_en(a, en[e], row, f, y[e] + bias);
    }
}

// The new rows app0 .. app0+napp-1 of one (layer, head) appended by a whole
// workgroup: item_append's enumeration with U chunks per thread loaded
// before any is stored, so a prompt's hundreds of rows stream instead of
// paying a load latency per chunk.  Loads past the end read the last chunk
// again (in bounds) and are not stored; Q8's D/8-lane groups stay whole.
constexpr int kSeqAppendUnroll = 4;
template <int D, bool Q8, int U>
__device__ __forceinline__ void seq_append(const AttnLaunch& a, const uint8_t* plan, uint32_t app0, uint32_t napp,
                                           uint32_t lay, uint32_t head, uint64_t layer_off, uint32_t nthreads) {
    constexpr uint32_t CH = D / 8;
    const uint32_t n = napp * 2 * CH;
    const AppendEntry* ent = reinterpret_cast<const AppendEntry*>(plan + a.off_app) + app0;
    for (uint32_t t0 = threadIdx.x; t0 < n; t0 += nthreads * U) {
        qkv_f4 x[U][2];
        AppendEntry e[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const uint32_t t = min(t0 + u * nthreads, n - 1);
            const uint32_t row = t / (2 * CH);
            const uint32_t rem2 = t - row * (2 * CH);
            const uint32_t is_v = rem2 >= CH;
            const uint32_t c = (rem2 - is_v * CH) * 8;
            e[u] = ent[row];
            const float* src = (is_v ? a.v : a.k) + (int64_t)lay * a.kv_layer_stride +
                               (int64_t)(app0 + row) * a.kv_row_stride + head * D + c;  // entry i: input row i
            x[u][0] = reinterpret_cast<const qkv_f4*>(src)[0];
            x[u][1] = reinterpret_cast<const qkv_f4*>(src)[1];
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            const uint32_t t = t0 + u * nthreads;
            if (t >= n) break;
            const uint32_t row = t / (2 * CH);
            const uint32_t rem2 = t - row * (2 * CH);
            const uint32_t is_v = rem2 >= CH;
            const uint32_t c = (rem2 - is_v * CH) * 8;
            const float4 x0 = make_float4(x[u][0].x, x[u][0].y, x[u][0].z, x[u][0].w);
            const float4 x1 = make_float4(x[u][1].x, x[u][1].y, x[u][1].z, x[u][1].w);
            const uint64_t pg = layer_off + (uint64_t)e[u].page * a.pool.page_halves;
            if constexpr (Q8) {
                q8_store8(q8_block(a.pool, is_v, pg), D, e[u].slot, c, x0, x1);
            } else {
                uint16_t* dst = (is_v ? a.pool.v : a.pool.k) + pg + e[u].slot * D + c;
                *reinterpret_cast<uint4*>(dst) = pack8(x0, x1);
            }
        }
    }
}

// Prompt-chunk groups on the Q8 cache (head_dim 64): int8 K/V tiles and
// their scales by DMA, K converted to f16 after an 8-byte LDS read, V^T
// through the 8-bit transposing read; p enters PV weighted by the value
// scales, its hi and lo parts' products into one accumulator (one layer per
// launch, 16 x 512 rows: 787-789 -> 764-765 us per step; all layers 483 ->
// 480).  SEQ: one workgroup per (sequence, layer, head) running the
// sequence's groups in turn, each after appending its rows for the head.
template <int INL, bool SEQ>
__global__ __launch_bounds__(256) void attn_prefill_q8_kernel(const AttnLaunch a, const PlanArg<INL> pa) {
    constexpr int D = 64, PT = kPrefillPages;
    constexpr int QC = D / 32;              // 32-dim chunks of the QK product
    constexpr int VC = D / 16;              // 16-dim chunks of the PV product
    constexpr int TK = PT * (int)kPage;     // keys per tile
    static_assert(PT == 2, "Q8 tiles: two pages");
    // A stage: [K int8 | V int8 | K scales | V scales], TK * D bytes each,
    // then TK floats each.
    constexpr int QS = 2 * TK * D;          // byte offset of the K scales in a stage
    constexpr int SB = QS + 8 * TK;
    __shared__ __attribute__((aligned(16))) uint8_t ring[kPrefillStages][SB];

    const int lane = threadIdx.x & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t H = a.pool.n_head;
    const uint32_t lh = a.n_lay * H;
    const uint8_t* plan = plan_base(pa, a.plan);
    const uint32_t unit = blockIdx.x / lh;
    const uint32_t rem = blockIdx.x - unit * lh;
    const uint32_t lay = rem / H;
    const uint32_t head = rem - lay * H;
    // One item per workgroup, or (a.n_pseqs) the items of one sequence of a
    // prompt-chunk step in turn, each appending its new rows for this (layer,
    // head) first -- no other workgroup reads or writes those blocks, and the
    // vector L1 starts the kernel clean, so after the barrier the tiles'
    // loads see the stores.
    // (SEQ: the launch has a.n_pseqs sequences; otherwise one item per unit.)
    uint32_t item0 = unit, n_items = 1;
    if constexpr (SEQ) {
        const PrefillSeq ps = reinterpret_cast<const PrefillSeq*>(plan + a.off_pseqs)[unit];
        item0 = ps.item0;
        n_items = ps.n_items;
    }
    for (uint32_t item_i = item0; item_i < item0 + n_items; item_i++) {
    const AttnItem it = reinterpret_cast<const AttnItem*>(plan + a.off_items)[item_i];
    if constexpr (SEQ) {
        if (it.napp) {  // rows past the previous item's keys: no wave still reads them
            const uint64_t loff =
                (uint64_t)(a.layer0 + lay) * a.pool.layer_halves + (uint64_t)head * a.pool.head_halves;
            seq_append<D, true, kSeqAppendUnroll>(a, plan, it.app0, it.napp, lay, head, loff, 256);
        }
        if (item_i != item0 || it.napp) __syncthreads();  // ring free again; the rows stored
    }
    const int col = lane & 15;  // query slot of S^T / O^T columns
    const int rg = lane >> 4;   // row group: keys (or dims) 4*rg .. 4*rg+3

    const uint64_t layer_off = (uint64_t)(a.layer0 + lay) * a.pool.layer_halves + (uint64_t)head * a.pool.head_halves;
    const uint64_t page_stride = a.pool.page_halves;
    const uint8_t* kb8 = reinterpret_cast<const uint8_t*>(a.pool.k + layer_off);  // in bytes
    const uint8_t* vb8 = reinterpret_cast<const uint8_t*>(a.pool.v + layer_off);
    // Page ids through the constant address space: wave-uniform scalar loads,
    // which a wait for the DMA tiles (in order with every vector load) does
    // not depend on.
    const __attribute__((address_space(4))) uint32_t* tab =
        (const __attribute__((address_space(4))) uint32_t*)(plan + a.off_table) + it.tab;
    const uint32_t pg_begin = it.kv_begin / kPage;
    const uint32_t pg_end = (it.kv_end + kPage - 1) / kPage;

    // This wave's queries: rows r0 .. r0+nqw-1 of the group.
    const uint32_t r0 = wave * 16;
    const uint32_t nqw = it.nq > r0 ? min(16u, it.nq - r0) : 0u;
    const bool qok = col < (int)nqw;
    const uint32_t qpos = it.pos0 + r0 + col;
    const uint32_t kend_w = min(it.kv_end, it.pos0 + r0 + nqw);  // keys this wave needs end here
    // Keys below this are visible to every query of the wave (no masking).
    const uint32_t kfull_w = min(it.kv_end, it.pos0 + r0 + 1);

    // Tile DMA: thread t copies int8 chunk t % 128 of K (waves 0, 1) or V
    // (waves 2, 3), and lanes 0..15 of wave 0 the 16 chunks of scales (4 keys
    // each, K then V): one DMA load per tile, wave 0 two, so "tile i landed"
    // is "at most the later tiles' loads outstanding".  A row past the item's
    // end reads the tile's first row, a key of this item.
    auto issue = [&](int st, uint32_t pg) {
        uint64_t base[PT];  // bytes
#pragma unroll
        for (int b = 0; b < PT; b++) base[b] = (uint64_t)tab[min(pg + b, pg_end - 1)] * page_stride * 2;
        const uint32_t u = threadIdx.x & 127, dkey = u / 4;
        const uint32_t dq = u % 4 ^ (tile_chunk_q8(dkey, 0) - dkey * 4);
        const bool in = pg * kPage + dkey < it.kv_end;
        uint64_t pb = base[0];
#pragma unroll
        for (int b = 1; b < PT; b++)
            if (in && dkey / kPage == (uint32_t)b) pb = base[b];
        const uint32_t off = (in ? (dkey % kPage) * D : 0u) + dq * 16;
        lds_dma16((threadIdx.x < 128 ? kb8 : vb8) + pb + off, &ring[st][0] + 1024 * wave);
        if (wave == 0 && lane < 16) {
            const uint32_t skey = 4 * (lane & 7);
            const bool sin = pg * kPage + skey < it.kv_end;
            uint64_t spb = base[0];
#pragma unroll
            for (int b = 1; b < PT; b++)
                if (sin && skey / kPage == (uint32_t)b) spb = base[b];
            const uint32_t soff = kPage * D + (sin ? (skey % kPage) * 4 : 0u);
            lds_dma16((lane < 8 ? kb8 : vb8) + spb + soff, &ring[st][QS]);
        }
    };
    const uint32_t n_tiles = (pg_end - pg_begin + PT - 1) / PT;
#pragma unroll
    for (int t = 0; t < kPrefillStages - 1; t++)
        if ((uint32_t)t < n_tiles) issue(t, pg_begin + t * PT);

    // Q^T as the B operand: query col, dims c*32 + 8*rg .. +7, f16 hi + lo
    // (lo = f16(q - hi) unscaled: the matrix cores take its subnormals
    // exactly, so both halves accumulate into one product); K^T's int8
    // values are exact in f16.
    half8_t qh[QC], ql[QC];
    {
        // (a lane without a query reads the item's first row: rows past nq
        // may lie past the end of the caller's q)
        const float* qb = a.q + (int64_t)lay * a.q_layer_stride +
                          (int64_t)(it.row0 + (qok ? r0 + col : 0)) * a.q_row_stride + head * D + 8 * rg;
#pragma unroll
        for (int c = 0; c < QC; c++) {
            float x[8] = {0, 0, 0, 0, 0, 0, 0, 0};
            if (qok) {
                const float4 x0 = reinterpret_cast<const float4*>(qb + c * 32)[0];
                const float4 x1 = reinterpret_cast<const float4*>(qb + c * 32)[1];
                x[0] = x0.x; x[1] = x0.y; x[2] = x0.z; x[3] = x0.w;
                x[4] = x1.x; x[5] = x1.y; x[6] = x1.z; x[7] = x1.w;
            }
#pragma unroll
            for (int e = 0; e < 8; e += 2) {
                float x0 = x[e] * a.qscale, x1 = x[e + 1] * a.qscale;
                asm("" : "+v"(x0), "+v"(x1));  // the f32 products, as the split's residual sees them
                uint32_t h, l;
                split_w16x2(x0, x1, h, l);
                const half2_t hh = __builtin_bit_cast(half2_t, h), ll = __builtin_bit_cast(half2_t, l);
                qh[c][e] = hh[0];
                qh[c][e + 1] = hh[1];
                ql[c][e] = ll[0];
                ql[c][e + 1] = ll[1];
            }
        }
    }
    // Weights are exp2(s - mref) with mref = m - kLog2PScalePre: p already
    // scaled by 2^7, and lsum and the accumulators in the same units.
    float m = kMinScore, mref = kMinScore - kLog2PScalePre, lsum = 0.f;
    // p enters PV as p * vs / vref and the accumulators hold the sum in
    // units of vref, which starts at 1 and follows the largest value scale
    // seen beyond that (as in attn_mfma_kernel): p * vs / vref <= 2^15.
    float vref = 1.f, vinv = 1.f;
    float4_t o[VC];  // PV products of p's hi and lo parts, into one accumulator
#pragma unroll
    for (int c = 0; c < VC; c++) o[c] = float4_t{0.f, 0.f, 0.f, 0.f};

    int st = 0;  // ring stage of tile ti
    for (uint32_t ti = 0; ti < n_tiles; ti++) {
        const uint32_t pg = pg_begin + ti * PT;
        // This wave's part of tile ti has landed (vmcnt is in order: only
        // the two loads of each later tile already issued may still be
        // outstanding); after the barrier every wave's part has, and every
        // wave is done with tile ti-1, whose stage the next tile takes.
        const uint32_t ahead = min(n_tiles - 1 - ti, (uint32_t)(kPrefillStages - 2));
        if (wave == 0)
            wait_tiles<2>(ahead);
        else
            wait_tiles<1>(ahead);
        __syncthreads();
        if (ti + kPrefillStages - 1 < n_tiles)
            issue(st == 0 ? kPrefillStages - 1 : st - 1, pg + (kPrefillStages - 1) * PT);
        const uint8_t* const kt8 = &ring[st][0];
        const uint8_t* const vt8 = kt8 + TK * D;
        const float* const kst = reinterpret_cast<const float*>(&ring[st][QS]);  // Q8 scales
        const float* const vst = kst + TK;
        if (pg * kPage < kend_w) {  // wave-uniform: the tile holds keys this wave needs
            // Pages b < nb of the tile are needed; one softmax update per tile.
            const uint32_t nb = min((uint32_t)PT, (kend_w - pg * kPage + kPage - 1) / kPage);
            const bool full = (pg + PT) * kPage <= kfull_w;  // every key visible to every query
            float sc[PT][4];
#pragma unroll
            for (int b = 0; b < PT; b++) {
                // S^T = K Q^T: scores of keys 4*rg+j of page b for query col
                // (also of a page past nb: its rows are finite, its scores
                // masked below).
                float4_t st = {0.f, 0.f, 0.f, 0.f};
                half8_t kh[QC];
#pragma unroll
                for (int c = 0; c < QC; c++) {  // 8 int8 of the row (chunk 2c + rg/2, half rg%2) as f16
                    const uint2 w = *reinterpret_cast<const uint2*>(
                        kt8 + tile_chunk_q8(b * kPage + col, 2 * c + (rg >> 1)) * 16 + (rg & 1) * 8);
                    kh[c] = __builtin_shufflevector(i8x4_f16(w.x), i8x4_f16(w.y), 0, 1, 2, 3, 4, 5, 6, 7);
                }
#pragma unroll
                for (int c = 0; c < QC; c++) st = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh[c], qh[c], st, 0, 0, 0);
#pragma unroll
                for (int c = 0; c < QC; c++) st = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh[c], ql[c], st, 0, 0, 0);
#pragma unroll
                for (int j = 0; j < 4; j++) sc[b][j] = st[j];
                // key scales of keys 4*rg .. 4*rg+3
                const float4 ks = *reinterpret_cast<const float4*>(kst + b * kPage + 4 * rg);
                sc[b][0] *= ks.x;
                sc[b][1] *= ks.y;
                sc[b][2] *= ks.z;
                sc[b][3] *= ks.w;
            }
            if (!full) {
#pragma unroll
                for (int b = 0; b < PT; b++)
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        const uint32_t key = (pg + b) * kPage + 4 * rg + j;
                        const bool ok = qok && b < (int)nb && key < it.kv_end && key <= qpos;
                        sc[b][j] = ok ? sc[b][j] : -INFINITY;
                    }
            }
            float mx = sc[0][0];
#pragma unroll
            for (int b = 0; b < PT; b++)
#pragma unroll
                for (int j = 0; j < 4; j++) mx = fmaxf(mx, sc[b][j]);
            mx = rows4_max(mx);
            // Move every query's reference to its running max (and rescale)
            // only when some query's max got more than kRefSlack above it.
            if (__any(mx > m + kRefSlack)) {
                const float mn = fmaxf(m, mx);
                const float alpha = fast_exp2(m - mn);
                m = mn;
                mref = mn - kLog2PScalePre;
                lsum *= alpha;
#pragma unroll
                for (int c = 0; c < VC; c++) o[c] *= alpha;
            }
            // Value scales of keys 4*rg .. 4*rg+3 of each page; past the
            // reference vref, move it to the tile's largest (rows of pages
            // past the end hold other keys' finite scales) and shrink the
            // accumulators with it.
            float4 vs[PT];
            float vm = 0.f;
#pragma unroll
            for (int b = 0; b < PT; b++) {
                vs[b] = *reinterpret_cast<const float4*>(vst + b * kPage + 4 * rg);
                vm = fmaxf(fmaxf(vm, fmaxf(vs[b].x, vs[b].y)), fmaxf(vs[b].z, vs[b].w));
            }
            if (__any(vm > vref)) {
                vm = rows4_max(vm);
                const float f = vref / vm;
#pragma unroll
                for (int c = 0; c < VC; c++) o[c] *= f;
                vref = vm;
                vinv = 1.f / vm;
            }
            half4_t ph[PT], pl[PT];
            float ps[PT];
#pragma unroll
            for (int b = 0; b < PT; b++) {
                float p[4];
#pragma unroll
                for (int j = 0; j < 4; j++) p[j] = fast_exp2(sc[b][j] - mref);
                ps[b] = (p[0] + p[1]) + (p[2] + p[3]);
                p[0] *= vs[b].x * vinv;
                p[1] *= vs[b].y * vinv;
                p[2] *= vs[b].z * vinv;
                p[3] *= vs[b].w * vinv;
                uint32_t h0, l0, h1, l1;
                split_w16x2(p[0], p[1], h0, l0);
                split_w16x2(p[2], p[3], h1, l1);
                ph[b] = __builtin_bit_cast(half4_t, u32x2_t{h0, h1});
                pl[b] = __builtin_bit_cast(half4_t, u32x2_t{l0, l1});
            }
#pragma unroll
            for (int b = 0; b < PT; b++) lsum += ps[b];
            // O^T += V^T P^T, 16 dims per product, the pages in pairs through
            // the 32-key product (k-slot 8*rg + 4*i + j of the pair is key
            // 4*rg + j of its page i, in both operands).  A lane's V^T operand
            // comes from one 8-bit transposing read (ds_read_b64_tr_b8:
            // within 16 lanes, lane 2e+a reads bytes 8a .. 8a+7 of its row and
            // lane 8a'+b' receives byte b' of lanes a', 2+a', .., 14+a'),
            // giving dim c*16 + col of the pair's 8 keys: lane 2e+a reads dims
            // c*16 + 8a .. of key 4*rg + e of page b (e < 4) or b+1.
            auto vread8 = [&](int b, int c) {
                const int e = (lane & 15) >> 1, av = lane & 1;
                const uint32_t key = (e < 4 ? b : b + 1) * kPage + 4 * rg + (e & 3);
                const v2i32_t r = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
                    (__attribute__((address_space(3))) v2i32_t*)(vt8 + tile_chunk_q8(key, c) * 16 + av * 8));
                return __builtin_shufflevector(i8x4_f16((uint32_t)r.x), i8x4_f16((uint32_t)r.y), 0, 1, 2, 3, 4, 5, 6,
                                               7);
            };
#pragma unroll
            for (int b = 0; b < PT; b += 2) {
                if (b >= (int)nb) break;  // a page past nb has p = 0 and finite V
                const half8_t p8h = __builtin_shufflevector(ph[b], ph[b + 1], 0, 1, 2, 3, 4, 5, 6, 7);
                const half8_t p8l = __builtin_shufflevector(pl[b], pl[b + 1], 0, 1, 2, 3, 4, 5, 6, 7);
#pragma unroll
                for (int c = 0; c < VC; c++) {
                    const half8_t v8 = vread8(b, c);
                    o[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(v8, p8h, o[c], 0, 0, 0);
                    o[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(v8, p8l, o[c], 0, 0, 0);
                }
            }
        }
        st = st == kPrefillStages - 1 ? 0 : st + 1;
    }
    // Lanes q, q+16, q+32, q+48 hold partial sums of query q's softmax.
    lsum = rows4_sum(lsum);
    if (qok) {
    const uint32_t row = it.row0 + r0 + col;
    if (it.part_slot == kNoSlot) {
        float* dst = a.out + (int64_t)lay * a.out_layer_stride + (int64_t)row * a.out_row_stride + head * D;
        const float scale = vref / lsum;  // lsum and o both carry the 2^7; o in units of vref
#pragma unroll
        for (int c = 0; c < VC; c++) {
            float4 y;
            y.x = o[c][0] * scale;
            y.y = o[c][1] * scale;
            y.z = o[c][2] * scale;
            y.w = o[c][3] * scale;
            *reinterpret_cast<float4*>(dst + c * 16 + 4 * rg) = y;
        }
    } else {
        float* p = a.partials + ((((uint64_t)it.part_slot * a.n_lay + lay) * H + head) * kPrefillRows + r0 + col) * (D + 2);
        if (rg == 0) {
            p[0] = m;
            p[1] = lsum * kPUnscalePre;
        }
#pragma unroll
        for (int c = 0; c < VC; c++)
#pragma unroll
            for (int j = 0; j < 4; j++) p[2 + c * 16 + 4 * rg + j] = o[c][j] * (kPUnscalePre * vref);
    }
    }  // qok
    }  // items
}

// Prompt-chunk groups on f16 pools: the tiles, ring and products of
// attn_prefill_q8_kernel (64-row groups, four 16-query waves, K/V tiles by
// LDS DMA through a 3-tile ring, q and p split into f16 hi + lo on the
// matrix cores), with the per-tile work cut to what the products need:
//  * a wave's rows of a tile lie in one page (64 / CH rows per wave), so its
//    DMA takes a scalar page base plus a fixed per-lane offset (the
//    global_load_lds SADDR form: no per-lane address arithmetic), the page id
//    read by v_readlane from a register holding 64 of the item's page ids;
//  * the loop body is instantiated once per ring stage, so every LDS address
//    is a per-lane constant plus an immediate offset;
//  * scores come out of the QK product already relative to the exponent
//    reference (its negation is the accumulator's initial value), and the
//    per-tile test of "some score moved more than kRefSlack above the
//    reference" is a per-lane max against a constant; the cross-lane max
//    and the rescale run only when it fires (and on a wave's first tile,
//    which sets the reference);
//  * each query's sum of weights accumulates on the matrix cores (the
//    weights times a V^T of ones), in the same f16 hi + lo parts as PV;
//  * the PV products of p's hi and lo parts go into one accumulator (the
//    lo part is ~2^-11 of the hi part: the f32 sum loses nothing), which
//    frees the registers for 6 waves per SIMD (74 VGPRs; two accumulators
//    took 90 at 5 waves: 418-420 against 412-413 us per 16 x 512 step).
// The prologue issues the first tiles' DMA from the page ids the item
// carries, the item's q rows and 64 page ids beside it, then splits q while
// the tiles land.  One workgroup per (head, layer, item): blockIdx.x, .y, .z,
// or (a.ordered) a 1-D grid whose block b runs unit order[b] of the plan.
template <int ST>
struct RingStage {
    static constexpr int value = ST;
};

template <int D, int PT, int INL>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(D == 64 ? 6 : 1, 8))) void attn_prefill_kernel(
    const AttnLaunch a, const PlanArg<INL> pa) {
    constexpr int QC = D / 32;           // 32-dim chunks of the QK product
    constexpr int VC = D / 16;           // 16-dim chunks of the PV product
    constexpr int TK = PT * (int)kPage;  // keys per tile
    constexpr int CH = D / 8;            // 16-byte chunks per key row
    constexpr int TH = TK * D;           // halves per K (or V) tile
    constexpr int SB = 4 * TH;           // bytes per ring stage: K tile, V tile
    constexpr int NS = kPrefillStages;
    constexpr int WR = 64 / CH;          // tile rows one wave's DMA covers
    static_assert(TK * CH == 256, "one 16-byte chunk of K and one of V per thread per tile");
    static_assert(kPage % WR == 0, "a wave's DMA rows lie in one page");
    constexpr float kHi = kRefSlack + kLog2PScalePre;  // scores relative to the reference past this
    __shared__ __attribute__((aligned(16))) uint8_t ring[NS][SB];

    const int lane = threadIdx.x & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint8_t* plan = plan_base(pa, a.plan);
    uint32_t head = blockIdx.x, lay = blockIdx.y, item = blockIdx.z;
    if (a.ordered) {  // a 1-D grid: block b runs unit order[b], dealt to the CUs by the host
        const AttnUnit un = attn_unit(a, plan, blockIdx.x);
        item = un.item;
        lay = un.lay;
        head = un.head;
    }
    const AttnItem it = reinterpret_cast<const AttnItem*>(plan + a.off_items)[item];
    const int col = lane & 15;  // query slot of S^T / O^T columns
    const int rg = lane >> 4;   // row group: keys (or dims) 4*rg .. 4*rg+3

    const uint64_t layer_off = (uint64_t)(a.layer0 + lay) * a.pool.layer_halves + (uint64_t)head * a.pool.head_halves;
    const uint8_t* kbase = reinterpret_cast<const uint8_t*>(a.pool.k + layer_off);
    const uint8_t* vbase = reinterpret_cast<const uint8_t*>(a.pool.v + layer_off);
    const uint64_t page_bytes = 2 * a.pool.page_halves;
    const __attribute__((address_space(4))) uint32_t* tab =
        (const __attribute__((address_space(4))) uint32_t*)(plan + a.off_table) + it.tab;
    const uint32_t pg_begin = it.kv_begin / kPage;
    const uint32_t pg_end = (it.kv_end + kPage - 1) / kPage;
    const uint32_t n_tiles = (pg_end - pg_begin + PT - 1) / PT;

    // This wave's queries: rows r0 .. r0+nqw-1 of the group.
    const uint32_t r0 = wave * 16;
    const uint32_t nqw = it.nq > r0 ? min(16u, it.nq - r0) : 0u;
    const bool qok = col < (int)nqw;
    const uint32_t qpos = it.pos0 + r0 + col;
    const uint32_t kend_w = min(it.kv_end, it.pos0 + r0 + nqw);  // keys this wave needs end here
    const uint32_t kfull_w = min(it.kv_end, it.pos0 + r0 + 1);   // keys below this: visible to all its queries


    // Tile DMA: thread t copies LDS chunk t of the tile's K and of its V (row
    // t / CH, logical chunk (t % CH) ^ sw, tile_chunk's inverse); a row past
    // the item's end copies row 0 of its page (a key of this item).
    const uint32_t wb = (64 * wave / CH) / kPage;  // this wave's page within a tile
    const uint32_t dk = threadIdx.x / CH;
    const uint32_t doff0 = ((threadIdx.x % CH) ^ (tile_chunk<CH>(dk, 0) - dk * CH)) * 16;  // bytes, in row 0
    const uint32_t doff = doff0 + (dk % kPage) * D * 2;
    const uint32_t lds_ring = (uint32_t)(uintptr_t)NI_LDS(&ring[0][0]) + 1024 * wave;  // this wave's 1 KB of stage 0
    // Tile at page pg from this wave's page id `pid` (page pg + wb, or a page
    // of the item when that one is past its end: its rows are then masked).
    auto issue_pid = [&](auto stc, uint32_t pg, uint32_t pid) {
        constexpr int S = decltype(stc)::value;
        const bool inr = pg + wb < pg_end;
        const uint64_t pb = (uint64_t)pid * page_bytes;
        uint32_t off = doff;
        if ((pg + PT) * kPage > it.kv_end) off = inr && pg * kPage + dk < it.kv_end ? doff : doff0;
        lds_dma16_sbase(kbase + pb, off, lds_ring + S * SB);
        lds_dma16_sbase(vbase + pb, off, lds_ring + S * SB + 2 * TH);
    };
    // The first two tiles from the ids in the item (pages pg_begin .. +3,
    // the last repeated past the item's end).
    // (selected, not indexed: a runtime index would put the item in memory)
    const uint32_t fp0 = wb ? it.first_pages[1] : it.first_pages[0];
    const uint32_t fp1 = PT == 1 ? it.first_pages[1] : (wb ? it.first_pages[3] : it.first_pages[2]);
    if (n_tiles > 0) issue_pid(RingStage<0>{}, pg_begin, fp0);
    if (n_tiles > 1) issue_pid(RingStage<1>{}, pg_begin + PT, fp1);
    // q rows and 64 page ids (from the item's first page) while those land.
    float4 xq[2 * QC];
    {
        // (a lane without a query reads the item's first row: rows past nq
        // may lie past the end of the caller's q)
        const float* qb = a.q + (int64_t)lay * a.q_layer_stride +
                          (int64_t)(it.row0 + (qok ? r0 + col : 0)) * a.q_row_stride + head * D + 8 * rg;
#pragma unroll
        for (int c = 0; c < QC; c++) {
            xq[2 * c] = reinterpret_cast<const float4*>(qb + c * 32)[0];
            xq[2 * c + 1] = reinterpret_cast<const float4*>(qb + c * 32)[1];
        }
    }
    uint32_t id_base = pg_begin;
    uint32_t ids = tab[min(id_base + (uint32_t)lane, pg_end - 1)];
    // The loads have landed before any DMA is issued after them (the loop's
    // waits count DMA loads only); waiting here also covers the first tiles,
    // issued before them.
#pragma unroll
    for (int c = 0; c < 2 * QC; c++) asm volatile("" : : "v"(xq[c].x), "v"(xq[c].y), "v"(xq[c].z), "v"(xq[c].w));
    asm volatile("" : : "v"(ids));
    auto issue = [&](auto stc, uint32_t pg) {
        const uint32_t idx = pg + wb;
        const uint32_t want = idx < pg_end ? idx : pg;
        if (want >= id_base + 64) {  // past the window of page ids (items over 64 pages)
            id_base = pg;
            ids = tab[min(id_base + (uint32_t)lane, pg_end - 1)];
            asm volatile("" : : "v"(ids));
        }
        issue_pid(stc, pg, __builtin_amdgcn_readlane(ids, want - id_base));
    };

    // Q^T as the B operand: query col, dims c*32 + 8*rg .. +7, f16 hi + lo
    // (lo = f16(q - hi) unscaled: the matrix cores take its subnormals
    // exactly, so both halves accumulate into one product).
    half8_t qh[QC], ql[QC];
#pragma unroll
    for (int c = 0; c < QC; c++) {
        const float x[8] = {xq[2 * c].x, xq[2 * c].y, xq[2 * c].z, xq[2 * c].w,
                            xq[2 * c + 1].x, xq[2 * c + 1].y, xq[2 * c + 1].z, xq[2 * c + 1].w};
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
            float x0 = qok ? x[e] * a.qscale : 0.f, x1 = qok ? x[e + 1] * a.qscale : 0.f;
            asm("" : "+v"(x0), "+v"(x1));  // the f32 products, as the split's residual sees them
            uint32_t h, l;
            split_w16x2(x0, x1, h, l);
            const half2_t hh = __builtin_bit_cast(half2_t, h), ll = __builtin_bit_cast(half2_t, l);
            qh[c][e] = hh[0];
            qh[c][e + 1] = hh[1];
            ql[c][e] = ll[0];
            ql[c][e + 1] = ll[1];
        }
    }
    // Weights are exp2(s - mref): mref = m - kLog2PScalePre for the running
    // reference m, so p enters PV scaled by 2^7 (at most 2^15).  The scores
    // come out of QK as s - mref (the product's accumulator starts at -mref).
    float mref = 0.f;
    float4_t negref = {0.f, 0.f, 0.f, 0.f};
    float4_t o[VC];  // PV products of p's hi and lo parts, into one accumulator
#pragma unroll
    for (int c = 0; c < VC; c++) o[c] = float4_t{0.f, 0.f, 0.f, 0.f};
    float4_t lacc = {0.f, 0.f, 0.f, 0.f};  // sum of weights (every lane of a query column)
    const half8_t ones8 = {1, 1, 1, 1, 1, 1, 1, 1};
    const half4_t ones4 = {1, 1, 1, 1};
    // Per-lane LDS offsets (bytes in a stage): K operand chunk 4c + rg of row
    // col of page 0 (page b: + b * kPage * CH chunks, the same swizzle), V^T
    // operand of the transposing read (ds_read_b64_tr_b16: within 16 lanes,
    // lane 4t+a reads dims c*16 + 4a .. +3 of key 4*rg + t).
    uint32_t koff[QC], voff[VC];
    const int vt_t = (lane >> 2) & 3, vt_a = lane & 3;
#pragma unroll
    for (int c = 0; c < QC; c++) koff[c] = tile_chunk<CH>(col, 4 * c + rg) * 16;
#pragma unroll
    for (int c = 0; c < VC; c++)
        voff[c] = 2 * TH + tile_chunk<CH>(4 * rg + vt_t, 2 * c + (vt_a >> 1)) * 16 + (vt_a & 1) * 8;

    auto tile = [&](auto stc, uint32_t ti) {
        constexpr int S = decltype(stc)::value;
        const uint32_t pg = pg_begin + ti * PT;
        // This wave's part of tile ti has landed (vmcnt is in order: only
        // the two loads of each later tile already issued may still be
        // outstanding); after the barrier every wave's part has, and every
        // wave is done with tile ti-1, whose stage the next tile takes.
        wait_tiles<2>(min(n_tiles - 1 - ti, (uint32_t)(NS - 2)));
        __syncthreads();
        if (ti + NS - 1 < n_tiles) issue(RingStage<(S + NS - 1) % NS>{}, pg + (NS - 1) * PT);
        if (pg * kPage >= kend_w) return;  // wave-uniform: no key of the tile for this wave
        const uint8_t* const st_base = &ring[S][0];
        const uint32_t nb = min((uint32_t)PT, (kend_w - pg * kPage + kPage - 1) / kPage);
        float sc[PT][4];
#pragma unroll
        for (int b = 0; b < PT; b++) {
            half8_t kh[QC];
#pragma unroll
            for (int c = 0; c < QC; c++)
                kh[c] = *reinterpret_cast<const half8_t*>(st_base + koff[c] + b * kPage * CH * 16);
            float4_t acc = negref;
#pragma unroll
            for (int c = 0; c < QC; c++) acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh[c], qh[c], acc, 0, 0, 0);
#pragma unroll
            for (int c = 0; c < QC; c++) acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh[c], ql[c], acc, 0, 0, 0);
#pragma unroll
            for (int j = 0; j < 4; j++) sc[b][j] = acc[j];
        }
        if ((pg + PT) * kPage > kfull_w) {  // some key is hidden from some query of the wave
#pragma unroll
            for (int b = 0; b < PT; b++)
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const uint32_t key = (pg + b) * kPage + 4 * rg + j;
                    const bool ok = qok && b < (int)nb && key < it.kv_end && key <= qpos;
                    sc[b][j] = ok ? sc[b][j] : -INFINITY;
                }
        }
        float lm = sc[0][0];
#pragma unroll
        for (int b = 0; b < PT; b++)
#pragma unroll
            for (int j = 0; j < 4; j++) lm = fmaxf(lm, sc[b][j]);
        if (ti == 0 || __any(lm > kHi)) {
            // Column max relative to the reference; the first tile moves the
            // reference to it, later ones only up, and only past the slack.
            const float mx = rows4_max(lm) - kLog2PScalePre;
            // (a column with no visible key keeps a finite reference)
            const float d = fmaxf(ti == 0 ? mx : fmaxf(mx, 0.f), -65536.f);
            if (ti != 0) {
                const float alpha = fast_exp2(-d);
                lacc *= alpha;
#pragma unroll
                for (int c = 0; c < VC; c++) o[c] *= alpha;
            }
            mref += d;
            negref = float4_t{-mref, -mref, -mref, -mref};
#pragma unroll
            for (int b = 0; b < PT; b++)
#pragma unroll
                for (int j = 0; j < 4; j++) sc[b][j] -= d;
        }
        half4_t ph[PT], pl[PT];
#pragma unroll
        for (int b = 0; b < PT; b++) {
            float p[4];
#pragma unroll
            for (int j = 0; j < 4; j++) p[j] = fast_exp2(sc[b][j]);
            uint32_t h0, l0, h1, l1;
            split_w16x2(p[0], p[1], h0, l0);
            split_w16x2(p[2], p[3], h1, l1);
            ph[b] = __builtin_bit_cast(half4_t, u32x2_t{h0, h1});
            pl[b] = __builtin_bit_cast(half4_t, u32x2_t{l0, l1});
        }
        // O^T += V^T P^T, 16 dims per product; pages in pairs through the
        // 32-key product (k-slot 8*rg + 4*i + j of the pair is key 4*rg + j
        // of its page i, in both operands).
        auto vread = [&](int b, int c) {
            const v4fp16_t r = __builtin_amdgcn_ds_read_tr16_b64_v4f16(
                (__attribute__((address_space(3))) v4fp16_t*)(st_base + voff[c] + b * kPage * CH * 16));
            return __builtin_bit_cast(half4_t, r);
        };
        if constexpr (PT % 2 == 0) {
#pragma unroll
            for (int b = 0; b < PT; b += 2) {
                if (b >= (int)nb) break;  // a page past nb has p = 0 and finite V
                const half8_t p8h = __builtin_shufflevector(ph[b], ph[b + 1], 0, 1, 2, 3, 4, 5, 6, 7);
                const half8_t p8l = __builtin_shufflevector(pl[b], pl[b + 1], 0, 1, 2, 3, 4, 5, 6, 7);
#pragma unroll
                for (int c = 0; c < VC; c++) {
                    const half8_t v8 = __builtin_shufflevector(vread(b, c), vread(b + 1, c), 0, 1, 2, 3, 4, 5, 6, 7);
                    o[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(v8, p8h, o[c], 0, 0, 0);
                    o[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(v8, p8l, o[c], 0, 0, 0);
                }
                lacc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ones8, p8h, lacc, 0, 0, 0);
                lacc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ones8, p8l, lacc, 0, 0, 0);
            }
        } else {
#pragma unroll
            for (int b = 0; b < PT; b++) {
                if (b >= (int)nb) break;
#pragma unroll
                for (int c = 0; c < VC; c++) {
                    const half4_t v4 = vread(b, c);
                    o[c] = __builtin_amdgcn_mfma_f32_16x16x16f16(v4, ph[b], o[c], 0, 0, 0);
                    o[c] = __builtin_amdgcn_mfma_f32_16x16x16f16(v4, pl[b], o[c], 0, 0, 0);
                }
                lacc = __builtin_amdgcn_mfma_f32_16x16x16f16(ones4, ph[b], lacc, 0, 0, 0);
                lacc = __builtin_amdgcn_mfma_f32_16x16x16f16(ones4, pl[b], lacc, 0, 0, 0);
            }
        }
    };
    for (uint32_t ti = 0; ti < n_tiles;) {
        tile(RingStage<0>{}, ti);
        if (++ti == n_tiles) break;
        tile(RingStage<1>{}, ti);
        if (++ti == n_tiles) break;
        tile(RingStage<2>{}, ti);
        ++ti;
    }
    static_assert(kPrefillStages == 3, "the loop body is instantiated per ring stage");

    if (!qok) return;
    const float lsum = lacc[0];
    const uint32_t row = it.row0 + r0 + col;
    if (it.part_slot == kNoSlot) {
        float* dst = a.out + (int64_t)lay * a.out_layer_stride + (int64_t)row * a.out_row_stride + head * D;
        const float scale = 1.f / lsum;  // lsum and o both carry the 2^7
#pragma unroll
        for (int c = 0; c < VC; c++) {
            float4 y;
            y.x = o[c][0] * scale;
            y.y = o[c][1] * scale;
            y.z = o[c][2] * scale;
            y.w = o[c][3] * scale;
            *reinterpret_cast<float4*>(dst + c * 16 + 4 * rg) = y;
        }
    } else {
        // (m, l, o) with l and o in units of exp2(s - m), m = mref + 2^7's
        // exponent; a row with no key of the partition weighs nothing.
        float* p = a.partials + ((((uint64_t)it.part_slot * a.n_lay + lay) * a.pool.n_head + head) * kPrefillRows + r0 + col) * (D + 2);
        if (rg == 0) {
            p[0] = lsum > 0.f ? mref + kLog2PScalePre : kMinScore;
            p[1] = lsum * kPUnscalePre;
        }
#pragma unroll
        for (int c = 0; c < VC; c++)
#pragma unroll
            for (int j = 0; j < 4; j++) p[2 + c * 16 + 4 * rg + j] = o[c][j] * kPUnscalePre;
    }
}

// One workgroup per (merge item, layer, head).  Thread t owns output unit
// u = (row, dim) of the group and partitions j, j+G, j+2G, ... where G =
// kMergeThreads / (rows * D) groups of threads split the partitions; each
// keeps a running log-sum-exp state (m, l, o) over its partitions, whose
// loads do not depend on earlier arithmetic, so they stream back to back
// (batch.metal:403-424 merges the same (m, l, o) partials).  The G states of
// a unit are combined through LDS.  A partition where a row has no key holds
// m = kMinScore, l = 0, o = 0 and weighs nothing.  (kMergeThreads: kv_plan.h.)

template <int D, int NQ, int INL>
__global__ __launch_bounds__(kMergeThreads) void attn_merge_kernel(const AttnLaunch a, const PlanArg<INL> pa) {
    constexpr uint32_t T = kMergeThreads;
    __shared__ float sm[T], sl[T], so[T];
    const uint32_t H = a.pool.n_head;
    const uint32_t lh = a.n_lay * H;
    // merge_split_of(item) workgroups share a (merge item, layer, head) (the
    // launch has a.merge_split, the largest, per unit; the rest return):
    // workgroup ms takes units ms*U .. ms*U+U-1 of its nq * D (U = nq * D /
    // split), so more groups of threads split the partitions.
    const uint32_t stride = a.merge_split ? a.merge_split : 1;
    const uint32_t bid = blockIdx.x / stride, ms = blockIdx.x - bid * stride;
    const uint32_t mi = bid / lh;
    const uint32_t rem = bid - mi * lh;
    const uint32_t lay = rem / H;
    const uint32_t head = rem - lay * H;
    const MergeItem g = reinterpret_cast<const MergeItem*>(plan_base(pa, a.plan) + a.off_merges)[mi];
    const uint32_t split = merge_split_of(g.n_parts, g.nq, D);
    if (ms >= split) return;
    const uint64_t slot_stride = (uint64_t)a.n_lay * H * NQ * (D + 2);
    const float* base = a.partials + (((uint64_t)g.slot0 * a.n_lay + lay) * H + head) * NQ * (D + 2);
    const uint32_t units = g.nq * D / split, ub = ms * units;
    const uint32_t G = units >= T ? 1u : T / units;
    const uint32_t t = threadIdx.x;
    for (uint32_t u0 = 0; u0 < units; u0 += T) {  // several passes only when G == 1
        const uint32_t j = G > 1 ? t / units : 0u;
        const uint32_t u = ub + (G > 1 ? t - j * units : u0 + t);
        const bool active = j < G && u < ub + units;
        const uint32_t r = u / D, d = u - r * D;
        float m = kMinScore, l = 0.f, o = 0.f;
        if (active) {
            const float* p = base + r * (D + 2);
#pragma unroll 4
            for (uint32_t s = j; s < g.n_parts; s += G) {
                const float* ps = p + s * slot_stride;
                const float ms = ps[0], ls = ps[1], os = ps[2 + d];
                const float mn = fmaxf(m, ms);
                const float a1 = fast_exp2(m - mn), a2 = fast_exp2(ms - mn);
                l = l * a1 + ls * a2;
                o = o * a1 + os * a2;
                m = mn;
            }
        }
        float* dst = a.out + (int64_t)lay * a.out_layer_stride + (int64_t)(g.row0 + r) * a.out_row_stride + head * D + d;
        if (G == 1) {
            if (active) *dst = o / l;
            continue;
        }
        sm[t] = m;
        sl[t] = l;
        so[t] = o;
        __syncthreads();
        if (t < units) {  // (j = 0: dst is unit ub + t's)
            float M = sm[t];
            for (uint32_t k = 1; k < G; k++) M = fmaxf(M, sm[k * units + t]);
            float L = 0.f, O = 0.f;
            for (uint32_t k = 0; k < G; k++) {
                const float w = fast_exp2(sm[k * units + t] - M);
                L += sl[k * units + t] * w;
                O += so[k * units + t] * w;
            }
            *dst = O / L;
        }
    }
}

// Pages per wave iteration of the matrix-core kernel (two, with the pair's
// PV through the 32-key product, 154 registers and 3 waves per SIMD: config 5
// -0.9%, Q8 -3.3%).
constexpr int kMfmaPages = 1;

// One kernel launch; with timing events the dispatch packet itself records
// the kernel's start and end (no separate event commands in the stream).
template <typename K, typename... Args>
hipError_t go(K kern, uint64_t blocks, uint32_t threads, hipStream_t s, const LaunchTiming& t, const Args&... args) {
    hipExtLaunchKernelGGL(kern, dim3((uint32_t)blocks), dim3(threads), 0, s, t.start, t.stop, 0, args...);
    return hipGetLastError();
}

// Launch `kern<INL>` with the plan inline (kInlinePlanTiny, kInlinePlanSmall
// or kInlinePlanBytes of arguments, the smallest that holds it) or through the
// device pointer in the launch struct.
template <typename L, typename Fn>
hipError_t with_plan(const L& a, const void* inline_plan, uint32_t inline_bytes, Fn&& launch) {
    if (inline_plan) {
        if (inline_bytes > kInlinePlanBytes) return hipErrorInvalidValue;
        if (inline_bytes <= kInlinePlanTiny) {
            PlanArg<kInlinePlanTiny> pa;
            memcpy(pa.b, inline_plan, inline_bytes);
            return launch(pa);
        }
        if (inline_bytes <= kInlinePlanSmall) {
            PlanArg<kInlinePlanSmall> pa;
            memcpy(pa.b, inline_plan, inline_bytes);
            return launch(pa);
        }
        PlanArg<kInlinePlanBytes> pa;
        memcpy(pa.b, inline_plan, inline_bytes);
        return launch(pa);
    }
    return launch(PlanArg<0>{});
}


template <int D, int NQ>
hipError_t attn_launch_t(const AttnLaunch& a, const void* ip, uint32_t ib, hipStream_t s, const LaunchTiming& t) {
    constexpr int PB = D == 128 ? kPagesD128 : kPagesPerIter;
    static_assert(NQ == 1, "groups of several rows run on the matrix cores");
    const uint64_t blocks = (uint64_t)a.n_items * a.n_lay * a.pool.n_head + a.n_orphan_blocks;
    if (blocks == 0) return hipSuccess;
    if constexpr (D == 64 && NQ == 1) {
        if (a.wide) {
            constexpr int WW = kWideWaves;
            constexpr int WPB = kWidePages;
            return with_plan(a, ip, ib, [&](auto pa) {
                constexpr int INL = sizeof(pa.b) > 4 ? (int)sizeof(pa.b) : 0;
                if (a.napp_total || a.n_orphan_blocks)
                    return go(attn_split_kernel<D, NQ, WW, WPB, true, INL>, blocks, 64 * WW, s, t, a, pa);
                return go(attn_split_kernel<D, NQ, WW, WPB, false, INL>, blocks, 64 * WW, s, t, a, pa);
            });
        }
    }
    if (a.wide) return hipErrorInvalidValue;
    return with_plan(a, ip, ib, [&](auto pa) {
        constexpr int INL = sizeof(pa.b) > 4 ? (int)sizeof(pa.b) : 0;
        if (a.napp_total || a.n_orphan_blocks)
            return go(attn_split_kernel<D, NQ, kWaves, PB, true, INL>, blocks, 64 * kWaves, s, t, a, pa);
        return go(attn_split_kernel<D, NQ, kWaves, PB, false, INL>, blocks, 64 * kWaves, s, t, a, pa);
    });
}

template <int D, int NQ>
hipError_t merge_launch_t(const AttnLaunch& a, const void* ip, uint32_t ib, hipStream_t s, const LaunchTiming& t) {
    const uint64_t blocks = (uint64_t)a.n_merges * a.n_lay * a.pool.n_head * (a.merge_split ? a.merge_split : 1);
    if (blocks == 0) return hipSuccess;
    return with_plan(a, ip, ib, [&](auto pa) {
        constexpr int INL = sizeof(pa.b) > 4 ? (int)sizeof(pa.b) : 0;
        return go(attn_merge_kernel<D, NQ, INL>, blocks, kMergeThreads, s, t, a, pa);
    });
}

template <int D, bool Q8>
hipError_t mfma_launch_t(const AttnLaunch& a, const void* ip, uint32_t ib, hipStream_t s, const LaunchTiming& t) {
    const uint64_t blocks = (uint64_t)a.n_items * a.n_lay * a.pool.n_head + a.n_orphan_blocks;
    if (blocks == 0) return hipSuccess;
    if constexpr (D == 64) {
        if (a.wide) {  // kWideWaves waves share each item's pages
            constexpr int WW = kWideWaves;
            return with_plan(a, ip, ib, [&](auto pa) {
                constexpr int INL = sizeof(pa.b) > 4 ? (int)sizeof(pa.b) : 0;
                if (a.napp_total || a.n_orphan_blocks)
                    return go(attn_mfma_kernel<D, WW, kMfmaPages, true, INL, Q8>, blocks, 64 * WW, s, t, a, pa);
                return go(attn_mfma_kernel<D, WW, kMfmaPages, false, INL, Q8>, blocks, 64 * WW, s, t, a, pa);
            });
        }
    }
    if (a.wide) return hipErrorInvalidValue;
    return with_plan(a, ip, ib, [&](auto pa) {
        constexpr int INL = sizeof(pa.b) > 4 ? (int)sizeof(pa.b) : 0;
        if (a.napp_total || a.n_orphan_blocks)
            return go(attn_mfma_kernel<D, kWaves, kMfmaPages, true, INL, Q8>, blocks, 64 * kWaves, s, t, a, pa);
        return go(attn_mfma_kernel<D, kWaves, kMfmaPages, false, INL, Q8>, blocks, 64 * kWaves, s, t, a, pa);
    });
}

template <int D>
hipError_t prefill_launch_t(const AttnLaunch& a, const void* ip, uint32_t ib, hipStream_t s, const LaunchTiming& t) {
    const uint64_t blocks = (uint64_t)(a.n_pseqs ? a.n_pseqs : a.n_items) * a.n_lay * a.pool.n_head;
    if (blocks == 0) return hipSuccess;
    return with_plan(a, ip, ib, [&](auto pa) {
        constexpr int INL = sizeof(pa.b) > 4 ? (int)sizeof(pa.b) : 0;
        // head_dim 128 stages one page per tile (two spill registers).
        constexpr int PT = D == 128 ? 1 : kPrefillPages;
        const bool seq = a.n_pseqs != 0;
        if constexpr (D == 64 && PT == 2) {
            if (a.pool.q8)
                return seq ? go(attn_prefill_q8_kernel<INL, true>, blocks, 256, s, t, a, pa)
                           : go(attn_prefill_q8_kernel<INL, false>, blocks, 256, s, t, a, pa);
        }
        if (a.pool.q8) return hipErrorInvalidValue;
        if (seq) return hipErrorInvalidValue;  // the host plans sequences on Q8 pools only
        if (a.ordered) {  // one block per unit of the host's order (uint16_t indices)
            if (blocks > 65536) return hipErrorInvalidValue;
            hipExtLaunchKernelGGL(attn_prefill_kernel<D, PT, INL>, dim3((uint32_t)blocks), dim3(256), 0, s, t.start,
                                  t.stop, 0, a, pa);
            return hipGetLastError();
        }
        if (a.n_items > 65535 || a.n_lay > 65535) return hipErrorInvalidValue;  // grid y and z
        hipExtLaunchKernelGGL(attn_prefill_kernel<D, PT, INL>, dim3(a.pool.n_head, a.n_lay, a.n_items), dim3(256),
                              0, s, t.start, t.stop, 0, a, pa);
        return hipGetLastError();
    });
}

template <int D>
hipError_t q8_launch_t(const AttnLaunch& a, const void* ip, uint32_t ib, hipStream_t s, const LaunchTiming& t) {
    const uint64_t blocks = (uint64_t)a.n_items * a.n_lay * a.pool.n_head + a.n_orphan_blocks;
    if (blocks == 0) return hipSuccess;
    if constexpr (D == 64) {
        if (a.wide) {
            constexpr int WW = kWideWavesQ8;
            return with_plan(a, ip, ib, [&](auto pa) {
                constexpr int INL = sizeof(pa.b) > 4 ? (int)sizeof(pa.b) : 0;
                constexpr int PB = kQ8Pages;
                if (a.napp_total || a.n_orphan_blocks)
                    return go(attn_q8_kernel<D, WW, PB, true, INL>, blocks, 64 * WW, s, t, a, pa);
                return go(attn_q8_kernel<D, WW, PB, false, INL>, blocks, 64 * WW, s, t, a, pa);
            });
        }
    }
    if (a.wide) return hipErrorInvalidValue;
    return with_plan(a, ip, ib, [&](auto pa) {
        constexpr int INL = sizeof(pa.b) > 4 ? (int)sizeof(pa.b) : 0;
        constexpr int PB = kQ8Pages;
        if (a.napp_total || a.n_orphan_blocks)
            return go(attn_q8_kernel<D, kWaves, PB, true, INL>, blocks, 64 * kWaves, s, t, a, pa);
        return go(attn_q8_kernel<D, kWaves, PB, false, INL>, blocks, 64 * kWaves, s, t, a, pa);
    });
}

template <int D>
hipError_t attn_dispatch_nq(const AttnLaunch& a, const void* ip, uint32_t ib, hipStream_t s, bool merge,
                            const LaunchTiming& t) {
    if (a.nq_tile == kPrefillRows) {  // prefill groups (Q8 pools: head_dim 64 only)
        return merge ? merge_launch_t<D, kPrefillRows>(a, ip, ib, s, t) : prefill_launch_t<D>(a, ip, ib, s, t);
    }
    if (a.pool.q8) {  // single rows on the vector kernel, groups on the matrix cores
        if (a.nq_tile == kMfmaTile)
            return merge ? merge_launch_t<D, kMfmaTile>(a, ip, ib, s, t) : mfma_launch_t<D, true>(a, ip, ib, s, t);
        if (a.nq_tile != 1) return hipErrorInvalidValue;
        return merge ? merge_launch_t<D, 1>(a, ip, ib, s, t) : q8_launch_t<D>(a, ip, ib, s, t);
    }
    // Groups of several rows always take the 16-row matrix tile.
    if (a.nq_tile == kMfmaTile)
        return merge ? merge_launch_t<D, kMfmaTile>(a, ip, ib, s, t) : mfma_launch_t<D, false>(a, ip, ib, s, t);
    if (a.nq_tile != 1) return hipErrorInvalidValue;
    return merge ? merge_launch_t<D, 1>(a, ip, ib, s, t) : attn_launch_t<D, 1>(a, ip, ib, s, t);
}

hipError_t attn_dispatch(const AttnLaunch& a, const void* ip, uint32_t ib, hipStream_t s, bool merge,
                          const LaunchTiming& t) {
    switch (a.pool.head_dim) {
        case 64: return attn_dispatch_nq<64>(a, ip, ib, s, merge, t);
        case 128: return attn_dispatch_nq<128>(a, ip, ib, s, merge, t);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace

bool attention_supported(uint32_t head_dim) { return head_dim == 64 || head_dim == 128; }

// Split-K partials of ni_kv_step_noalloc's launches: a file-scope device
// array, so that entry point calls no allocator.  Each GPU the library runs
// on holds its own copy until the process ends; every such call on a GPU
// shares it (calls that overlap on one GPU race).  Nothing in it needs to
// start at zero: a merge reads only the partials its own call's attention
// launch wrote first, on the same stream.
static __device__ __align__(256) float scratch[kScratchBytes / sizeof(float)];

hipError_t scratch_address(void** out) {
    // In host code `scratch` names a host-side stand-in, not device memory:
    // only the address hipGetSymbolAddress returns for the current device
    // may reach a kernel or a copy.
    static std::mutex mu;
    static std::vector<void*> per_device;
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    std::lock_guard<std::mutex> lock(mu);
    if ((size_t)dev >= per_device.size()) per_device.resize((size_t)dev + 1, nullptr);
    if (!per_device[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        per_device[dev] = p;
    }
    *out = per_device[dev];
    return hipSuccess;
}

hipError_t launch_append(const AppendLaunch& a, const void* ip, uint32_t ib, hipStream_t s, const LaunchTiming& t) {
    const uint64_t threads = (uint64_t)a.n_lay * a.n_rows * 2 * ((a.pool.n_head * a.pool.head_dim) >> 3);
    if (threads == 0) return hipSuccess;
    return with_plan(a, ip, ib, [&](auto pa) {
        constexpr int INL = sizeof(pa.b) > 4 ? (int)sizeof(pa.b) : 0;
        return go(kv_append_kernel<INL>, (threads + 255) / 256, 256, s, t, a, pa);
    });
}

// Compute units of the current device (a round of a grid), looked up once
// per device; 256 (MI355X) if the query fails.
uint32_t device_cus() {
    static std::mutex mu;
    static std::vector<uint32_t> per_device;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0) return 256;
    std::lock_guard<std::mutex> lock(mu);
    if ((size_t)dev >= per_device.size()) per_device.resize((size_t)dev + 1, 0);
    if (!per_device[dev]) {
        int n = 0;
        per_device[dev] =
            hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0 ? n : 256;
    }
    return per_device[dev];
}

// Workgroups of `threads` threads of kernel f that one CU of the current
// device holds at once, looked up once per (device, kernel); 0 if unknown.
static uint32_t blocks_per_cu(const void* f, int threads) {
    static std::mutex mu;
    static std::vector<std::pair<std::pair<int, const void*>, uint32_t>> cache;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 0;
    std::lock_guard<std::mutex> lock(mu);
    for (const auto& c : cache)
        if (c.first.first == dev && c.first.second == f) return c.second;
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, f, threads, 0) != hipSuccess || n < 0) n = 0;
    cache.push_back({{dev, f}, (uint32_t)n});
    return (uint32_t)n;
}

uint32_t wide_blocks_per_cu(uint32_t head_dim, bool q8, uint32_t nq_tile, bool fused) {
    if (head_dim != 64) return 0;
    // the kernel attn_dispatch picks for a wide launch with these parameters
    const void* f = nullptr;
    int threads = 0;
    constexpr int INL = (int)kInlinePlanSmall;
    if (nq_tile == kMfmaTile) {
        threads = 64 * kWideWaves;
        f = q8 ? (fused ? (const void*)attn_mfma_kernel<64, kWideWaves, kMfmaPages, true, INL, true>
                        : (const void*)attn_mfma_kernel<64, kWideWaves, kMfmaPages, false, INL, true>)
               : (fused ? (const void*)attn_mfma_kernel<64, kWideWaves, kMfmaPages, true, INL, false>
                        : (const void*)attn_mfma_kernel<64, kWideWaves, kMfmaPages, false, INL, false>);
    } else if (nq_tile == 1 && q8) {
        threads = 64 * kWideWavesQ8;
        f = fused ? (const void*)attn_q8_kernel<64, kWideWavesQ8, kQ8Pages, true, INL>
                  : (const void*)attn_q8_kernel<64, kWideWavesQ8, kQ8Pages, false, INL>;
    } else if (nq_tile == 1) {
        threads = 64 * kWideWaves;
        f = fused ? (const void*)attn_split_kernel<64, 1, kWideWaves, kWidePages, true, INL>
                  : (const void*)attn_split_kernel<64, 1, kWideWaves, kWidePages, false, INL>;
    } else {
        return 0;
    }
    return blocks_per_cu(f, threads);
}

uint32_t prefill_blocks_per_cu(uint32_t head_dim) {
    constexpr int INL = (int)kInlinePlanSmall;
    if (head_dim == 64) return blocks_per_cu((const void*)attn_prefill_kernel<64, kPrefillPages, INL>, 256);
    if (head_dim == 128) return blocks_per_cu((const void*)attn_prefill_kernel<128, 1, INL>, 256);
    return 0;
}

template <int WF>
hipError_t launch_qkv_t(const QkvLaunch& a, const void* ip, uint32_t ib, hipStream_t s, const LaunchTiming& t) {
    if (a.n_rows <= kQkvSmallRows) {
        constexpr int RB = kQkvSmallRb;
        const dim3 grid((a.n_rows + 16 * RB - 1) / (16 * RB), a.n_feat / 16);
        return with_plan(a, ip, ib, [&](auto pa) {
            constexpr int INL = sizeof(pa.b) > 4 ? (int)sizeof(pa.b) : 0;
            hipExtLaunchKernelGGL(qkv_small_kernel<RB, INL, WF>, grid, dim3(64 * kQkvParts), 0, s, t.start, t.stop, 0,
                                  a, pa);
            return hipGetLastError();
        });
    }
    if (a.n_rows <= kQkvMidRows && a.d_in <= (uint32_t)(kQkvMidChunks * kQkvChunk)) {
        const dim3 grid((a.n_rows + 15) / 16 * (a.n_feat / 16));  // (row tile, feature tile), dealt by XCD
        return with_plan(a, ip, ib, [&](auto pa) {
            constexpr int INL = sizeof(pa.b) > 4 ? (int)sizeof(pa.b) : 0;
            // Registers for as many chunks as d_in has: 6 up to 768 (GPT-2), else 8.
            if (a.d_in <= 6u * kQkvChunk)
                hipExtLaunchKernelGGL(qkv_mid_kernel<INL, WF, 6>, grid, dim3(64 * kQkvParts), 0, s, t.start, t.stop,
                                      0, a, pa);
            else
                hipExtLaunchKernelGGL(qkv_mid_kernel<INL, WF, kQkvMidChunks>, grid, dim3(64 * kQkvParts), 0, s,
                                      t.start, t.stop, 0, a, pa);
            return hipGetLastError();
        });
    }
    // 16-feature tiles: the most workgroups to stream W with (64-feature tiles
    // measured slower from 64 to 512 rows).  Large batches take 48-feature
    // tiles (x read by a third as many workgroups; 48 KB of LDS, 3 per CU)
    // when that grid fills whole rounds of the GPU or spans two or more:
    // 12 layers of GPT-2, 512 rows 327 -> 281 us, 1024 556 -> 502, 2048
    // 1053 -> 955, while partial rounds lose (384 rows 284 against 293, 640
    // 376 against 387).  Both issue the same products in the same order.
    const uint32_t row_tiles = (a.n_rows + kQkvTileRows - 1) / kQkvTileRows;
    if (a.n_feat % 48 == 0) {
        const uint64_t wg = (uint64_t)row_tiles * (a.n_feat / 48), round = 3ull * device_cus();
        if (wg >= 2 * round || (wg >= round && wg % round == 0)) {
            return with_plan(a, ip, ib, [&](auto pa) {
                constexpr int INL = sizeof(pa.b) > 4 ? (int)sizeof(pa.b) : 0;
                hipExtLaunchKernelGGL(qkv_kernel<3, INL, WF>, dim3(row_tiles, a.n_feat / 48), dim3(256), 0, s,
                                      t.start, t.stop, 0, a, pa);
                return hipGetLastError();
            });
        }
    }
    const dim3 grid(row_tiles, a.n_feat / kQkvTileFeat);
    return with_plan(a, ip, ib, [&](auto pa) {
        constexpr int INL = sizeof(pa.b) > 4 ? (int)sizeof(pa.b) : 0;
        hipExtLaunchKernelGGL(qkv_kernel<kQkvTileFeat / 16, INL, WF>, grid, dim3(256), 0, s, t.start, t.stop, 0, a,
                              pa);
        return hipGetLastError();
    });
}

hipError_t launch_qkv(const QkvLaunch& a, const void* ip, uint32_t ib, hipStream_t s, const LaunchTiming& t) {
    if (a.n_rows == 0) return hipSuccess;
    switch (a.wfmt) {
        case kWF32: return launch_qkv_t<kWF32>(a, ip, ib, s, t);
        case kWF16: return launch_qkv_t<kWF16>(a, ip, ib, s, t);
        case kWQ8: return launch_qkv_t<kWQ8>(a, ip, ib, s, t);
        case kWQ4: return launch_qkv_t<kWQ4>(a, ip, ib, s, t);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_gather_q8(const GatherQ8Launch& a, const void* ip, uint32_t ib, hipStream_t s) {
    const uint64_t threads = (uint64_t)a.n_lay * a.n_rows * 2 * a.pool.n_head;
    if (threads == 0) return hipSuccess;
    return with_plan(a, ip, ib, [&](auto pa) {
        constexpr int INL = sizeof(pa.b) > 4 ? (int)sizeof(pa.b) : 0;
        hipLaunchKernelGGL(kv_gather_q8_kernel<INL>, dim3((uint32_t)((threads + 255) / 256)), dim3(256), 0, s, a, pa);
        return hipGetLastError();
    });
}

hipError_t launch_gather(const GatherLaunch& a, const void* ip, uint32_t ib, hipStream_t s) {
    const uint64_t threads = (uint64_t)a.n_lay * a.n_rows * 2 * ((a.pool.n_head * a.pool.head_dim) >> 3);
    if (threads == 0) return hipSuccess;
    return with_plan(a, ip, ib, [&](auto pa) {
        constexpr int INL = sizeof(pa.b) > 4 ? (int)sizeof(pa.b) : 0;
        hipLaunchKernelGGL(kv_gather_kernel<INL>, dim3((uint32_t)((threads + 255) / 256)), dim3(256), 0, s, a, pa);
        return hipGetLastError();
    });
}

hipError_t launch_attention(const AttnLaunch& a, const void* ip, uint32_t ib, hipStream_t s, const LaunchTiming& t) {
    return attn_dispatch(a, ip, ib, s, false, t);
}

uint32_t orphan_blocks(const AttnLaunch& a) {
    const uint64_t threads = (uint64_t)a.n_lay * a.n_orphans * 2 * ((a.pool.n_head * a.pool.head_dim) >> 3);
    // Threads per workgroup of the launch the orphan blocks join.
    const bool q8_rows = a.pool.q8 && a.nq_tile == 1;
    const uint64_t per_block = 64ull * (a.wide ? (q8_rows ? kWideWavesQ8 : kWideWaves) : kWaves);
    return (uint32_t)((threads + per_block - 1) / per_block);
}

hipError_t launch_merge(const AttnLaunch& a, const void* ip, uint32_t ib, hipStream_t s, const LaunchTiming& t) {
    return attn_dispatch(a, ip, ib, s, true, t);
}

hipError_t launch_stream(bool copy, bool span, const void* src, void* dst, size_t bytes, uint32_t blocks,
                         hipStream_t s) {
    const uint64_t n16 = bytes / 16;
    if (n16 == 0 || blocks == 0) return hipSuccess;
    const auto* in = static_cast<const u32x4*>(src);
    auto* out = static_cast<u32x4*>(dst);
    const dim3 g(blocks), t(256);
    if (copy && span) hipLaunchKernelGGL((stream_kernel<true, true>), g, t, 0, s, in, out, n16);
    if (copy && !span) hipLaunchKernelGGL((stream_kernel<true, false>), g, t, 0, s, in, out, n16);
    if (!copy && span) hipLaunchKernelGGL((stream_kernel<false, true>), g, t, 0, s, in, out, n16);
    if (!copy && !span) hipLaunchKernelGGL((stream_kernel<false, false>), g, t, 0, s, in, out, n16);
    return hipGetLastError();
}

hipError_t launch_attention_rows(const RowsLaunch& a, hipStream_t s) {
    const uint64_t blocks = (uint64_t)a.n_q * a.n_head;
    if (blocks == 0) return hipSuccess;
    constexpr int W = 4;
    switch (a.head_dim) {
        case 64: hipLaunchKernelGGL((attn_rows_kernel<64, W>), dim3((uint32_t)blocks), dim3(64 * W), 0, s, a); break;
        case 128: hipLaunchKernelGGL((attn_rows_kernel<128, W>), dim3((uint32_t)blocks), dim3(64 * W), 0, s, a); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_f32_to_f16(const float* in, uint16_t* out, size_t n, hipStream_t s) {
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(f32_to_f16_kernel, dim3((uint32_t)((n + 255) / 256)), dim3(256), 0, s, in, out, n);
    return hipGetLastError();
}

}  // namespace ni
