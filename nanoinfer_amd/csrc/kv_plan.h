// kv_plan.h -- the per-call plan the host builds and the kernels read.
//
// Shared by the host side (kv_host.cpp) and the gfx950 kernels
// (kv_kernels.hip).  A data-path call turns its rows into a compact plan
// (append destinations, attention work items, merge items and the block-table
// segments those items read), uploads it with one async copy and launches the
// kernels over it.  The device never sees the host's full block tables.
#pragma once

#include <hip/hip_runtime_api.h>
#include <stddef.h>
#include <stdint.h>

namespace ni {

constexpr uint32_t kPage = 16;           // positions per page (batch.rs:33)
constexpr uint32_t kNoSlot = 0xffffffffu; // AttnItem::part_slot: the item is its group's only partition
// Groups of several queries run on matrix cores (tile of 16 query slots).
constexpr uint32_t kMfmaTile = 16;
// Prefill: groups of kMfmaTile+1 .. kPrefillRows consecutive query rows of one
// sequence run on attn_prefill_kernel, one 16-row tile per wave, every wave
// reading the same K/V tiles from LDS.
constexpr uint32_t kPrefillRows = 64;
// Waves per workgroup of a "wide" launch of single-row items: when a launch has
// too few (item, layer, head) units to fill the GPU, each item's pages are
// spread over this many waves of one workgroup (merged through LDS) instead of
// being split into partitions merged by a second kernel.  8 measured best (per
// layer, config 3: 2900 -> 3464 GB/s f16, 1697 -> 2167 Q8; 16 waves: 3078, 1594).
constexpr uint32_t kWideWaves = 8;
// The same for single rows on the Q8 cache (attn_q8_kernel), one layer per
// launch config 3: 5 waves 2634 GB/s, 6 2602, 8 2444.
constexpr uint32_t kWideWavesQ8 = 5;
constexpr uint32_t kMaxGroupRows = kMfmaTile;  // most query rows sharing one K/V stream

// Where one appended row goes: pool page `page`, position `slot` (0..15) in it.
struct AppendEntry {
    uint32_t src_row;  // row index in the k/v input (in a call's own append list, the entry's index)
    uint32_t page;
    uint32_t slot;
    uint32_t pad;
};

// One attention work item: the queries of one group (consecutive rows of one
// sequence at consecutive positions pos0 .. pos0+nq-1) over the keys of one
// partition [kv_begin, kv_end).  One workgroup runs it per (layer, head).
struct AttnItem {
    uint32_t tab;       // offset of this sequence's page list in the plan table
    uint32_t row0;      // q/out row of the first query
    uint32_t pos0;      // position of the first query; query r sees keys <= pos0 + r
    uint32_t nq;        // queries (1..kMaxGroupRows)
    uint32_t kv_begin;  // first key (multiple of 16)
    uint32_t kv_end;    // one past the last key: min(partition end, pos0 + nq)
    uint32_t part_slot; // partial-result slot, or kNoSlot (write out directly)
    union {
        struct {
            uint32_t app0;     // fused launches: first append entry of this step's new
            uint32_t napp;     //   rows inside [kv_begin, kv_end), and their count,
            uint32_t app_pos;  //   the position of the first of them
            uint32_t app_src;  //   and its k/v input row (the others follow consecutively)
        };
        // Prefill items on f16 pools (never appending): the page ids of pages
        // kv_begin/16 .. +3 (the last page repeated past the item's end), so
        // the first tiles' DMA needs no table read.
        uint32_t first_pages[4];
    };
    uint32_t pad;
};
static_assert(sizeof(AttnItem) == 48, "plan item layout");

// A sequence of a prompt-chunk step on a Q8 pool run by one prefill
// workgroup per (layer, head): its prefill items item0 .. item0 + n_items - 1
// in turn, each first appending, for the workgroup's head, the item's new
// rows (append entries app0 .. app0 + napp - 1 of the item).  (On f16 pools
// the same measured 1% slower, 16 x 512 prompts 470 against 465 us, so they
// take an append launch; Q8 511 against 533.)
struct PrefillSeq {
    uint32_t item0;
    uint32_t n_items;
};

// A group split into n_parts partitions, merged by log-sum-exp.
// Threads per merge workgroup.
constexpr int kMergeThreads = 512;
constexpr uint32_t kMergeSplitMax = 8;
// Workgroups that merge one (merge item, layer, head) of nq rows and n_parts
// partitions: enough that each thread merges at most 4 partitions (the loads
// of one unrolled batch).  A function of the item alone, so a row's merge
// (and its bits) does not depend on the rest of the call.
__host__ __device__ inline uint32_t merge_split_of(uint32_t n_parts, uint32_t nq, uint32_t D) {
    const uint32_t per = nq * D;
    const uint32_t G = per >= (uint32_t)kMergeThreads ? 1u : (uint32_t)kMergeThreads / per;
    uint32_t split = 1;
    while (split < kMergeSplitMax && n_parts > 4 * G * split) split *= 2;
    return split;
}

struct MergeItem {
    uint32_t row0;
    uint32_t nq;
    uint32_t slot0;   // partial slots slot0 .. slot0+n_parts-1
    uint32_t n_parts;
};

// Device pool geometry.  The (layer, page, head) block of K starts at
// k + layer*layer_halves + page*page_halves + head*head_halves and holds the
// page's 16 positions x head_dim halves contiguously; V likewise from v.
struct PoolGeom {
    uint16_t* k;
    uint16_t* v;
    uint64_t layer_halves;
    uint64_t page_halves;
    uint32_t head_halves;
    uint32_t n_head;
    uint32_t head_dim;
    // Q8 blocks (kv8.metal:15-48): [16][head_dim] int8, then 16 f32 scales
    // (amax / 127 per position) at byte 16 * head_dim.
    uint32_t q8;
};

struct AppendLaunch {
    PoolGeom pool;
    const float* k;
    const float* v;
    int64_t row_stride;
    int64_t layer_stride;
    const uint8_t* plan;         // device staging buffer (unused when inline)
    uint32_t off_entries;
    uint32_t n_rows;
    uint32_t layer0;
    uint32_t n_lay;
};

struct GatherLaunch {
    PoolGeom pool;
    uint16_t* k_out;
    uint16_t* v_out;
    int64_t row_stride;  // halves
    int64_t layer_stride;
    const uint8_t* plan;
    uint32_t off_entries;        // src_row = output row
    uint32_t n_rows;
    uint32_t layer0;
    uint32_t n_lay;
};

// Weight formats of the projection (the values of NI_W_* in nanoinfer_kv.h).
enum : uint32_t { kWF32 = 0, kWF16 = 1, kWQ8 = 2, kWQ4 = 3 };

// The QKV projection y = x W^T + b of n rows (W [n_feat][d_in] row-major, the
// reference's weight layout, n_feat = 3C, in one of its formats).  Fused: q
// columns to `out` ([n][C]), k/v columns as f16 to each row's page slot of
// `layer` (entries in the plan, src_row = x row).  Plain: every column to
// `out` ([n][3C]).
struct QkvLaunch {
    PoolGeom pool;
    const float* x;
    int64_t x_row_stride;
    const void* w;      // [n_feat][d_in] in format `wfmt`
    uint32_t wfmt;
    const float* bias;  // [n_feat] or null
    float* out;
    int64_t out_row_stride;
    const uint8_t* plan;
    uint32_t off_entries;
    uint32_t n_rows;
    uint32_t d_in;
    uint32_t n_feat;
    uint32_t layer;
    uint32_t fused;
};
constexpr uint32_t kQkvTileRows = 32, kQkvTileFeat = 16, kQkvK = 16;  // d_in must be a multiple of kQkvK

// Q8 gather: int8 K/V values [n_lay][n][C] and f32 scales [n_lay][n][n_head].
struct GatherQ8Launch {
    PoolGeom pool;
    int8_t* k_out;
    int8_t* v_out;
    float* k_scale;
    float* v_scale;
    const uint8_t* plan;
    uint32_t off_entries;  // src_row = output row
    uint32_t n_rows;
    uint32_t layer0;
    uint32_t n_lay;
};

struct AttnLaunch {
    PoolGeom pool;
    // Fused append (0 rows when the step's rows were appended beforehand):
    // item rows come from `app`, rows of sequences without queries from
    // `orphans`, handled by the n_orphan_blocks blocks after the items'.
    const float* k;
    const float* v;
    int64_t kv_row_stride;
    int64_t kv_layer_stride;
    uint32_t off_app;
    uint32_t off_orphans;
    uint32_t n_orphans;
    uint32_t n_orphan_blocks;
    uint32_t napp_total;  // rows the items append (0: not fused)
    const float* q;
    int64_t q_row_stride;
    int64_t q_layer_stride;
    float* out;
    int64_t out_row_stride;
    int64_t out_layer_stride;
    const uint8_t* plan;      // device staging buffer (unused when inline)
    uint32_t off_items;       // AttnItem[n_items], sorted longest first
    uint32_t off_table;       // uint32_t page ids the items index
    uint32_t off_merges;      // MergeItem[n_merges]
    float* partials;          // [slot][n_lay][n_head][nq_tile][head_dim + 2] (this launch's region)
    uint32_t n_items;
    uint32_t n_merges;
    uint32_t layer0;
    uint32_t n_lay;
    uint32_t nq_tile;         // query tile: 1..8 (vector kernel), kMfmaTile (matrix cores) or kPrefillRows
    float qscale;             // log2(e) / sqrt(head_dim)
    uint32_t wide;            // 1: kWideWaves waves per workgroup (single-row items, head_dim 64)
    uint32_t off_pseqs;       // prefill launch: PrefillSeq[n_pseqs]; 0 sequences: one workgroup per item
    uint32_t n_pseqs;
    uint32_t merge_split;     // merge launch: the largest merge_split_of over its items (0 = 1)
    // Wide one-layer launches: workgroup b runs (item, layer, head) unit
    // order[b] (uint16_t[n_items * n_lay * n_head] at off_order) instead of
    // unit b, so that each CU receives an even share of the work.
    uint32_t off_order;
    uint32_t ordered;
};

// A plan travels to the device either inside the kernel arguments (up to
// kInlinePlanBytes: the runtime copies arguments with the launch, so no
// separate transfer sits on the stream) or in a device staging buffer.
// Launch structs locate each part of the plan by its byte offset.  Inline
// plans go in the smallest argument block of kInlinePlanTiny,
// kInlinePlanSmall or kInlinePlanBytes bytes that holds them: a launch's
// host cost grows with the block (measured ~3.5 us at 256 B, ~4.1-4.7 us at
// 16 KB, ~6.0 us at 32 KB; back-to-back launches of an empty 768-workgroup
// kernel every 2.3 us at 1 KB, 2.9 at 2 KB, 3.3 at 4 KB, 4.1 at 8 KB, 3-6 at
// 16 KB), a per-layer call's plan (64 sequences) is 5-9 KB and a 64-row
// projection's 1 KB.
constexpr uint32_t kInlinePlanBytes = 32768, kInlinePlanSmall = 16384, kInlinePlanTiny = 2048;

// Device scratch of the no-allocation entry point (ni_kv_step_noalloc): the
// split-K partials of its launches, in a file-scope device array of this
// many bytes (kv_kernels.hip), one copy per GPU the library runs on.
constexpr size_t kScratchBytes = 32u << 20;
// The device address of that array on the current device, looked up once
// per device (hipGetSymbolAddress) and kept.
hipError_t scratch_address(void** out);

// Kernel launchers (kv_kernels.hip).  They validate nothing; the host checks
// every index the plan holds before calling them.
// `inline_plan` (nullptr: the plan is at a.plan on the device) holds
// `inline_bytes` <= kInlinePlanBytes of plan passed with the arguments.
// Events the dispatch itself records at the kernel's start and end (both
// null: no timing).
struct LaunchTiming {
    hipEvent_t start = nullptr;
    hipEvent_t stop = nullptr;
};

hipError_t launch_append(const AppendLaunch& a, const void* inline_plan, uint32_t inline_bytes, hipStream_t s,
                         const LaunchTiming& t = {});
hipError_t launch_gather(const GatherLaunch& a, const void* inline_plan, uint32_t inline_bytes, hipStream_t s);
hipError_t launch_gather_q8(const GatherQ8Launch& a, const void* inline_plan, uint32_t inline_bytes, hipStream_t s);
hipError_t launch_attention(const AttnLaunch& a, const void* inline_plan, uint32_t inline_bytes, hipStream_t s,
                            const LaunchTiming& t = {});
hipError_t launch_merge(const AttnLaunch& a, const void* inline_plan, uint32_t inline_bytes, hipStream_t s,
                        const LaunchTiming& t = {});
hipError_t launch_f32_to_f16(const float* in, uint16_t* out, size_t n, hipStream_t s);
// Streaming read (copy = false; dst receives nothing in practice but needs
// blocks * 256 * 16 bytes) or copy of `bytes` (a multiple of 16), in a grid
// stride or (span) one contiguous span per workgroup.
hipError_t launch_stream(bool copy, bool span, const void* src, void* dst, size_t bytes, uint32_t blocks,
                         hipStream_t s);
hipError_t launch_qkv(const QkvLaunch& a, const void* inline_plan, uint32_t inline_bytes, hipStream_t s,
                      const LaunchTiming& t = {});

// Contiguous f32 attention (Kernels::attention): query i at position
// q_pos0 + i over K/V rows 0 .. q_pos0 + i, row j of head h at
// k + j * k_stride + h * head_dim; out row i at out + i * out_stride.
struct RowsLaunch {
    const float* q;
    const float* k;
    const float* v;
    float* out;
    int64_t q_stride, k_stride, v_stride, out_stride;
    uint32_t n_q, q_pos0, n_head, head_dim;
    float qscale;  // log2(e) / sqrt(head_dim)
};
hipError_t launch_attention_rows(const RowsLaunch& a, hipStream_t s);
// Blocks a fused launch needs for its orphan rows (n_orphans set).
uint32_t orphan_blocks(const AttnLaunch& a);
// Compute units of the current device, looked up once per device (256 if
// the query fails).
uint32_t device_cus();
// Workgroups of the wide (one item per workgroup of several waves) attention
// launch for these parameters that one CU holds at once, from the kernel's
// own resource use (hipOccupancyMaxActiveBlocksPerMultiprocessor); 0 if
// unknown.
uint32_t wide_blocks_per_cu(uint32_t head_dim, bool q8, uint32_t nq_tile, bool fused);
// The same for the f16 prefill launch (attn_prefill_kernel) at this head_dim.
uint32_t prefill_blocks_per_cu(uint32_t head_dim);
bool attention_supported(uint32_t head_dim);

}  // namespace ni
