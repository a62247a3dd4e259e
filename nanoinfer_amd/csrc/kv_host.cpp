// kv_host.cpp -- host side of the paged f16 KV-cache path and its C ABI.
//
// The page allocator and block tables restate Batch's bookkeeping
// (crates/metal/src/batch.rs:129-254): a LIFO free stack initialised so that
// pages are handed out 0, 1, 2, ... (:174), pages grown on demand
// (ensure_blocks, :243-254), rollback freeing whole trailing pages last-first
// (truncate, :220-227).  Error texts are the reference's.
//
// Each data-path call builds a compact plan (kv_plan.h) from its rows -- the
// destination slot of every appended row, attention work items sorted
// longest first, merge items, and the page lists those items read -- and
// launches the kernels over it.  A plan of up to 32 KB travels inside the
// kernel arguments (the runtime copies them with the dispatch); a larger one
// is copied into a pinned staging slot and uploaded on the handle's copy
// stream, the caller's stream waiting on an event.  Staging slots are
// recycled through events, so bookkeeping calls after a data call never
// race with the work it enqueued.
#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "kv_plan.h"
#include "nanoinfer_kv.h"

using namespace ni;

namespace {

constexpr uint32_t kRingSlots = 4;

// Plans are uploaded on the handle's own copy stream and the caller's stream
// waits for the upload with an event, so the copy overlaps the previous
// step's kernels instead of sitting between them.
// Query groups (matrix-core kernel) take wide workgroups from this many
// (item, layer, head) units on, instead of splitting into partitions.
constexpr uint64_t kWideMinGroupUnits = 256;
// A step of prompt chunks (every sequence queried as prefill groups, no
// partitions) on a Q8 pool with at least this many (sequence, layer, head)
// units: the prefill launch appends each sequence's rows (one workgroup per
// sequence, layer and head, its groups in turn) instead of an append launch
// before it (plan_attention).
constexpr uint64_t kSeqPrefillMinUnits = 1536;
constexpr size_t kAlign = 256;
constexpr uint32_t kMinSplit = 64;  // smallest partition the planner uses (tokens)
constexpr size_t kProfileEvents = 8192;  // events created when profiling starts

thread_local std::string g_create_error;

// ni_kv_step_noalloc's scratch array is one per GPU: the first handle to call
// that entry point on a device holds it until ni_kv_destroy, and calls
// through any other handle on that device are refused (their launches would
// overwrite each other's partials whenever the two overlap).
std::mutex g_scratch_mu;
std::vector<const void*> g_scratch_holder;  // per device index

bool claim_scratch(const void* kv, int dev) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (dev < 0) return false;
    if ((size_t)dev >= g_scratch_holder.size()) g_scratch_holder.resize((size_t)dev + 1, nullptr);
    if (!g_scratch_holder[dev]) g_scratch_holder[dev] = kv;
    return g_scratch_holder[dev] == kv;
}

void release_scratch(const void* kv, int dev) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (dev >= 0 && (size_t)dev < g_scratch_holder.size() && g_scratch_holder[dev] == kv)
        g_scratch_holder[dev] = nullptr;
}

inline size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

struct StagingSlot {
    uint8_t* host = nullptr;  // pinned
    uint8_t* dev = nullptr;
    size_t cap = 0;
    hipEvent_t done = nullptr;      // the kernels that read this slot finished
    hipEvent_t uploaded = nullptr;  // the slot's upload finished (copy stream)
    bool pending = false;
    bool held = false;  // the plan of an open step: not handed out again before ni_kv_step_end
};

// Work of one data-path call, before serialisation.
struct Plan {
    std::vector<AppendEntry> app;
    std::vector<AppendEntry> orphans;  // fused: rows of sequences without queries
    std::vector<AttnItem> items;
    std::vector<MergeItem> merges;
    std::vector<AttnItem> pitems;    // prefill groups (attn_prefill_kernel), their merges
    std::vector<MergeItem> pmerges;  //   and partial slots (a region after the others')
    std::vector<uint32_t> table;
    std::vector<PrefillSeq> pseqs;  // prompt-chunk step: the prefill launch appends, a workgroup per sequence
    std::vector<uint16_t> order;    // balanced wide launch: the (item, layer, head) unit of each workgroup
    std::vector<uint16_t> porder;   // balanced one-round prefill launch: the same, over pitems
    uint32_t n_slots = 0;
    uint32_t n_pslots = 0;
    uint32_t nq_tile = 1;
    uint32_t napp_total = 0;  // fused: rows the attention items append
    bool fused = false;
    bool wide = false;        // kWideWaves waves per attention workgroup
    bool seq_prefill = false; // every row belongs to a sequence queried as prefill groups (see pseqs)
    // Some launch of the plan reads the append entries `app` (an append
    // launch, a workgroup prologue, a prefill workgroup's appends); a fused
    // launch whose items take their new rows as their pages stream and whose
    // other rows are orphans reads none, and its plan leaves them out.
    bool app_read = true;
    void clear() {
        app.clear();
        orphans.clear();
        pseqs.clear();
        order.clear();
        porder.clear();
        seq_prefill = false;
        items.clear();
        merges.clear();
        pitems.clear();
        pmerges.clear();
        table.clear();
        n_slots = 0;
        n_pslots = 0;
        nq_tile = 1;
        napp_total = 0;
        fused = false;
        wide = false;
        app_read = true;
    }
};

// Byte offsets of each part of a serialised plan.
struct Offsets {
    size_t app, orphans, items, merges, pitems, pmerges, pseqs, table, order, porder, total;
};

// Where the kernels find a plan: in the launch arguments (small plans) or in
// a staging slot uploaded on the copy stream.
struct PlanRef {
    const void* inl = nullptr;
    uint32_t inl_bytes = 0;
    const uint8_t* dev = nullptr;
    StagingSlot* slot = nullptr;
};

// A query row as the planner sees it.  [new_begin, new_end) are the positions
// its sequence appends in this call, starting at append entry app_first
// (new_begin == new_end when the call appends nothing).
struct QRow {
    uint32_t row, seq, pos;
    uint32_t new_begin, new_end, app_first;
    uint32_t pre = 0;  // fused or prompt-chunk step: a chunk queried at more rows than one matrix tile (prefill launch)
};

}  // namespace

struct ni_kv {
    ni_kv_opts o{};
    uint32_t max_pages = 0;  // per sequence: ceil(max_ctx / 16) (batch.rs:164)
    std::vector<uint32_t> seq_len;
    std::vector<uint8_t> live;
    std::vector<std::vector<uint32_t>> pages;
    std::vector<uint32_t> free_pages;  // LIFO stack, back() is handed out next
    std::string err;
    bool host_only = false;
    int device = 0;

    uint16_t* kpool = nullptr;
    uint16_t* vpool = nullptr;
    size_t pool_bytes = 0;  // K and V together
    uint64_t layer_halves = 0;
    uint64_t page_halves = 0;
    uint32_t head_halves = 0;

    StagingSlot ring[kRingSlots];
    uint32_t ring_next = 0;
    hipStream_t copy_stream = nullptr;
    float* partials = nullptr;
    size_t partials_bytes = 0;
    // Outgrown partials buffers, each with an event recorded when it was
    // retired: launches enqueued before may still use it, so it is freed by
    // the next ni_kv_sync that finds its event complete (or ni_kv_destroy).
    std::vector<std::pair<float*, hipEvent_t>> partials_retired;
    // ni_kv_step_noalloc: this device's scratch array (null if its address
    // could not be found), and set for the duration of such a call.
    float* scratch = nullptr;
    hipError_t scratch_err = hipSuccess;
    bool no_alloc = false;

    // Order of data-path calls across streams (begin_call): `dirty` says
    // that work of this handle was enqueued on dirty_stream after `order`
    // was last recorded; `order` (valid if order_valid) marks the end of the
    // handle's work enqueued on order_stream before it.
    hipEvent_t order = nullptr;
    hipStream_t order_stream = nullptr;
    bool order_valid = false;
    hipStream_t dirty_stream = nullptr;
    bool dirty = false;

    uint32_t profile = 0;  // bit k: bracket kernel k's launches with events
    std::vector<std::pair<hipEvent_t, hipEvent_t>> prof_ev[NI_K_COUNT];
    std::vector<hipEvent_t> ev_pool;

    // scratch reused across calls
    Plan plan;
    std::vector<uint8_t> blob;  // the serialised plan
    std::vector<QRow> qrows;
    std::vector<int64_t> seq_tab;     // seq -> offset in plan.table, -1 if absent
    std::vector<uint32_t> seq_need;   // seq -> pages needed this call
    std::vector<uint32_t> step_mark;  // seq -> stamp of the last step that listed it
    uint32_t step_stamp = 0;

    // A step planned by ni_kv_step_begin and run one layer per
    // ni_kv_step_layer call until ni_kv_step_end.
    struct OpenStep {
        bool open = false;
        Plan plan;
        std::vector<uint8_t> blob;
        std::vector<std::pair<uint32_t, uint32_t>> commit;  // (seq, n_new) for ni_kv_step_end
        bool placed = false;  // plan serialised and reachable (at the first layer call)
        Offsets off{};
        PlanRef ref;
        hipStream_t stream = nullptr;  // of the last layer call
    } step;

    int fail(int code, const char* fmt, ...) __attribute__((format(printf, 3, 4))) {
        char buf[512];
        va_list ap;
        va_start(ap, fmt);
        vsnprintf(buf, sizeof buf, fmt, ap);
        va_end(ap);
        err = buf;
        return code;
    }
    int hip_fail(hipError_t e, const char* what) {
        return fail(NI_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
    }
    PoolGeom geom() const {
        PoolGeom g;
        g.k = kpool;
        g.v = vpool;
        g.layer_halves = layer_halves;
        g.page_halves = page_halves;
        g.head_halves = head_halves;
        g.n_head = o.n_head;
        g.head_dim = o.head_dim;
        g.q8 = (o.flags & NI_KV_Q8) ? 1u : 0u;
        return g;
    }
};

namespace {

int check_seq(ni_kv* kv, uint32_t s) {
    if (s >= kv->o.max_seqs) return kv->fail(NI_ERR_BAD_ARG, "sequence %u out of range (%u slots)", s, kv->o.max_seqs);
    return NI_OK;
}

// Batch::ensure_blocks (batch.rs:243-254).
int ensure_pages(ni_kv* kv, uint32_t s, uint64_t len) {
    if (len > kv->o.max_ctx)
        return kv->fail(NI_ERR_CONTEXT_FULL, "sequence %u: context full (%llu > %u)", s, (unsigned long long)len,
                        kv->o.max_ctx);
    auto& pg = kv->pages[s];
    while ((uint64_t)pg.size() * kPage < len) {
        if (kv->free_pages.empty()) return kv->fail(NI_ERR_POOL_EXHAUSTED, "KV cache pool exhausted");
        pg.push_back(kv->free_pages.back());
        kv->free_pages.pop_back();
    }
    return NI_OK;
}

// Batch::truncate (batch.rs:220-227).
int truncate_seq(ni_kv* kv, uint32_t s, uint32_t len) {
    if (len > kv->seq_len[s]) return kv->fail(NI_ERR_BAD_LEN, "assertion failed: len <= self.seq_len[s]");
    kv->seq_len[s] = len;
    const size_t keep = (len + kPage - 1) / kPage;
    auto& pg = kv->pages[s];
    while (pg.size() > keep) {
        kv->free_pages.push_back(pg.back());
        pg.pop_back();
    }
    return NI_OK;
}

// Is position `pos` of live sequence `s` backed by a page?
int check_row(ni_kv* kv, const ni_row& r) {
    if (r.seq >= kv->o.max_seqs)
        return kv->fail(NI_ERR_BAD_ARG, "sequence %u out of range (%u slots)", r.seq, kv->o.max_seqs);
    if (!kv->live[r.seq]) return kv->fail(NI_ERR_NOT_LIVE, "sequence %u is not live", r.seq);
    if ((uint64_t)r.pos >= (uint64_t)kv->pages[r.seq].size() * kPage)
        return kv->fail(NI_ERR_NOT_RESERVED, "sequence %u: position %u has no page (reserved %zu)", r.seq, r.pos,
                        kv->pages[r.seq].size() * kPage);
    return NI_OK;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

bool is_q8(const ni_kv_opts& o) { return (o.flags & NI_KV_Q8) != 0; }

// Rows of one sequence that share one pass over the keys (the matrix-core
// tile, f16 and Q8 pools alike).
uint32_t max_group_rows(const ni_kv*) { return kMaxGroupRows; }

// Halves of one K (or V) block of a (page, head).
uint64_t kv_block_halves(const ni_kv_opts& o) {
    return is_q8(o) ? (uint64_t)kPage * o.head_dim / 2 + kPage * 2 : (uint64_t)kPage * o.head_dim;
}

int check_f32_operand(ni_kv* kv, const char* name, const void* p, int64_t row_stride, int64_t layer_stride,
                      bool all_layers) {
    if (!p) return kv->fail(NI_ERR_BAD_ARG, "%s is NULL", name);
    if (!aligned16(p) || row_stride % 4 != 0 || (all_layers && layer_stride % 4 != 0) || row_stride < 0 ||
        (all_layers && layer_stride < 0))
        return kv->fail(NI_ERR_BAD_ARG, "%s must be 16-byte aligned with non-negative strides that are multiples of 4",
                        name);
    return NI_OK;
}

int layer_range(ni_kv* kv, int32_t layer, uint32_t* layer0, uint32_t* n_lay) {
    if (layer == NI_ALL_LAYERS) {
        *layer0 = 0;
        *n_lay = kv->o.n_layer;
        return NI_OK;
    }
    if (layer < 0 || (uint32_t)layer >= kv->o.n_layer)
        return kv->fail(NI_ERR_BAD_ARG, "layer %d out of range (%u layers)", layer, kv->o.n_layer);
    *layer0 = (uint32_t)layer;
    *n_lay = 1;
    return NI_OK;
}

// A wide launch whose workgroups are all resident at once ends with its most
// loaded CU.  The dispatcher deals such a launch's workgroups to the CUs in
// rounds: block b shares a CU with blocks b +- C, b +- 2C, ... (C = the
// device's CUs; per-workgroup timestamps and hardware ids on MI355X put
// blocks b, b + 256 and b + 512 of a 768-block launch on one CU in each of
// 240 launches traced, and a CU's finish time followed the pages of its
// blocks: correlation 0.8, an appended prompt row costing ~1.9 pages' time
// per 16 rows beyond its page).  Items sorted longest first would give one CU
// the largest item of every round.  Instead the (item, layer, head) units go
// to CUs longest first, each to the least loaded CU with a free slot, and
// P.order records the unit each block runs.
// Longest first, round by round: round r gives block c + r * C to every CU
// c that takes one (all but the last round: every CU; the last: CUs below
// rem), the largest units of the round to the least loaded CUs.  `cost`:
// (cost, item) sorted by cost, largest first; order[b] = the unit (item *
// lh + layer * heads + head) block b runs.
void deal_units(const std::vector<std::pair<uint64_t, uint32_t>>& cost, uint64_t lh, uint64_t C, uint64_t R,
                uint64_t rem, std::vector<uint16_t>& order) {
    std::vector<uint64_t> load(C, 0);
    std::vector<uint32_t> cus(C);
    order.assign((R - 1) * C + rem, 0);
    uint64_t u = 0;  // position in the cost order, (item, unit of the item)
    for (uint64_t r = 0; r < R; r++) {
        const uint32_t n_r = (uint32_t)(r + 1 < R ? C : rem);
        for (uint32_t c = 0; c < n_r; c++) cus[c] = c;
        if (r > 0)
            std::stable_sort(cus.begin(), cus.begin() + n_r, [&](uint32_t x, uint32_t y) { return load[x] < load[y]; });
        for (uint32_t k = 0; k < n_r; k++, u++) {
            const auto& ci = cost[u / lh];
            const uint32_t c = cus[k];
            order[c + C * r] = (uint16_t)(ci.second * lh + u % lh);
            load[c] += ci.first;
        }
    }
}

void balance_units(ni_kv* kv, Plan& P, uint32_t n_lay) {
    P.order.clear();
    if (!P.wide || P.items.empty() || kv->host_only) return;
    const uint64_t lh = (uint64_t)n_lay * kv->o.n_head;
    const uint64_t n_units = (uint64_t)P.items.size() * lh;
    const uint64_t C = device_cus();
    const bool fused = P.napp_total > 0 || !P.orphans.empty();
    const uint64_t S = wide_blocks_per_cu(kv->o.head_dim, is_q8(kv->o), P.nq_tile, fused);
    // (one round: every block has a CU of its own already)
    if (S == 0 || n_units <= C || n_units > C * S || n_units > 65536) return;
    const uint64_t R = (n_units + C - 1) / C;  // rounds; CUs below `rem` receive R blocks, the others R - 1
    const uint64_t rem = n_units - (R - 1) * C;
    // cost in 1/16 pages: the item's pages, and ~1.9 pages more per 16
    // appended rows (2/16 per row)
    std::vector<std::pair<uint64_t, uint32_t>> cost(P.items.size());
    for (uint32_t i = 0; i < P.items.size(); i++) {
        const AttnItem& it = P.items[i];
        const uint64_t pages = (it.kv_end + kPage - 1) / kPage - it.kv_begin / kPage;
        cost[i] = {16 * pages + 2ull * it.napp, i};
    }
    std::stable_sort(cost.begin(), cost.end(),
                     [](const std::pair<uint64_t, uint32_t>& x, const std::pair<uint64_t, uint32_t>& y) {
                         return x.first > y.first;
                     });
    deal_units(cost, lh, C, R, rem, P.order);
}

// A one-layer-per-launch prefill step on an f16 pool whose (item, layer,
// head) units all fit on the GPU at once (at most prefill_blocks_per_cu x
// CUs): block b runs on CU b % C as in the wide launches above, so the units
// are dealt to CUs the same way (cost: the item's 32-key tiles) and P.porder
// records the unit each block runs.  16 x 512-row prompts, one layer per
// launch (1536 units, 6 per CU): in plan order the most loaded CU held 1.26x
// the mean work, dealt 1.00x; 470.0-471.7 against 485.5-488.4 us per step
// (`ni_drive prefill --step-layers`).
void balance_prefill_units(Plan& P, uint32_t n_lay, uint32_t n_head, uint64_t C, uint64_t S) {
    P.porder.clear();
    const uint64_t lh = (uint64_t)n_lay * n_head;
    const uint64_t n_units = (uint64_t)P.pitems.size() * lh;
    if (S == 0 || n_units <= C || n_units > C * S || n_units > 65536) return;
    const uint64_t R = (n_units + C - 1) / C;
    const uint64_t rem = n_units - (R - 1) * C;
    std::vector<std::pair<uint64_t, uint32_t>> cost(P.pitems.size());
    for (uint32_t i = 0; i < P.pitems.size(); i++) {
        const AttnItem& it = P.pitems[i];
        cost[i] = {(it.kv_end - it.kv_begin + 31) / 32, i};
    }
    std::stable_sort(cost.begin(), cost.end(),
                     [](const std::pair<uint64_t, uint32_t>& x, const std::pair<uint64_t, uint32_t>& y) {
                         return x.first > y.first;
                     });
    deal_units(cost, lh, C, R, rem, P.porder);
}

// Attention part of a plan: group consecutive query rows of one sequence at
// consecutive positions, split each group's keys into partitions, sort the
// items longest first.
int plan_attention(ni_kv* kv, uint32_t split_tokens, uint32_t n_lay) {
    Plan& P = kv->plan;
    const auto& qr = kv->qrows;
    if (qr.empty()) return NI_OK;
    struct Group {
        uint32_t seq, row0, pos0, nq;
        uint32_t new_begin, new_end, app_first;
        uint32_t pre;  // runs in the prefill launch whatever its size
    };
    std::vector<Group> groups;
    groups.reserve(qr.size());
    // Runs longer than one matrix tile form prefill groups (f16 pools, and Q8
    // pools at head_dim 64).
    const bool prefill = !is_q8(kv->o) || kv->o.head_dim == 64;
    const uint32_t max_group = prefill ? kPrefillRows : max_group_rows(kv);
    for (const QRow& r : qr) {
        if (!groups.empty()) {
            Group& g = groups.back();
            if (g.seq == r.seq && g.row0 + g.nq == r.row && g.pos0 + g.nq == r.pos && g.nq < max_group) {
                g.nq++;
                continue;
            }
        }
        groups.push_back({r.seq, r.row, r.pos, 1, r.new_begin, r.new_end, r.app_first, r.pre});
    }
    // Partition size: the caller's, or (0) automatic.  Splitting costs a
    // merge launch (~5-7 us) and the partials' round trip, so it pays only
    // when the unsplit items cannot keep the GPU busy: 256 CUs hold 1024
    // workgroups at once, and with >= 2048 of them, sorted longest first,
    // the tail is short -- only items longer than kLongItem keys are split
    // then.  Below that, the largest of 1024/512/256/128 tokens that yields
    // >= 2048 workgroups.
    // Between kWideMinUnits and kFillWorkgroups units of single-row items
    // (head_dim 64: a launch of one layer of 43..170 sequences), workgroups
    // of kWideWaves waves share each item's pages instead of splitting it:
    // no partials, no merge launch.  Query groups of up to one matrix tile
    // (a verify step's rows) do the same from kWideMinGroupUnits units.
    // Prefill groups (more rows than one matrix tile, in a launch of their
    // own) are split automatically only past kLongItem keys: each of their
    // workgroups already carries 64 queries, and splitting them to fill the
    // GPU cost more than it gained (prompt steps, every row queried, no split
    // against the fill choice: one launch per layer 16 x 512 rows 611 against
    // 753 us, 4 x 512 286 against 436, 1 x 512 254 against 305; all layers 1 x
    // 512 45 against 67 us, 4 x 512 146 against 167, 2 x 512 and 8 x 256 the
    // same).
    constexpr uint32_t kLongItem = 4096;
    uint32_t part = split_tokens, pre_part = split_tokens;
    if (part == 0) {
        constexpr uint64_t kFillWorkgroups = 2048;
        constexpr uint64_t kWideMinUnits = 512;
        static const uint32_t kChoices[] = {1024, 512, 256, 128};
        pre_part = kLongItem;
        const uint64_t per_unit = (uint64_t)n_lay * kv->o.n_head;
        const uint64_t units = (uint64_t)groups.size() * per_unit;
        constexpr uint32_t kShortItem = 1280;  // keys (a 1024-token context and its new rows)
        bool single = true, tiles = true;  // every group one row; every group within one matrix tile
        uint32_t max_keys = 0;
        for (const Group& g : groups) {
            single &= g.nq == 1;
            tiles &= g.nq <= kMfmaTile && !g.pre;
            max_keys = std::max(max_keys, g.pos0 + g.nq);
        }
        if (units >= kFillWorkgroups) {
            part = kLongItem;
        } else if (tiles && units >= (single ? kWideMinUnits : kWideMinGroupUnits) && kv->o.head_dim == 64) {
            part = kLongItem;
            P.wide = true;
        } else if (n_lay == 1 && max_keys <= kShortItem) {
            // One layer per launch and no item past kShortItem keys: the
            // merge launch a split needs costs more than the fill it buys
            // (decode rows of 4..32 sequences with contexts U[64,1024]: 213-240
            // against 251-284 us per step of 12 such launches; 8 x 1024 keys
            // 208 against 246; from 2048 keys the split wins, 4 x 2048 242
            // against 285, 4 x 4096 246 against 524, and 16 x U[1024,2048]
            // 262 against 273).
            part = kLongItem;
        } else {
            part = kChoices[3];
            for (uint32_t c : kChoices) {
                uint64_t items = 0;
                for (const Group& g : groups) items += ((uint64_t)g.pos0 + g.nq + c - 1) / c;
                if (items * per_unit >= kFillWorkgroups) {
                    part = c;
                    break;
                }
            }
        }
    } else if (part % kPage != 0 || part < kMinSplit) {
        return kv->fail(NI_ERR_BAD_ARG, "split_tokens %u must be 0 or a multiple of 16 that is >= %u", split_tokens,
                        kMinSplit);
    }
    // Page lists: one segment per sequence, long enough for its last query.
    for (const Group& g : groups) {
        const uint32_t need = (g.pos0 + g.nq + kPage - 1) / kPage;
        kv->seq_need[g.seq] = std::max(kv->seq_need[g.seq], need);
    }
    for (const Group& g : groups) {
        if (kv->seq_tab[g.seq] >= 0) continue;
        kv->seq_tab[g.seq] = (int64_t)P.table.size();
        const auto& pg = kv->pages[g.seq];
        P.table.insert(P.table.end(), pg.begin(), pg.begin() + kv->seq_need[g.seq]);
    }
    uint32_t max_nq = 1;
    // An item [b, e) of a fused step appends this call's new rows in [b, e).
    // (In a fused step a sequence queried at more than max_group_rows rows
    // forms prefill groups only; the launch's extra blocks append its rows.)
    auto item = [&](const Group& g, uint32_t tab, uint32_t b, uint32_t e, uint32_t slot) {
        AttnItem it{};
        it.tab = tab;
        it.row0 = g.row0;
        it.pos0 = g.pos0;
        it.nq = g.nq;
        it.kv_begin = b;
        it.kv_end = e;
        it.part_slot = slot;
        if (P.fused && !g.pre) {  // (a prefill group's rows are appended by the extra blocks)
            const uint32_t lo = std::max(b, g.new_begin), hi = std::min(e, g.new_end);
            if (hi > lo) {
                it.app0 = g.app_first + (lo - g.new_begin);
                it.napp = hi - lo;
                it.app_pos = lo;
                it.app_src = P.app[it.app0].src_row;
                P.napp_total += it.napp;
            }
        }
        (g.pre || g.nq > kMfmaTile ? P.pitems : P.items).push_back(it);
    };
    // Per sequence (page-list offset): its appended rows, for prefill
    // workgroups that append them (P.seq_prefill).
    struct SeqRows {
        uint32_t app_first, new_begin, new_end;
    };
    std::vector<SeqRows> app_of;  // by table offset
    for (const Group& g : groups) {
        const bool pre = g.pre || g.nq > kMfmaTile;
        if (P.seq_prefill) {
            const uint32_t tab = (uint32_t)kv->seq_tab[g.seq];
            if (app_of.size() <= tab) app_of.resize(tab + 1, {0u, 0u, 0u});
            app_of[tab] = {g.app_first, g.new_begin, g.new_end};
        }
        if (!pre) max_nq = std::max(max_nq, g.nq);
        const uint32_t L = g.pos0 + g.nq;
        const uint32_t gpart = pre ? pre_part : part;
        const uint32_t n_parts = (L + gpart - 1) / gpart;
        const uint32_t tab = (uint32_t)kv->seq_tab[g.seq];
        if (n_parts <= 1) {
            item(g, tab, 0, L, kNoSlot);
            continue;
        }
        uint32_t& n_slots = pre ? P.n_pslots : P.n_slots;
        const uint32_t slot0 = n_slots;
        for (uint32_t p = 0; p < n_parts; p++) item(g, tab, p * gpart, std::min((p + 1) * gpart, L), slot0 + p);
        (pre ? P.pmerges : P.merges).push_back({g.row0, g.nq, slot0, n_parts});
        n_slots += n_parts;
    }
    for (const Group& g : groups) {
        kv->seq_need[g.seq] = 0;
        kv->seq_tab[g.seq] = -1;
    }
    // Longest first, so the long items start early and the short ones fill
    // the tail.
    auto longest_first = [](const AttnItem& x, const AttnItem& y) {
        return (x.kv_end - x.kv_begin) > (y.kv_end - y.kv_begin);
    };
    std::stable_sort(P.items.begin(), P.items.end(), longest_first);
    // Prefill groups of one sequence next to each other (its longest first),
    // sequences by their longest group: a launch's workgroups of one (item,
    // layer, head) are n_lay * n_head apart, so the groups of one sequence
    // sharing a (layer, head)'s keys then run at about the same time (16 x
    // 512-row prefill 504 -> 463 us per step against longest first; the
    // attention launch's L2 hits 2.4M -> 10.4M and misses 15.3M -> 7.3M,
    // rocprofv3 TCC_HIT/TCC_MISS).
    {
        std::vector<uint32_t> longest;  // by table offset (one per sequence)
        for (const AttnItem& it : P.pitems) {
            if (longest.size() <= it.tab) longest.resize(it.tab + 1, 0);
            longest[it.tab] = std::max(longest[it.tab], it.kv_end - it.kv_begin);
        }
        std::stable_sort(P.pitems.begin(), P.pitems.end(), [&](const AttnItem& x, const AttnItem& y) {
            if (longest[x.tab] != longest[y.tab]) return longest[x.tab] > longest[y.tab];
            if (x.tab != y.tab) return x.tab < y.tab;
            return (x.kv_end - x.kv_begin) > (y.kv_end - y.kv_begin);
        });
    }
    // Prompt-chunk step without partitions: one prefill workgroup per
    // (sequence, layer, head) runs the sequence's groups shortest first, each
    // after appending the new rows up to its last key (the last group: all
    // that are left), so the append's loads interleave with attention.
    // Only with enough workgroups to fill the GPU (kSeqPrefillMinUnits
    // (sequence, layer, head) units); below that the groups' own workgroups
    // after an append launch run faster (all layers, 512-row prompts: 2 of
    // them 65 against 95 us, 8 (1152 units) 251 against 276; from 12 (1728)
    // the single launch is ahead, 363 against 366 us, 16 467 against 479).
    uint32_t n_seqs = 0;
    for (uint32_t i = 0; i < P.pitems.size(); i++) n_seqs += i == 0 || P.pitems[i].tab != P.pitems[i - 1].tab;
    if (P.seq_prefill && (uint64_t)n_seqs * n_lay * kv->o.n_head < kSeqPrefillMinUnits) P.seq_prefill = false;
    if (P.seq_prefill && P.items.empty() && P.n_pslots == 0 && !P.pitems.empty()) {
        uint64_t rows = 0;  // the sequences' new rows: all of the step's, or an append launch
        for (uint32_t i = 0; i < P.pitems.size(); i++)
            if (i == 0 || P.pitems[i].tab != P.pitems[i - 1].tab)
                rows += app_of[P.pitems[i].tab].new_end - app_of[P.pitems[i].tab].new_begin;
        for (uint32_t i = 0; rows == P.app.size() && i < P.pitems.size();) {
            const uint32_t tab = P.pitems[i].tab;
            uint32_t e = i + 1;
            while (e < P.pitems.size() && P.pitems[e].tab == tab) e++;
            std::reverse(P.pitems.begin() + i, P.pitems.begin() + e);  // longest first -> shortest first
            const SeqRows& sr = app_of[tab];
            uint32_t lo = sr.new_begin;
            for (uint32_t j = i; j < e; j++) {
                AttnItem& it = P.pitems[j];
                const uint32_t hi = j + 1 == e ? sr.new_end : std::max(lo, std::min(it.kv_end, sr.new_end));
                it.app0 = sr.app_first + (lo - sr.new_begin);
                it.napp = hi - lo;
                lo = hi;
            }
            P.pseqs.push_back({i, e - i});
            i = e;
        }
    }
    P.seq_prefill = !P.pseqs.empty();
    // f16 prefill items carry their first pages' ids (the prefill kernel
    // issues its first tiles' DMA from them, beside the item's q and page-id
    // loads instead of after them).
    if (!is_q8(kv->o)) {
        for (AttnItem& it : P.pitems) {
            const uint32_t pb = it.kv_begin / kPage, pe = (it.kv_end + kPage - 1) / kPage;
            for (uint32_t i = 0; i < 4; i++) it.first_pages[i] = pe > pb ? P.table[it.tab + std::min(pb + i, pe - 1)] : 0u;
        }
        // A launch whose workgroups are all resident at once has its units
        // dealt to the CUs (balance_prefill_units).  A launch of at most two
        // rounds of the GPU's resident workgroups ends on the groups that
        // start last: there the groups of at most a quarter of the longest
        // group's keys go last, longest first (each sequence's other groups
        // keep the order above; the short ones re-read only its first keys).
        // One layer per launch, 16 x 512 rows, when 5 workgroups fit a CU
        // (1.2 rounds): 30.0 -> 26.9 us; all 12 layers (14 rounds) do not
        // take it (~0.8% slower reordered).
        const uint64_t units = (uint64_t)P.pitems.size() * n_lay * kv->o.n_head;
        const uint64_t per_cu = prefill_blocks_per_cu(kv->o.head_dim), C = device_cus();
        const uint64_t resident = per_cu * C;
        if (units <= resident) {
            // (not in ni_kv_step_noalloc, whose plans travel inline: the order
            // array would lower the size of step it takes)
            if (!kv->no_alloc) balance_prefill_units(P, n_lay, kv->o.n_head, C, per_cu);
        } else if (units <= 2 * resident) {
            uint32_t longest_all = 0;
            for (const AttnItem& it : P.pitems) longest_all = std::max(longest_all, it.kv_end - it.kv_begin);
            const uint32_t short_keys = longest_all / 4;
            const auto tail = std::stable_partition(P.pitems.begin(), P.pitems.end(), [&](const AttnItem& x) {
                return x.kv_end - x.kv_begin > short_keys;
            });
            std::stable_sort(tail, P.pitems.end(), [](const AttnItem& x, const AttnItem& y) {
                return (x.kv_end - x.kv_begin) > (y.kv_end - y.kv_begin);
            });
        } else {
            // Longer launches run each sequence's groups shortest first (16 x
            // 512-row prompts, all layers: 392.3-393.2 against 395.7-397.0 us
            // per step; one layer per launch keeps the order above: 506
            // against 500).
            for (size_t i = 0; i < P.pitems.size();) {
                size_t e = i + 1;
                while (e < P.pitems.size() && P.pitems[e].tab == P.pitems[i].tab) e++;
                std::reverse(P.pitems.begin() + i, P.pitems.begin() + e);
                i = e;
            }
        }
    }
    // Single queries stream on the vector kernel; groups go to matrix cores.
    P.nq_tile = max_nq > 1 ? kMfmaTile : 1;
    // Only single rows at head_dim 64 take their new rows as their pages
    // stream (attn_split_kernel; on Q8 pools its wide launches); every other
    // fused launch appends in workgroup prologues from the entries.
    const bool streams = kv->o.head_dim == 64 && P.nq_tile == 1 && (!is_q8(kv->o) || P.wide);
    P.app_read = !P.fused || P.seq_prefill || !streams;
    balance_units(kv, P, n_lay);
    return NI_OK;
}

hipEvent_t take_event(ni_kv* kv) {
    if (!kv->ev_pool.empty()) {
        hipEvent_t e = kv->ev_pool.back();
        kv->ev_pool.pop_back();
        return e;
    }
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    return e;
}

// Timing of one launch of kernel `k` when profiling is on: the events go to
// the launch, whose dispatch records the kernel's start and end in them.
struct ProfileScope {
    ni_kv* kv;
    int kernel;
    LaunchTiming t;
    ProfileScope(ni_kv* kv_, int k) : kv(kv_), kernel(k) {
        // No event creation inside ni_kv_step_noalloc.
        if (!(kv->profile & (1u << k)) || kv->no_alloc) return;
        t.start = take_event(kv);
        t.stop = take_event(kv);
        if (!t.start || !t.stop) t = LaunchTiming{};
    }
    ~ProfileScope() {
        if (t.start) kv->prof_ev[kernel].push_back({t.start, t.stop});
    }
};

// Reserve a staging slot of at least `bytes`; waits for the slot's previous
// use to finish.
int acquire_slot(ni_kv* kv, size_t bytes, StagingSlot** out) {
    if (kv->ring[kv->ring_next].held) kv->ring_next = (kv->ring_next + 1) % kRingSlots;  // at most one is held
    StagingSlot& sl = kv->ring[kv->ring_next];
    kv->ring_next = (kv->ring_next + 1) % kRingSlots;
    if (sl.pending) {
        hipError_t e = hipEventSynchronize(sl.done);
        if (e != hipSuccess) return kv->hip_fail(e, "hipEventSynchronize(staging)");
        sl.pending = false;
    }
    if (sl.cap < bytes) {
        size_t cap = std::max<size_t>(align_up(bytes * 2, 1 << 16), 1 << 18);
        if (sl.host) (void)hipHostFree(sl.host);
        if (sl.dev) (void)hipFree(sl.dev);
        sl.host = nullptr;
        sl.dev = nullptr;
        sl.cap = 0;
        hipError_t e = hipHostMalloc(reinterpret_cast<void**>(&sl.host), cap, hipHostMallocDefault);
        if (e != hipSuccess) return kv->hip_fail(e, "hipHostMalloc(staging)");
        e = hipMalloc(reinterpret_cast<void**>(&sl.dev), cap);
        if (e != hipSuccess) return kv->hip_fail(e, "hipMalloc(staging)");
        sl.cap = cap;
    }
    *out = &sl;
    return NI_OK;
}

// The merge launch's workgroups per (merge item, layer, head): the largest
// merge_split_of over its items (the others' extra workgroups return at once).
uint32_t merge_split(const std::vector<MergeItem>& merges, uint32_t D) {
    uint32_t split = 1;
    for (const MergeItem& m : merges) split = std::max(split, merge_split_of(m.n_parts, m.nq, D));
    return split;
}

int ensure_partials(ni_kv* kv, size_t bytes, hipStream_t s, float** out) {
    if (kv->no_alloc) {
        if (bytes > kScratchBytes)
            return kv->fail(NI_ERR_BAD_ARG,
                            "the step needs %zu bytes of split partials; ni_kv_step_noalloc holds at most %zu "
                            "(a larger split_tokens, or ni_kv_step)",
                            bytes, kScratchBytes);
        *out = kv->scratch;
        return NI_OK;
    }
    *out = kv->partials;
    if (bytes <= kv->partials_bytes) return NI_OK;
    // Launches already enqueued may still use the old buffer: retire it
    // (no host wait here) rather than free it.  Every earlier call's work is
    // ordered before this point of `s` (begin_call), so an event recorded
    // here marks when the old buffer is free.
    const size_t cap = align_up(bytes + bytes / 2, 1 << 20);
    float* p = nullptr;
    hipError_t e = hipMalloc(reinterpret_cast<void**>(&p), cap);
    if (e != hipSuccess) return kv->hip_fail(e, "hipMalloc(partials)");
    if (kv->partials) {
        hipEvent_t ev = take_event(kv);
        if (!ev) {
            (void)hipFree(p);
            return kv->fail(NI_ERR_HIP, "hipEventCreate(partials)");
        }
        e = hipEventRecord(ev, s);
        if (e != hipSuccess) {
            kv->ev_pool.push_back(ev);
            (void)hipFree(p);
            return kv->hip_fail(e, "hipEventRecord(partials)");
        }
        kv->partials_retired.push_back({kv->partials, ev});
    }
    kv->partials = p;
    kv->partials_bytes = cap;
    *out = p;
    return NI_OK;
}

Offsets layout(const Plan& P) {
    Offsets o;
    o.app = 0;
    o.orphans = align_up(o.app + (P.app_read ? P.app.size() : 0) * sizeof(AppendEntry), kAlign);
    o.items = align_up(o.orphans + P.orphans.size() * sizeof(AppendEntry), kAlign);
    o.merges = align_up(o.items + P.items.size() * sizeof(AttnItem), kAlign);
    o.pitems = align_up(o.merges + P.merges.size() * sizeof(MergeItem), kAlign);
    o.pmerges = align_up(o.pitems + P.pitems.size() * sizeof(AttnItem), kAlign);
    o.pseqs = align_up(o.pmerges + P.pmerges.size() * sizeof(MergeItem), kAlign);
    o.table = align_up(o.pseqs + P.pseqs.size() * sizeof(PrefillSeq), kAlign);
    o.order = align_up(o.table + P.table.size() * sizeof(uint32_t), kAlign);
    o.porder = align_up(o.order + P.order.size() * sizeof(uint16_t), kAlign);
    o.total = align_up(o.porder + P.porder.size() * sizeof(uint16_t), kAlign);
    return o;
}

// Data-path calls of one handle run in call order, whatever streams they are
// made on: they share the handle's split partials and staging slots, and
// the pages they read or write change owners at once on the host (a page
// that truncate or free_seq returns may go to the next append).  So a call
// on a stream other than the one of the handle's previous work first makes
// its stream wait for that work: an event recorded on the previous stream
// (at the switch, so a call on one stream costs nothing extra), then
// hipStreamWaitEvent.  Work captured into a graph runs when the caller
// replays the graph, so calls on a capturing stream are not ordered here.
int begin_call(ni_kv* kv, hipStream_t s) {
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    hipError_t e = hipStreamIsCapturing(s, &cap);
    if (e != hipSuccess) return kv->hip_fail(e, "hipStreamIsCapturing");
    if (cap != hipStreamCaptureStatusNone) return NI_OK;
    if (kv->dirty && kv->dirty_stream != s) {
        e = hipEventRecord(kv->order, kv->dirty_stream);
        if (e != hipSuccess) return kv->hip_fail(e, "hipEventRecord(call order)");
        kv->order_stream = kv->dirty_stream;
        kv->order_valid = true;
    }
    if (kv->order_valid && kv->order_stream != s) {
        e = hipStreamWaitEvent(s, kv->order, 0);
        if (e != hipSuccess) return kv->hip_fail(e, "hipStreamWaitEvent(call order)");
    }
    kv->dirty = true;
    kv->dirty_stream = s;
    return NI_OK;
}

// Serialise plan P into `blob` and make it reachable from `s`: inside the
// launch arguments when it fits, else through a staging slot uploaded on the
// handle's copy stream (`s` waits for the upload).
int place_plan(ni_kv* kv, const Plan& P, std::vector<uint8_t>& blob, hipStream_t s, Offsets* off, PlanRef* ref) {
    if (int rc = begin_call(kv, s)) return rc;
    *off = layout(P);
    blob.resize(off->total);
    if (P.app_read && !P.app.empty())
        memcpy(blob.data() + off->app, P.app.data(), P.app.size() * sizeof(AppendEntry));
    if (!P.orphans.empty())
        memcpy(blob.data() + off->orphans, P.orphans.data(), P.orphans.size() * sizeof(AppendEntry));
    if (!P.items.empty()) memcpy(blob.data() + off->items, P.items.data(), P.items.size() * sizeof(AttnItem));
    if (!P.merges.empty()) memcpy(blob.data() + off->merges, P.merges.data(), P.merges.size() * sizeof(MergeItem));
    if (!P.pitems.empty()) memcpy(blob.data() + off->pitems, P.pitems.data(), P.pitems.size() * sizeof(AttnItem));
    if (!P.pmerges.empty())
        memcpy(blob.data() + off->pmerges, P.pmerges.data(), P.pmerges.size() * sizeof(MergeItem));
    if (!P.pseqs.empty()) memcpy(blob.data() + off->pseqs, P.pseqs.data(), P.pseqs.size() * sizeof(PrefillSeq));
    if (!P.table.empty()) memcpy(blob.data() + off->table, P.table.data(), P.table.size() * sizeof(uint32_t));
    if (!P.order.empty()) memcpy(blob.data() + off->order, P.order.data(), P.order.size() * sizeof(uint16_t));
    if (!P.porder.empty())
        memcpy(blob.data() + off->porder, P.porder.data(), P.porder.size() * sizeof(uint16_t));
    *ref = PlanRef{};
    if (kv->no_alloc) {
        // No staging slot (it would be allocated): the plan travels inline.
        if (off->total > kInlinePlanBytes)
            return kv->fail(NI_ERR_BAD_ARG,
                            "the step's plan is %zu bytes; ni_kv_step_noalloc passes plans of at most %u bytes "
                            "with the launch (fewer sequences or shorter contexts per call, or ni_kv_step)",
                            off->total, kInlinePlanBytes);
        ref->inl = blob.data();
        ref->inl_bytes = (uint32_t)off->total;
        return NI_OK;
    }
    if (off->total <= kInlinePlanBytes) {
        ref->inl = blob.data();
        ref->inl_bytes = (uint32_t)off->total;
        return NI_OK;
    }
    StagingSlot* sl = nullptr;
    int rc = acquire_slot(kv, off->total, &sl);
    if (rc) return rc;
    memcpy(sl->host, blob.data(), off->total);
    hipError_t e = hipMemcpyAsync(sl->dev, sl->host, off->total, hipMemcpyHostToDevice, kv->copy_stream);
    if (e != hipSuccess) return kv->hip_fail(e, "hipMemcpyAsync(plan)");
    e = hipEventRecord(sl->uploaded, kv->copy_stream);
    if (e != hipSuccess) return kv->hip_fail(e, "hipEventRecord(upload)");
    e = hipStreamWaitEvent(s, sl->uploaded, 0);
    if (e != hipSuccess) return kv->hip_fail(e, "hipStreamWaitEvent(upload)");
    ref->dev = sl->dev;
    ref->slot = sl;
    return NI_OK;
}

// After the launches that read a staged plan: mark its slot busy until they end.
int release_plan(ni_kv* kv, const PlanRef& ref, hipStream_t s) {
    if (!ref.slot) return NI_OK;
    hipError_t e = hipEventRecord(ref.slot->done, s);
    if (e != hipSuccess) return kv->hip_fail(e, "hipEventRecord(staging)");
    ref.slot->pending = true;
    return NI_OK;
}

// Append + attention + merge of layers layer0 .. layer0+n_lay-1 over plan P,
// already placed (off, ref).
int run_placed(ni_kv* kv, const Plan& P, const Offsets& off, const PlanRef& ref, uint32_t layer0, uint32_t n_lay,
               const float* k, const float* v, int64_t kv_row_stride, int64_t kv_layer_stride, const float* q,
               int64_t q_row_stride, int64_t q_layer_stride, float* out, int64_t out_row_stride,
               int64_t out_layer_stride, hipStream_t s) {
    const uint32_t D = kv->o.head_dim, H = kv->o.n_head;
    // Partials: the single-row/group launch's slots, then the prefill launch's.
    const size_t main_floats = (size_t)P.n_slots * n_lay * H * P.nq_tile * (D + 2);
    const size_t pre_floats = (size_t)P.n_pslots * n_lay * H * kPrefillRows * (D + 2);
    float* partials = nullptr;
    if (main_floats + pre_floats > 0) {
        int rc = ensure_partials(kv, (main_floats + pre_floats) * sizeof(float), s, &partials);
        if (rc) return rc;
    }
    if (!P.app.empty() && !P.fused && !P.seq_prefill) {
        AppendLaunch a;
        a.pool = kv->geom();
        a.k = k;
        a.v = v;
        a.row_stride = kv_row_stride;
        a.layer_stride = kv_layer_stride;
        a.plan = ref.dev;
        a.off_entries = (uint32_t)off.app;
        a.n_rows = (uint32_t)P.app.size();
        a.layer0 = layer0;
        a.n_lay = n_lay;
        ProfileScope ps(kv, NI_K_APPEND);
        hipError_t e = launch_append(a, ref.inl, ref.inl_bytes, s, ps.t);
        if (e != hipSuccess) return kv->hip_fail(e, "append kernel");
    }
    if (!P.items.empty() || !P.orphans.empty()) {
        AttnLaunch a{};
        a.pool = kv->geom();
        a.k = k;
        a.v = v;
        a.kv_row_stride = kv_row_stride;
        a.kv_layer_stride = kv_layer_stride;
        a.off_app = (uint32_t)off.app;
        a.off_orphans = (uint32_t)off.orphans;
        a.n_orphans = (uint32_t)P.orphans.size();
        a.napp_total = P.napp_total;
        a.q = q;
        a.q_row_stride = q_row_stride;
        a.q_layer_stride = q_layer_stride;
        a.out = out;
        a.out_row_stride = out_row_stride;
        a.out_layer_stride = out_layer_stride;
        a.plan = ref.dev;
        a.off_items = (uint32_t)off.items;
        a.off_table = (uint32_t)off.table;
        a.off_merges = (uint32_t)off.merges;
        a.partials = partials;
        a.n_items = (uint32_t)P.items.size();
        a.n_merges = (uint32_t)P.merges.size();
        a.layer0 = layer0;
        a.n_lay = n_lay;
        a.nq_tile = P.nq_tile;
        a.qscale = (float)(1.4426950408889634 / std::sqrt((double)D));
        a.wide = P.wide ? 1u : 0u;
        a.off_order = (uint32_t)off.order;
        a.ordered = P.order.empty() ? 0u : 1u;
        a.n_orphan_blocks = P.fused ? orphan_blocks(a) : 0;
        {
            ProfileScope ps(kv, NI_K_ATTN);
            hipError_t e = launch_attention(a, ref.inl, ref.inl_bytes, s, ps.t);
            if (e != hipSuccess) return kv->hip_fail(e, "attention kernel");
        }
        if (!P.merges.empty()) {
            a.merge_split = merge_split(P.merges, D);
            ProfileScope ps(kv, NI_K_MERGE);
            hipError_t e = launch_merge(a, ref.inl, ref.inl_bytes, s, ps.t);
            if (e != hipSuccess) return kv->hip_fail(e, "merge kernel");
        }
    }
    if (!P.pitems.empty()) {
        // Prefill groups: their own launch (after the append above), items,
        // merges and partials region; never fused.
        AttnLaunch a{};
        a.pool = kv->geom();
        a.q = q;
        a.q_row_stride = q_row_stride;
        a.q_layer_stride = q_layer_stride;
        a.out = out;
        a.out_row_stride = out_row_stride;
        a.out_layer_stride = out_layer_stride;
        a.plan = ref.dev;
        a.off_items = (uint32_t)off.pitems;
        a.off_table = (uint32_t)off.table;
        a.off_merges = (uint32_t)off.pmerges;
        a.partials = partials ? partials + main_floats : nullptr;
        a.n_items = (uint32_t)P.pitems.size();
        a.n_merges = (uint32_t)P.pmerges.size();
        a.layer0 = layer0;
        a.n_lay = n_lay;
        a.nq_tile = kPrefillRows;
        a.off_order = (uint32_t)off.porder;
        a.ordered = P.porder.empty() ? 0u : 1u;
        a.qscale = (float)(1.4426950408889634 / std::sqrt((double)D));
        if (P.seq_prefill) {  // the launch appends the rows too
            a.k = k;
            a.v = v;
            a.kv_row_stride = kv_row_stride;
            a.kv_layer_stride = kv_layer_stride;
            a.off_app = (uint32_t)off.app;
            a.off_pseqs = (uint32_t)off.pseqs;
            a.n_pseqs = (uint32_t)P.pseqs.size();
        }
        {
            ProfileScope ps(kv, NI_K_ATTN);
            hipError_t e = launch_attention(a, ref.inl, ref.inl_bytes, s, ps.t);
            if (e != hipSuccess) return kv->hip_fail(e, "prefill attention kernel");
        }
        if (!P.pmerges.empty()) {
            a.merge_split = merge_split(P.pmerges, D);
            ProfileScope ps(kv, NI_K_MERGE);
            hipError_t e = launch_merge(a, ref.inl, ref.inl_bytes, s, ps.t);
            if (e != hipSuccess) return kv->hip_fail(e, "prefill merge kernel");
        }
    }
    return NI_OK;
}

// Place kv->plan and run it over layers layer0 .. layer0+n_lay-1.
int run_plan(ni_kv* kv, uint32_t layer0, uint32_t n_lay, const float* k, const float* v, int64_t kv_row_stride,
             int64_t kv_layer_stride, const float* q, int64_t q_row_stride, int64_t q_layer_stride, float* out,
             int64_t out_row_stride, int64_t out_layer_stride, hipStream_t s) {
    Offsets off;
    PlanRef ref;
    int rc = place_plan(kv, kv->plan, kv->blob, s, &off, &ref);
    if (rc) return rc;
    rc = run_placed(kv, kv->plan, off, ref, layer0, n_lay, k, v, kv_row_stride, kv_layer_stride, q, q_row_stride,
                    q_layer_stride, out, out_row_stride, out_layer_stride, s);
    // Even after a failed launch: the slot is reused only once this point
    // of the stream is reached.
    int rc2 = release_plan(kv, ref, s);
    return rc ? rc : rc2;
}

void reset_plan(ni_kv* kv) {
    kv->plan.clear();
    kv->qrows.clear();
}

}  // namespace

static int enqueue_step(ni_kv* kv, const ni_work* work, uint32_t n_work, const float* q, const float* k,
                        const float* v, int64_t row_stride, int64_t layer_stride, float* out, int64_t out_row_stride,
                        int64_t out_layer_stride, uint32_t split_tokens, hipStream_t stream);
static int prepare_step(ni_kv* kv, const ni_work* work, uint32_t n_work);
static int build_step_plan(ni_kv* kv, const ni_work* work, uint32_t n_work, uint32_t split_tokens, uint32_t n_lay);

// ============================================================= C ABI

extern "C" {

const char* ni_version(void) { return "nanoinfer-amd 0.1 (gfx950 paged f16 KV)"; }

const char* ni_kv_last_error(const ni_kv* kv) { return kv ? kv->err.c_str() : g_create_error.c_str(); }

int ni_kv_create(const ni_kv_opts* opts, ni_kv** out) {
    if (!out) return NI_ERR_BAD_ARG;
    *out = nullptr;
    if (!opts) {
        g_create_error = "opts is NULL";
        return NI_ERR_BAD_ARG;
    }
    const ni_kv_opts& o = *opts;
    const uint64_t C = (uint64_t)o.n_head * o.head_dim;
    if (o.n_layer == 0 || o.n_head == 0 || o.head_dim == 0 || o.kv_pages == 0 || o.max_seqs == 0 || o.max_ctx == 0 ||
        o.max_rows == 0 || o.head_dim % 8 != 0) {
        g_create_error = "n_layer, n_head, kv_pages, max_seqs, max_ctx and max_rows must be > 0; head_dim a multiple of 8";
        return NI_ERR_BAD_ARG;
    }
    if (o.flags & ~(NI_KV_HOST_ONLY | NI_KV_Q8)) {
        g_create_error = "unknown flags";
        return NI_ERR_BAD_ARG;
    }
    const bool host_only = (o.flags & NI_KV_HOST_ONLY) != 0;
    if (!host_only && !attention_supported(o.head_dim)) {
        g_create_error = "head_dim " + std::to_string(o.head_dim) + " unsupported on the device (64 or 128)";
        return NI_ERR_BAD_ARG;
    }
    // 32-bit index limits of the append/gather grids.
    if ((uint64_t)o.n_layer * o.max_rows * 2 * (C / 8) >= (1ull << 31)) {
        g_create_error = "n_layer * max_rows * C too large";
        return NI_ERR_BAD_ARG;
    }
    ni_kv* kv = new ni_kv();
    kv->o = o;
    kv->o.page_order = nullptr;
    kv->host_only = host_only;
    kv->max_pages = (o.max_ctx + kPage - 1) / kPage;
    kv->seq_len.assign(o.max_seqs, 0);
    kv->live.assign(o.max_seqs, 0);
    kv->pages.assign(o.max_seqs, {});
    kv->seq_tab.assign(o.max_seqs, -1);
    kv->seq_need.assign(o.max_seqs, 0);
    kv->step_mark.assign(o.max_seqs, 0);
    // batch.rs:174: (0..kv_blocks).rev() so that pop() yields 0, 1, 2, ...
    kv->free_pages.resize(o.kv_pages);
    if (o.page_order) {
        std::vector<uint8_t> seen(o.kv_pages, 0);
        for (uint32_t i = 0; i < o.kv_pages; i++) {
            const uint32_t p = o.page_order[i];
            if (p >= o.kv_pages || seen[p]) {
                g_create_error = "page_order must be a permutation of 0..kv_pages-1";
                delete kv;
                return NI_ERR_BAD_ARG;
            }
            seen[p] = 1;
            kv->free_pages[o.kv_pages - 1 - i] = p;
        }
    } else {
        for (uint32_t i = 0; i < o.kv_pages; i++) kv->free_pages[i] = o.kv_pages - 1 - i;
    }
    if (!host_only) {
        hipError_t e = hipGetDevice(&kv->device);
        if (e == hipSuccess) {
            // One allocation, [n_layer][kv_pages][n_head][K|V block]: a
            // (page, head) holds its K block and then its V block.  f16: a
            // block is [16][head_dim] halves.  Q8: [16][head_dim] int8 then
            // 16 f32 scales, 16 * head_dim + 64 bytes (kv_block_halves()).
            const uint64_t block = kv_block_halves(o);
            kv->head_halves = (uint32_t)(2 * block);
            kv->page_halves = 2 * block * o.n_head;
            kv->layer_halves = kv->page_halves * o.kv_pages;
            kv->pool_bytes = (size_t)(kv->layer_halves * o.n_layer * sizeof(uint16_t));
            e = hipMalloc(reinterpret_cast<void**>(&kv->kpool), kv->pool_bytes);
            if (e == hipSuccess) kv->vpool = kv->kpool + block;
        }
        // Zero pages: a page that was never written reads as finite zeros.
        if (e == hipSuccess) e = hipMemset(kv->kpool, 0, kv->pool_bytes);
        for (uint32_t i = 0; e == hipSuccess && i < kRingSlots; i++) {
            e = hipEventCreateWithFlags(&kv->ring[i].done, hipEventDisableTiming);
            if (e == hipSuccess) e = hipEventCreateWithFlags(&kv->ring[i].uploaded, hipEventDisableTiming);
        }
        if (e == hipSuccess) e = hipEventCreateWithFlags(&kv->order, hipEventDisableTiming);
        // Default priority: the copy stream only moves plans.
        if (e == hipSuccess) e = hipStreamCreateWithFlags(&kv->copy_stream, hipStreamNonBlocking);
        // The no-allocation entry point's scratch on this device (a failure
        // here disables only that entry point).
        if (e == hipSuccess) {
            void* p = nullptr;
            kv->scratch_err = scratch_address(&p);
            kv->scratch = kv->scratch_err == hipSuccess ? static_cast<float*>(p) : nullptr;
        }
        if (e != hipSuccess) {
            g_create_error = std::string("device setup failed: ") + hipGetErrorString(e);
            ni_kv_destroy(kv);
            return NI_ERR_HIP;
        }
    }
    *out = kv;
    return NI_OK;
}

void ni_kv_destroy(ni_kv* kv) {
    if (!kv) return;
    if (!kv->host_only) {
        for (auto& sl : kv->ring)
            if (sl.pending) (void)hipEventSynchronize(sl.done);
        (void)hipDeviceSynchronize();
        for (auto& sl : kv->ring) {
            if (sl.host) (void)hipHostFree(sl.host);
            if (sl.dev) (void)hipFree(sl.dev);
            if (sl.done) (void)hipEventDestroy(sl.done);
            if (sl.uploaded) (void)hipEventDestroy(sl.uploaded);
        }
        for (auto& v : kv->prof_ev)
            for (auto& pr : v) {
                (void)hipEventDestroy(pr.first);
                (void)hipEventDestroy(pr.second);
            }
        for (hipEvent_t e : kv->ev_pool) (void)hipEventDestroy(e);
        if (kv->order) (void)hipEventDestroy(kv->order);
        if (kv->partials) (void)hipFree(kv->partials);
        for (auto& pr : kv->partials_retired) {
            (void)hipFree(pr.first);
            (void)hipEventDestroy(pr.second);
        }
        if (kv->kpool) (void)hipFree(kv->kpool);
        if (kv->copy_stream) (void)hipStreamDestroy(kv->copy_stream);
        release_scratch(kv, kv->device);
    }
    delete kv;
}

size_t ni_kv_page_bytes(const ni_kv* kv) {
    return kv ? (size_t)2 * kv->o.n_layer * kv->o.n_head * kv_block_halves(kv->o) * 2 : 0;
}

int ni_kv_add_seq(ni_kv* kv, uint32_t* seq) {
    if (!kv || !seq) return NI_ERR_BAD_ARG;
    for (uint32_t s = 0; s < kv->o.max_seqs; s++) {
        if (!kv->live[s]) {
            kv->live[s] = 1;
            kv->seq_len[s] = 0;
            *seq = s;
            return NI_OK;
        }
    }
    return kv->fail(NI_ERR_NO_SLOT, "no sequence slot");
}

int ni_kv_free_seq(ni_kv* kv, uint32_t s) {
    if (!kv) return NI_ERR_BAD_ARG;
    if (kv->step.open) return kv->fail(NI_ERR_BAD_ARG, "a step begun by ni_kv_step_begin is still open");
    if (int rc = check_seq(kv, s)) return rc;
    truncate_seq(kv, s, 0);
    kv->live[s] = 0;
    return NI_OK;
}

int ni_kv_seq_len(const ni_kv* kv, uint32_t s, uint32_t* len) {
    if (!kv || !len) return NI_ERR_BAD_ARG;
    if (s >= kv->o.max_seqs) return NI_ERR_BAD_ARG;
    *len = kv->seq_len[s];
    return NI_OK;
}

int ni_kv_is_live(const ni_kv* kv, uint32_t s, int* live) {
    if (!kv || !live) return NI_ERR_BAD_ARG;
    if (s >= kv->o.max_seqs) return NI_ERR_BAD_ARG;
    *live = kv->live[s] ? 1 : 0;
    return NI_OK;
}

int ni_kv_truncate(ni_kv* kv, uint32_t s, uint32_t len) {
    if (!kv) return NI_ERR_BAD_ARG;
    if (kv->step.open) return kv->fail(NI_ERR_BAD_ARG, "a step begun by ni_kv_step_begin is still open");
    if (int rc = check_seq(kv, s)) return rc;
    return truncate_seq(kv, s, len);
}

int ni_kv_reserve(ni_kv* kv, uint32_t s, uint32_t len) {
    if (!kv) return NI_ERR_BAD_ARG;
    if (int rc = check_seq(kv, s)) return rc;
    if (!kv->live[s]) return kv->fail(NI_ERR_NOT_LIVE, "sequence %u is not live", s);
    return ensure_pages(kv, s, len);
}

int ni_kv_commit(ni_kv* kv, uint32_t s, uint32_t n) {
    if (!kv) return NI_ERR_BAD_ARG;
    if (kv->step.open) return kv->fail(NI_ERR_BAD_ARG, "a step begun by ni_kv_step_begin is still open");
    if (int rc = check_seq(kv, s)) return rc;
    if (!kv->live[s]) return kv->fail(NI_ERR_NOT_LIVE, "sequence %u is not live", s);
    const uint64_t len = (uint64_t)kv->seq_len[s] + n;
    if (len > (uint64_t)kv->pages[s].size() * kPage)
        return kv->fail(NI_ERR_NOT_RESERVED, "sequence %u: commit to %llu past reserved %zu", s,
                        (unsigned long long)len, kv->pages[s].size() * kPage);
    kv->seq_len[s] = (uint32_t)len;
    return NI_OK;
}

int ni_kv_block_table(const ni_kv* kv, uint32_t s, const uint32_t** pages, uint32_t* n) {
    if (!kv || !pages || !n) return NI_ERR_BAD_ARG;
    if (s >= kv->o.max_seqs) return NI_ERR_BAD_ARG;
    *pages = kv->pages[s].data();
    *n = (uint32_t)kv->pages[s].size();
    return NI_OK;
}

uint32_t ni_kv_blocks_used(const ni_kv* kv) { return kv ? kv->o.kv_pages - (uint32_t)kv->free_pages.size() : 0; }

uint32_t ni_kv_free_block_count(const ni_kv* kv) { return kv ? (uint32_t)kv->free_pages.size() : 0; }

int ni_kv_pools(const ni_kv* kv, void** k_pool, void** v_pool, size_t* bytes) {
    if (!kv) return NI_ERR_BAD_ARG;
    if (k_pool) *k_pool = kv->kpool;
    if (v_pool) *v_pool = kv->vpool;
    if (bytes) *bytes = kv->pool_bytes;
    return NI_OK;
}

int ni_kv_append(ni_kv* kv, int32_t layer, const ni_row* rows, uint32_t n, const float* k, const float* v,
                 int64_t row_stride, int64_t layer_stride, ni_stream stream) {
    if (!kv) return NI_ERR_BAD_ARG;
    if (kv->host_only) return kv->fail(NI_ERR_NO_DEVICE, "host-only handle has no device pools");
    uint32_t layer0, n_lay;
    if (int rc = layer_range(kv, layer, &layer0, &n_lay)) return rc;
    if (n == 0) return NI_OK;
    if (!rows) return kv->fail(NI_ERR_BAD_ARG, "rows is NULL");
    if (n > kv->o.max_rows) return kv->fail(NI_ERR_TOO_MANY_ROWS, "%u rows > max_rows %u", n, kv->o.max_rows);
    const bool all = layer == NI_ALL_LAYERS;
    if (int rc = check_f32_operand(kv, "k", k, row_stride, layer_stride, all)) return rc;
    if (int rc = check_f32_operand(kv, "v", v, row_stride, layer_stride, all)) return rc;
    reset_plan(kv);
    for (uint32_t i = 0; i < n; i++) {
        if (int rc = check_row(kv, rows[i])) return rc;
        const ni_row& r = rows[i];
        kv->plan.app.push_back({i, kv->pages[r.seq][r.pos / kPage], r.pos % kPage, 0});
    }
    return run_plan(kv, layer0, n_lay, k, v, row_stride, all ? layer_stride : 0, nullptr, 0, 0, nullptr, 0, 0,
                    (hipStream_t)stream);
}

// Shared checks and launch of the QKV projection; rows == NULL: plain.
static int qkv_run(ni_kv* kv, int32_t layer, const ni_row* rows, uint32_t n, const float* x, int64_t x_row_stride,
                   uint32_t d_in, const void* w, uint32_t wfmt, const float* bias, float* out, int64_t out_row_stride,
                   hipStream_t s) {
    if (!kv) return NI_ERR_BAD_ARG;
    if (kv->host_only) return kv->fail(NI_ERR_NO_DEVICE, "host-only handle has no device pools");
    const bool fused = rows != nullptr;
    if (fused && is_q8(kv->o))
        return kv->fail(NI_ERR_BAD_ARG, "Q8 cache: project with ni_kv_qkv_project and append with ni_kv_append");
    const uint32_t C = kv->o.n_head * kv->o.head_dim, n_feat = 3 * C;
    if (fused && (layer < 0 || (uint32_t)layer >= kv->o.n_layer))
        return kv->fail(NI_ERR_BAD_ARG, "layer %d out of range (%u layers)", layer, kv->o.n_layer);
    if (n == 0) return NI_OK;
    if (n > kv->o.max_rows) return kv->fail(NI_ERR_TOO_MANY_ROWS, "%u rows > max_rows %u", n, kv->o.max_rows);
    if (wfmt > NI_W_Q4_0) return kv->fail(NI_ERR_BAD_ARG, "unknown weight format %u", wfmt);
    const uint32_t k_mult = wfmt >= NI_W_Q8_0 ? 32u : kQkvK;  // block formats: whole blocks per row
    if (d_in == 0 || d_in % k_mult != 0)
        return kv->fail(NI_ERR_BAD_ARG, "d_in %u must be a positive multiple of %u", d_in, k_mult);
    if (n_feat % kQkvTileFeat != 0)
        return kv->fail(NI_ERR_BAD_ARG, "3 * n_head * head_dim = %u must be a multiple of %u", n_feat, kQkvTileFeat);
    if (int rc = check_f32_operand(kv, "x", x, x_row_stride, 0, false)) return rc;
    if (x_row_stride < (int64_t)d_in) return kv->fail(NI_ERR_BAD_ARG, "x row stride %lld < d_in %u", (long long)x_row_stride, d_in);
    if (!w || !aligned16(w)) return kv->fail(NI_ERR_BAD_ARG, "w must be a 16-byte aligned [3C][d_in] weight matrix");
    if (bias && (reinterpret_cast<uintptr_t>(bias) & 3u)) return kv->fail(NI_ERR_BAD_ARG, "bias must be 4-byte aligned");
    if (int rc = check_f32_operand(kv, fused ? "q_out" : "out", out, out_row_stride, 0, false)) return rc;
    if (out_row_stride < (int64_t)(fused ? C : n_feat))
        return kv->fail(NI_ERR_BAD_ARG, "output row stride %lld < %u", (long long)out_row_stride, fused ? C : n_feat);
    reset_plan(kv);
    if (fused)
        for (uint32_t i = 0; i < n; i++) {
            if (int rc = check_row(kv, rows[i])) return rc;
            const ni_row& r = rows[i];
            kv->plan.app.push_back({i, kv->pages[r.seq][r.pos / kPage], r.pos % kPage, 0});
        }
    Offsets off;
    PlanRef ref;
    if (int rc = place_plan(kv, kv->plan, kv->blob, s, &off, &ref)) return rc;
    QkvLaunch q;
    q.pool = kv->geom();
    q.x = x;
    q.x_row_stride = x_row_stride;
    q.w = w;
    q.wfmt = wfmt;
    q.bias = bias;
    q.out = out;
    q.out_row_stride = out_row_stride;
    q.plan = ref.dev;
    q.off_entries = (uint32_t)off.app;
    q.n_rows = n;
    q.d_in = d_in;
    q.n_feat = n_feat;
    q.layer = fused ? (uint32_t)layer : 0u;
    q.fused = fused;
    {
        ProfileScope ps(kv, NI_K_QKV);
        hipError_t e = launch_qkv(q, ref.inl, ref.inl_bytes, s, ps.t);
        if (e != hipSuccess) return kv->hip_fail(e, "qkv kernel");
    }
    return release_plan(kv, ref, s);
}

int ni_kv_qkv_append_w(ni_kv* kv, int32_t layer, const ni_row* rows, uint32_t n, const float* x,
                       int64_t x_row_stride, uint32_t d_in, const void* w, uint32_t w_format, const float* bias,
                       float* q_out, int64_t q_row_stride, ni_stream stream) {
    if (kv && n && !rows) return kv->fail(NI_ERR_BAD_ARG, "rows is NULL");
    static const ni_row none{0, 0};
    return qkv_run(kv, layer, rows ? rows : &none, n, x, x_row_stride, d_in, w, w_format, bias, q_out, q_row_stride,
                   (hipStream_t)stream);
}

int ni_kv_qkv_project_w(ni_kv* kv, const float* x, int64_t x_row_stride, uint32_t n, uint32_t d_in, const void* w,
                        uint32_t w_format, const float* bias, float* out, int64_t out_row_stride, ni_stream stream) {
    return qkv_run(kv, 0, nullptr, n, x, x_row_stride, d_in, w, w_format, bias, out, out_row_stride,
                   (hipStream_t)stream);
}

int ni_kv_qkv_append(ni_kv* kv, int32_t layer, const ni_row* rows, uint32_t n, const float* x,
                     int64_t x_row_stride, uint32_t d_in, const float* w, const float* bias, float* q_out,
                     int64_t q_row_stride, ni_stream stream) {
    return ni_kv_qkv_append_w(kv, layer, rows, n, x, x_row_stride, d_in, w, NI_W_F32, bias, q_out, q_row_stride,
                              stream);
}

int ni_kv_qkv_project(ni_kv* kv, const float* x, int64_t x_row_stride, uint32_t n, uint32_t d_in, const float* w,
                      const float* bias, float* out, int64_t out_row_stride, ni_stream stream) {
    return ni_kv_qkv_project_w(kv, x, x_row_stride, n, d_in, w, NI_W_F32, bias, out, out_row_stride, stream);
}

int ni_kv_gather(ni_kv* kv, int32_t layer, const ni_row* rows, uint32_t n, uint16_t* k_out, uint16_t* v_out,
                 int64_t row_stride, int64_t layer_stride, ni_stream stream) {
    if (!kv) return NI_ERR_BAD_ARG;
    if (kv->host_only) return kv->fail(NI_ERR_NO_DEVICE, "host-only handle has no device pools");
    uint32_t layer0, n_lay;
    if (int rc = layer_range(kv, layer, &layer0, &n_lay)) return rc;
    if (n == 0) return NI_OK;
    if (!rows) return kv->fail(NI_ERR_BAD_ARG, "rows is NULL");
    if (n > kv->o.max_rows) return kv->fail(NI_ERR_TOO_MANY_ROWS, "%u rows > max_rows %u", n, kv->o.max_rows);
    if (is_q8(kv->o)) return kv->fail(NI_ERR_BAD_ARG, "Q8 cache: use ni_kv_gather_q8");
    const bool all = layer == NI_ALL_LAYERS;
    if (!k_out || !v_out || !aligned16(k_out) || !aligned16(v_out) || row_stride % 8 != 0 || row_stride < 0 ||
        (all && (layer_stride % 8 != 0 || layer_stride < 0)))
        return kv->fail(NI_ERR_BAD_ARG, "k_out/v_out must be 16-byte aligned with strides that are multiples of 8");
    reset_plan(kv);
    for (uint32_t i = 0; i < n; i++) {
        if (int rc = check_row(kv, rows[i])) return rc;
        const ni_row& r = rows[i];
        kv->plan.app.push_back({i, kv->pages[r.seq][r.pos / kPage], r.pos % kPage, 0});
    }
    Offsets off;
    PlanRef ref;
    hipStream_t s = (hipStream_t)stream;
    if (int rc = place_plan(kv, kv->plan, kv->blob, s, &off, &ref)) return rc;
    GatherLaunch g;
    g.pool = kv->geom();
    g.k_out = k_out;
    g.v_out = v_out;
    g.row_stride = row_stride;
    g.layer_stride = all ? layer_stride : 0;
    g.plan = ref.dev;
    g.off_entries = (uint32_t)off.app;
    g.n_rows = n;
    g.layer0 = layer0;
    g.n_lay = n_lay;
    hipError_t e = launch_gather(g, ref.inl, ref.inl_bytes, s);
    if (e != hipSuccess) return kv->hip_fail(e, "gather kernel");
    return release_plan(kv, ref, s);
}

int ni_kv_gather_q8(ni_kv* kv, int32_t layer, const ni_row* rows, uint32_t n, int8_t* k_out, int8_t* v_out,
                    float* k_scale, float* v_scale, ni_stream stream) {
    if (!kv) return NI_ERR_BAD_ARG;
    if (kv->host_only) return kv->fail(NI_ERR_NO_DEVICE, "host-only handle has no device pools");
    if (!is_q8(kv->o)) return kv->fail(NI_ERR_BAD_ARG, "not a Q8 cache: use ni_kv_gather");
    uint32_t layer0, n_lay;
    if (int rc = layer_range(kv, layer, &layer0, &n_lay)) return rc;
    if (n == 0) return NI_OK;
    if (!rows) return kv->fail(NI_ERR_BAD_ARG, "rows is NULL");
    if (n > kv->o.max_rows) return kv->fail(NI_ERR_TOO_MANY_ROWS, "%u rows > max_rows %u", n, kv->o.max_rows);
    if (!k_out || !v_out || !k_scale || !v_scale || !aligned16(k_out) || !aligned16(v_out) ||
        (reinterpret_cast<uintptr_t>(k_scale) & 3u) || (reinterpret_cast<uintptr_t>(v_scale) & 3u))
        return kv->fail(NI_ERR_BAD_ARG, "k_out/v_out must be 16-byte aligned, scales 4-byte aligned");
    reset_plan(kv);
    for (uint32_t i = 0; i < n; i++) {
        if (int rc = check_row(kv, rows[i])) return rc;
        const ni_row& r = rows[i];
        kv->plan.app.push_back({i, kv->pages[r.seq][r.pos / kPage], r.pos % kPage, 0});
    }
    Offsets off;
    PlanRef ref;
    hipStream_t s = (hipStream_t)stream;
    if (int rc = place_plan(kv, kv->plan, kv->blob, s, &off, &ref)) return rc;
    GatherQ8Launch g;
    g.pool = kv->geom();
    g.k_out = k_out;
    g.v_out = v_out;
    g.k_scale = k_scale;
    g.v_scale = v_scale;
    g.plan = ref.dev;
    g.off_entries = (uint32_t)off.app;
    g.n_rows = n;
    g.layer0 = layer0;
    g.n_lay = n_lay;
    hipError_t e = launch_gather_q8(g, ref.inl, ref.inl_bytes, s);
    if (e != hipSuccess) return kv->hip_fail(e, "gather kernel");
    return release_plan(kv, ref, s);
}

int ni_paged_decode_attention(ni_kv* kv, int32_t layer, const float* q, int64_t q_row_stride,
                              int64_t q_layer_stride, const ni_row* rows, uint32_t n, float* out,
                              int64_t out_row_stride, int64_t out_layer_stride, uint32_t split_tokens,
                              ni_stream stream) {
    if (!kv) return NI_ERR_BAD_ARG;
    if (kv->host_only) return kv->fail(NI_ERR_NO_DEVICE, "host-only handle has no device pools");
    uint32_t layer0, n_lay;
    if (int rc = layer_range(kv, layer, &layer0, &n_lay)) return rc;
    if (n == 0) return NI_OK;
    if (!rows) return kv->fail(NI_ERR_BAD_ARG, "rows is NULL");
    if (n > kv->o.max_rows) return kv->fail(NI_ERR_TOO_MANY_ROWS, "%u rows > max_rows %u", n, kv->o.max_rows);
    const bool all = layer == NI_ALL_LAYERS;
    if (int rc = check_f32_operand(kv, "q", q, q_row_stride, q_layer_stride, all)) return rc;
    if (int rc = check_f32_operand(kv, "out", out, out_row_stride, out_layer_stride, all)) return rc;
    reset_plan(kv);
    for (uint32_t i = 0; i < n; i++) {
        if (int rc = check_row(kv, rows[i])) return rc;
        kv->qrows.push_back({i, rows[i].seq, rows[i].pos, 0, 0, 0});
    }
    if (int rc = plan_attention(kv, split_tokens, n_lay)) return rc;
    return run_plan(kv, layer0, n_lay, nullptr, nullptr, 0, 0, q, q_row_stride, all ? q_layer_stride : 0, out,
                    out_row_stride, all ? out_layer_stride : 0, (hipStream_t)stream);
}

int ni_kv_step(ni_kv* kv, const ni_work* work, uint32_t n_work, const float* q, const float* k, const float* v,
               int64_t row_stride, int64_t layer_stride, float* out, int64_t out_row_stride,
               int64_t out_layer_stride, uint32_t split_tokens, ni_stream stream) {
    if (!kv) return NI_ERR_BAD_ARG;
    if (kv->host_only) return kv->fail(NI_ERR_NO_DEVICE, "host-only handle has no device pools");
    if (n_work == 0) return NI_OK;
    if (!work) return kv->fail(NI_ERR_BAD_ARG, "work is NULL");
    if (int rc = check_f32_operand(kv, "k", k, row_stride, layer_stride, true)) return rc;
    if (int rc = check_f32_operand(kv, "v", v, row_stride, layer_stride, true)) return rc;
    bool any_query = false;
    for (uint32_t w = 0; w < n_work; w++) any_query |= work[w].n_query > 0;
    if (any_query) {
        if (int rc = check_f32_operand(kv, "q", q, row_stride, layer_stride, true)) return rc;
        if (int rc = check_f32_operand(kv, "out", out, out_row_stride, out_layer_stride, true)) return rc;
    }
    if (kv->step.open) return kv->fail(NI_ERR_BAD_ARG, "a step begun by ni_kv_step_begin is still open");
    if (int rc = prepare_step(kv, work, n_work)) return rc;
    return enqueue_step(kv, work, n_work, q, k, v, row_stride, layer_stride, out, out_row_stride, out_layer_stride,
                        split_tokens, (hipStream_t)stream);
}

int ni_kv_step_noalloc(ni_kv* kv, const ni_work* work, uint32_t n_work, const float* q, const float* k,
                       const float* v, int64_t row_stride, int64_t layer_stride, float* out, int64_t out_row_stride,
                       int64_t out_layer_stride, uint32_t split_tokens, ni_stream stream) {
    if (!kv) return NI_ERR_BAD_ARG;
    if (kv->host_only) return kv->fail(NI_ERR_NO_DEVICE, "host-only handle has no device pools");
    if (!kv->scratch)
        return kv->fail(NI_ERR_HIP, "ni_kv_step_noalloc: no scratch on this device (hipGetSymbolAddress: %s)",
                        hipGetErrorString(kv->scratch_err));
    if (!claim_scratch(kv, kv->device))
        return kv->fail(NI_ERR_BAD_ARG,
                        "ni_kv_step_noalloc: device %d's scratch array is held by another handle (the first handle "
                        "to call this entry point on a GPU holds it until ni_kv_destroy)",
                        kv->device);
    struct Scope {
        ni_kv* kv;
        explicit Scope(ni_kv* k_) : kv(k_) { kv->no_alloc = true; }
        ~Scope() { kv->no_alloc = false; }
    } scope(kv);
    return ni_kv_step(kv, work, n_work, q, k, v, row_stride, layer_stride, out, out_row_stride, out_layer_stride,
                      split_tokens, stream);
}

int ni_kv_step_begin(ni_kv* kv, const ni_work* work, uint32_t n_work, uint32_t split_tokens) {
    if (!kv) return NI_ERR_BAD_ARG;
    if (kv->step.open) return kv->fail(NI_ERR_BAD_ARG, "a step is already open");
    if (n_work && !work) return kv->fail(NI_ERR_BAD_ARG, "work is NULL");
    if (int rc = prepare_step(kv, work, n_work)) return rc;
    // Partitions and launch shape for one layer per launch.
    if (int rc = build_step_plan(kv, work, n_work, split_tokens, 1)) return rc;
    auto& st = kv->step;
    std::swap(st.plan, kv->plan);
    kv->plan.clear();
    st.commit.clear();
    for (uint32_t w = 0; w < n_work; w++) st.commit.push_back({work[w].seq, work[w].n_new});
    st.placed = false;
    st.ref = PlanRef{};
    st.stream = nullptr;
    st.open = true;
    return NI_OK;
}

int ni_kv_step_layer(ni_kv* kv, int32_t layer, const float* q, const float* k, const float* v, int64_t row_stride,
                     float* out, int64_t out_row_stride, ni_stream stream) {
    if (!kv) return NI_ERR_BAD_ARG;
    auto& st = kv->step;
    if (!st.open) return kv->fail(NI_ERR_BAD_ARG, "no step is open (ni_kv_step_begin)");
    if (kv->host_only) return kv->fail(NI_ERR_NO_DEVICE, "host-only handle has no device pools");
    if (layer < 0 || (uint32_t)layer >= kv->o.n_layer)
        return kv->fail(NI_ERR_BAD_ARG, "layer %d out of range (one layer per call)", layer);
    const Plan& P = st.plan;
    if (!P.app.empty()) {
        if (int rc = check_f32_operand(kv, "k", k, row_stride, 0, false)) return rc;
        if (int rc = check_f32_operand(kv, "v", v, row_stride, 0, false)) return rc;
    }
    if (!P.items.empty() || !P.pitems.empty()) {
        if (int rc = check_f32_operand(kv, "q", q, row_stride, 0, false)) return rc;
        if (int rc = check_f32_operand(kv, "out", out, out_row_stride, 0, false)) return rc;
    }
    const hipStream_t s = (hipStream_t)stream;
    // Every layer's launch uses the step's one set of split partials and its
    // one staged plan, so the layers of a step run in order on one stream.
    if (st.placed && s != st.stream)
        return kv->fail(NI_ERR_BAD_ARG, "every layer of a step must run on the stream of its first layer");
    if (!st.placed) {
        if (int rc = place_plan(kv, P, st.blob, s, &st.off, &st.ref)) return rc;
        if (st.ref.slot) st.ref.slot->held = true;
        st.placed = true;
        st.stream = s;
    } else if (int rc = begin_call(kv, s)) {  // (calls on other streams may have come between the layers)
        return rc;
    }
    return run_placed(kv, P, st.off, st.ref, (uint32_t)layer, 1, k, v, row_stride, 0, q, row_stride, 0, out,
                      out_row_stride, 0, s);
}

int ni_kv_step_end(ni_kv* kv) {
    if (!kv) return NI_ERR_BAD_ARG;
    auto& st = kv->step;
    if (!st.open) return kv->fail(NI_ERR_BAD_ARG, "no step is open (ni_kv_step_begin)");
    st.open = false;
    int rc = NI_OK;
    if (st.placed) rc = release_plan(kv, st.ref, st.stream);
    if (st.ref.slot) st.ref.slot->held = false;
    st.placed = false;
    st.ref = PlanRef{};
    // batch.rs:270: the step's rows now belong to their sequences.
    for (const auto& c : st.commit) kv->seq_len[c.first] += c.second;
    st.commit.clear();
    st.plan.clear();
    return rc;
}

int ni_kv_decode_steps(ni_kv* kv, const uint32_t* seqs, uint32_t n, uint32_t steps, const float* q, const float* k,
                       const float* v, int64_t row_stride, int64_t layer_stride, int64_t step_stride, float* out,
                       int64_t out_row_stride, int64_t out_layer_stride, int64_t out_step_stride,
                       uint32_t split_tokens, ni_stream stream) {
    if (!kv) return NI_ERR_BAD_ARG;
    if (kv->step.open) return kv->fail(NI_ERR_BAD_ARG, "a step begun by ni_kv_step_begin is still open");
    if (kv->host_only) return kv->fail(NI_ERR_NO_DEVICE, "host-only handle has no device pools");
    if (n == 0 || steps == 0) return NI_OK;
    if (!seqs) return kv->fail(NI_ERR_BAD_ARG, "seqs is NULL");
    // batch.rs:335-337
    if (n > kv->o.max_rows) return kv->fail(NI_ERR_TOO_MANY_ROWS, "batch %u too large", n);
    if (step_stride % 4 || out_step_stride % 4)
        return kv->fail(NI_ERR_BAD_ARG, "step strides must be multiples of 4 floats");
    for (const char* name : {"q", "k", "v", "out"}) {
        const bool is_out = name[0] == 'o';
        const void* p = name[0] == 'q' ? (const void*)q : name[0] == 'k' ? (const void*)k
                      : name[0] == 'v' ? (const void*)v : (const void*)out;
        if (int rc = check_f32_operand(kv, name, p, is_out ? out_row_stride : row_stride,
                                       is_out ? out_layer_stride : layer_stride, true))
            return rc;
    }
    if (++kv->step_stamp == 0) {
        std::fill(kv->step_mark.begin(), kv->step_mark.end(), 0u);
        kv->step_stamp = 1;
    }
    // batch.rs:341-349: every sequence's pages for all steps first; an error
    // leaves earlier sequences' pages reserved, as the reference does.
    for (uint32_t i = 0; i < n; i++) {
        const uint32_t s = seqs[i];
        if (int rc = check_seq(kv, s)) return rc;
        if (!kv->live[s]) return kv->fail(NI_ERR_NOT_LIVE, "sequence %u is not live", s);
        if (kv->step_mark[s] == kv->step_stamp)
            return kv->fail(NI_ERR_BAD_ARG, "sequence %u appears twice in one call", s);
        kv->step_mark[s] = kv->step_stamp;
        if (int rc = ensure_pages(kv, s, (uint64_t)kv->seq_len[s] + steps)) return rc;
    }
    // batch.rs:351-357: every step enqueued at once; step t appends and
    // attends position seq_len + t of each sequence.
    std::vector<ni_work> work(n);
    for (uint32_t i = 0; i < n; i++) work[i] = ni_work{seqs[i], 1, 1};
    for (uint32_t t = 0; t < steps; t++) {
        const int64_t o = (int64_t)t * step_stride, oo = (int64_t)t * out_step_stride;
        if (int rc = enqueue_step(kv, work.data(), n, q + o, k + o, v + o, row_stride, layer_stride, out + oo,
                                  out_row_stride, out_layer_stride, split_tokens, (hipStream_t)stream))
            return rc;
    }
    return NI_OK;
}

}  // extern "C"

// The launch half of ni_kv_step: lay out the validated, reserved work's rows,
// plan, launch, and commit seq_len += n_new (batch.rs:270).
// Batch::encode_step (batch.rs:280-305): check each item, grow its pages.
static int prepare_step(ni_kv* kv, const ni_work* work, uint32_t n_work) {
    if (++kv->step_stamp == 0) {  // stamps wrapped: forget every old mark
        std::fill(kv->step_mark.begin(), kv->step_mark.end(), 0u);
        kv->step_stamp = 1;
    }
    uint64_t n_rows = 0;
    for (uint32_t w = 0; w < n_work; w++) {
        const ni_work& it = work[w];
        if (int rc = check_seq(kv, it.seq)) return rc;
        if (!kv->live[it.seq]) return kv->fail(NI_ERR_NOT_LIVE, "sequence %u is not live", it.seq);
        if (it.n_new == 0) return kv->fail(NI_ERR_EMPTY_WORK, "empty work item");
        if (it.n_query > it.n_new)
            return kv->fail(NI_ERR_BAD_ARG, "work item %u: n_query %u > n_new %u", w, it.n_query, it.n_new);
        if (kv->step_mark[it.seq] == kv->step_stamp)
            return kv->fail(NI_ERR_BAD_ARG, "sequence %u appears twice in one step", it.seq);
        kv->step_mark[it.seq] = kv->step_stamp;
        const uint32_t len = kv->seq_len[it.seq];
        if (int rc = ensure_pages(kv, it.seq, (uint64_t)len + it.n_new)) return rc;
        n_rows += it.n_new;
    }
    if (n_rows > kv->o.max_rows)
        return kv->fail(NI_ERR_TOO_MANY_ROWS, "%llu rows > max_rows %u", (unsigned long long)n_rows, kv->o.max_rows);
    return NI_OK;
}

// The step's rows (batch.rs:300-306: sequence s's n_new rows at positions
// seq_len .. seq_len+n_new-1) and its plan in kv->plan, partitioned for
// launches of n_lay layers.
static int build_step_plan(ni_kv* kv, const ni_work* work, uint32_t n_work, uint32_t split_tokens, uint32_t n_lay) {
    reset_plan(kv);
    // Fuse the append into the attention launch when every sequence has a
    // single query group: then exactly one workgroup per (layer, head, page)
    // touches this step's new rows.
    // With the prefill kernel, a sequence queried at more rows than that (a
    // prompt chunk with every row queried) has its rows appended by the
    // launch's extra blocks like a sequence without queries, and all its
    // query groups run in the prefill launch that follows; the others still
    // fuse.
    const bool prefill = !is_q8(kv->o) || kv->o.head_dim == 64;
    // A step of prompt chunks only keeps the append launch of its own (the
    // plain append kernel moves those rows faster than extra blocks of an
    // attention launch: 16 x 512 prefill 3521 against 3340 GB/s).
    bool fused = true, small = false, big = false;
    for (uint32_t w = 0; w < n_work; w++) {
        small |= work[w].n_query > 0 && work[w].n_query <= max_group_rows(kv);
        big |= work[w].n_query > max_group_rows(kv);
    }
    if (big) fused = prefill && small;
    // All layers per launch, an append launch goes first where the fused
    // form would put the append in workgroup prologues (the rows' input
    // loads and stores, then a barrier, before the first page loads):
    // * f16, every queried sequence a verify-style group (2 .. max_group_rows
    //   rows; the group kernel appends in its prologue): config 5 5584 ->
    //   5716 GB/s, the append launch included;
    // * Q8 (the all-layer Q8 kernel appends in its prologue), a queried
    //   sequence appending more than max_group_rows rows (a prompt chunk whose
    //   last row is queried) or at least kQ8SplitUnits queried (sequence,
    //   layer, head) units: Q8 config 3 (9216 units, prompt chunks) 4815 ->
    //   4944, while config 2 (2304 units, one row each) measured 4786 fused
    //   against 4741, config 4 and 5 the same either way.
    // f16 single rows take their rows as their pages stream (no prologue),
    // and stay fused (config 3: 6146 fused against 6118); so does one layer
    // per launch (a second launch per layer: f16 config 5 3808 -> 3411).
    if (fused && n_lay > 1) {
        constexpr uint64_t kQ8SplitUnits = 8192;
        bool any_group = false, any_single = false, long_rows = false;
        uint64_t units = 0;
        for (uint32_t w = 0; w < n_work; w++) {
            if (work[w].n_query == 0) continue;  // (rows appended by extra blocks, not prologues)
            any_group |= work[w].n_query > 1;
            any_single |= work[w].n_query == 1;
            long_rows |= work[w].n_new > max_group_rows(kv);
            units += (uint64_t)n_lay * kv->o.n_head;
        }
        if (is_q8(kv->o) ? long_rows || units >= kQ8SplitUnits : any_group && !any_single) fused = false;
    }
    kv->plan.fused = fused;
    // A step of prompt chunks whose every sequence is queried as prefill
    // groups, on a Q8 pool: the prefill launch appends each sequence's rows
    // itself (one workgroup per sequence, layer and head), no append launch.
    bool every_big = n_work > 0;
    for (uint32_t w = 0; w < n_work; w++) every_big &= work[w].n_query > max_group_rows(kv);
    kv->plan.seq_prefill = prefill && !fused && every_big && is_q8(kv->o);
    uint32_t row = 0;
    for (uint32_t w = 0; w < n_work; w++) {
        const ni_work& it = work[w];
        const uint32_t len = kv->seq_len[it.seq];
        const auto& pg = kv->pages[it.seq];
        const uint32_t first = (uint32_t)kv->plan.app.size();
        for (uint32_t i = 0; i < it.n_new; i++, row++) {
            const uint32_t pos = len + i;
            const AppendEntry e{row, pg[pos / kPage], pos % kPage, 0};
            kv->plan.app.push_back(e);
            // (a prompt chunk's short last group too: in a fused step its rows
            // are appended by the extra blocks, in a prompt-chunk step by its
            // sequence's prefill workgroup)
            const bool pre = (fused || kv->plan.seq_prefill) && it.n_query > max_group_rows(kv);
            if (fused && (it.n_query == 0 || pre)) kv->plan.orphans.push_back(e);
            if (i >= it.n_new - it.n_query) kv->qrows.push_back({row, it.seq, pos, len, len + it.n_new, first, pre});
        }
    }
    return plan_attention(kv, split_tokens, n_lay);
}

static int enqueue_step(ni_kv* kv, const ni_work* work, uint32_t n_work, const float* q, const float* k,
                        const float* v, int64_t row_stride, int64_t layer_stride, float* out, int64_t out_row_stride,
                        int64_t out_layer_stride, uint32_t split_tokens, hipStream_t stream) {
    if (int rc = build_step_plan(kv, work, n_work, split_tokens, kv->o.n_layer)) return rc;
    int rc = run_plan(kv, 0, kv->o.n_layer, k, v, row_stride, layer_stride, q, row_stride, layer_stride, out,
                      out_row_stride, out_layer_stride, stream);
    if (rc) return rc;
    // batch.rs:270: the step's rows now belong to their sequences.
    for (uint32_t w = 0; w < n_work; w++) kv->seq_len[work[w].seq] += work[w].n_new;
    return NI_OK;
}

extern "C" {

int ni_kv_sync(ni_kv* kv, ni_stream stream) {
    if (!kv) return NI_ERR_BAD_ARG;
    if (kv->host_only) return NI_OK;
    const hipStream_t s = (hipStream_t)stream;
    hipError_t e = hipStreamSynchronize(s);
    if (e != hipSuccess) return kv->hip_fail(e, "hipStreamSynchronize");
    // The handle's work on `s` is done: no later call needs to wait for it.
    if (kv->dirty && kv->dirty_stream == s) kv->dirty = false;
    if (kv->order_valid && kv->order_stream == s) kv->order_valid = false;
    // Outgrown partials buffers that no enqueued launch can still read.
    for (size_t i = 0; i < kv->partials_retired.size();) {
        auto& pr = kv->partials_retired[i];
        if (hipEventQuery(pr.second) != hipSuccess) {
            i++;
            continue;
        }
        (void)hipFree(pr.first);
        kv->ev_pool.push_back(pr.second);
        pr = kv->partials_retired.back();
        kv->partials_retired.pop_back();
    }
    return NI_OK;
}

int ni_attention(float* out, int64_t out_stride, const float* q, int64_t q_stride, const float* k, int64_t k_stride,
                 const float* v, int64_t v_stride, uint32_t n_q, uint32_t q_pos0, uint32_t n_head, uint32_t head_dim,
                 ni_stream stream) {
    auto fail = [](const std::string& msg) {
        g_create_error = msg;
        return NI_ERR_BAD_ARG;
    };
    if (n_q == 0) return NI_OK;
    if (!attention_supported(head_dim)) return fail("head_dim " + std::to_string(head_dim) + " unsupported (64 or 128)");
    if (n_head == 0) return fail("n_head must be > 0");
    if ((uint64_t)n_q * n_head >= (1ull << 31)) return fail("n_q * n_head too large");
    if ((uint64_t)q_pos0 + n_q > (1ull << 31)) return fail("q_pos0 + n_q too large");
    const struct {
        const char* name;
        const void* p;
        int64_t stride;
    } args[] = {{"out", out, out_stride}, {"q", q, q_stride}, {"k", k, k_stride}, {"v", v, v_stride}};
    for (const auto& x : args) {
        if (!x.p) return fail(std::string(x.name) + " is NULL");
        if (!aligned16(x.p) || x.stride < 0 || x.stride % 4 != 0)
            return fail(std::string(x.name) + " must be 16-byte aligned with a non-negative row stride that is a multiple of 4");
    }
    RowsLaunch a{};
    a.q = q;
    a.k = k;
    a.v = v;
    a.out = out;
    a.q_stride = q_stride;
    a.k_stride = k_stride;
    a.v_stride = v_stride;
    a.out_stride = out_stride;
    a.n_q = n_q;
    a.q_pos0 = q_pos0;
    a.n_head = n_head;
    a.head_dim = head_dim;
    a.qscale = (float)(1.4426950408889634 / std::sqrt((double)head_dim));
    const hipError_t e = launch_attention_rows(a, (hipStream_t)stream);
    if (e != hipSuccess) {
        g_create_error = std::string("attention launch failed: ") + hipGetErrorString(e);
        return NI_ERR_HIP;
    }
    return NI_OK;
}

int ni_f32_to_f16(const float* in, uint16_t* out, size_t n, ni_stream stream) {
    if (n == 0) return NI_OK;
    if (!in || !out) return NI_ERR_BAD_ARG;
    hipError_t e = launch_f32_to_f16(in, out, n, (hipStream_t)stream);
    return e == hipSuccess ? NI_OK : NI_ERR_HIP;
}

int ni_stream_probe(uint32_t mode, const void* src, void* dst, size_t bytes, uint32_t blocks, ni_stream stream) {
    if (!src || !dst || bytes % 16 || blocks == 0 || (mode & ~3u)) return NI_ERR_BAD_ARG;
    if ((size_t)blocks * 256 * 16 > bytes) return NI_ERR_BAD_ARG;  // a read's dst holds a unit per thread
    hipError_t e = launch_stream((mode & NI_PROBE_COPY) != 0, (mode & NI_PROBE_SPAN) != 0, src, dst, bytes, blocks,
                                 (hipStream_t)stream);
    return e == hipSuccess ? NI_OK : NI_ERR_HIP;
}

int ni_kv_profile(ni_kv* kv, uint32_t kernel_mask) {
    if (!kv) return NI_ERR_BAD_ARG;
    if (kv->host_only) return kv->fail(NI_ERR_NO_DEVICE, "host-only handle has no device");
    if (kernel_mask >> NI_K_COUNT) return kv->fail(NI_ERR_BAD_ARG, "kernel mask %#x has unknown bits", kernel_mask);
    // Create the events up front: hipEventCreate inside a timed loop costs
    // far more than recording.
    while (kernel_mask && kv->ev_pool.size() < kProfileEvents) {
        hipEvent_t e = nullptr;
        hipError_t rc = hipEventCreate(&e);
        if (rc != hipSuccess) return kv->hip_fail(rc, "hipEventCreate(profile)");
        kv->ev_pool.push_back(e);
    }
    kv->profile = kernel_mask;
    return NI_OK;
}

int ni_kv_profile_read(ni_kv* kv, int kernel, double* total_ms, uint64_t* launches) {
    if (!kv || kernel < 0 || kernel >= NI_K_COUNT) return NI_ERR_BAD_ARG;
    double ms = 0;
    uint64_t cnt = 0;
    for (auto& pr : kv->prof_ev[kernel]) {
        hipError_t e = hipEventSynchronize(pr.second);
        float t = 0;
        if (e == hipSuccess) e = hipEventElapsedTime(&t, pr.first, pr.second);
        if (e != hipSuccess) return kv->hip_fail(e, "profile events");
        ms += t;
        cnt++;
        kv->ev_pool.push_back(pr.first);
        kv->ev_pool.push_back(pr.second);
    }
    kv->prof_ev[kernel].clear();
    if (total_ms) *total_ms = ms;
    if (launches) *launches = cnt;
    return NI_OK;
}

}  // extern "C"
