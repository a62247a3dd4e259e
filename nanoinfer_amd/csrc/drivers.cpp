// drivers.cpp -- the reference's serving harnesses as C++ callers of the KV
// C ABI (include/nanoinfer_drivers.h).
//
// ni_serve restates the continuous-batching scheduler of
// crates/cli/src/metal_serve.rs:255-363 (request stream :97-126) on a step
// clock; ni_spec the verify side of crates/cli/src/metal_spec.rs:118-169;
// ni_drive_run a whole synthetic run of either on the device.  Nothing here
// touches the pools or kernels directly: every KV operation is an ni_kv_*
// call, as a HIP build of the reference's CLI would make it.
#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <deque>
#include <string>
#include <vector>

#include "nanoinfer_drivers.h"

namespace {

thread_local std::string g_drive_error;

int drive_fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int drive_fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_drive_error = buf;
    return code;
}

// metal_serve.rs:97-111.
struct XorShift {
    uint64_t s;
    static XorShift seeded(uint64_t seed) { return XorShift{(seed * 0x9E3779B97F4A7C15ull) | 1ull}; }  // :114
    uint64_t next() {
        s ^= s << 13;
        s ^= s >> 7;
        s ^= s << 17;
        return s;
    }
    double unif() { return (double)(next() >> 11) / (double)(1ull << 53); }
    uint32_t range(uint32_t lo, uint32_t hi) { return lo + (uint32_t)(next() % (uint64_t)(hi - lo + 1)); }
    // Box-Muller on top of the reference's generator (it has no normal sampler).
    float normal() {
        double u1 = std::max(unif(), 1e-300), u2 = unif();
        return (float)(std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2));
    }
};

uint32_t pages(uint32_t n) { return (n + NI_KV_BLOCK - 1) / NI_KV_BLOCK; }

struct Req {
    double arrival;
    uint32_t prompt_len, out_len;
};

// metal_serve.rs:113-126: Poisson gaps -ln(u)/rate, uniform prompt and output
// lengths; the text offset is drawn (and unused here) so the stream of
// random numbers is the reference's.  Text length 4*prompt_max + 64 as the
// reference builds it (metal_serve.rs:475-477).
std::vector<Req> requests(const ni_serve_opts& o) {
    XorShift rng = XorShift::seeded(o.seed);
    const uint32_t text_len = 4 * o.prompt_max + 64;
    std::vector<Req> r(o.n_requests);
    double t = 0;
    for (auto& q : r) {
        if (o.rate > 0) t += -std::log(std::max(rng.unif(), 1e-12)) / o.rate;
        q.arrival = t;
        q.prompt_len = rng.range(o.prompt_min, o.prompt_max);
        rng.range(0, text_len - q.prompt_len - 1);
        q.out_len = rng.range(o.out_min, o.out_max);
    }
    return r;
}

}  // namespace

struct ni_serve {
    ni_kv* kv;
    ni_serve_opts o;
    std::vector<Req> reqs;
    double clock = 0;
    size_t next = 0;
    std::deque<uint32_t> waiting;
    struct Live {
        uint32_t req, seq, prefilled, generated;
    };
    std::vector<Live> live;
    uint32_t done = 0;
    struct Kind {
        uint32_t j;
        bool prefill;
        uint32_t n;
    };
    std::vector<Kind> kinds;
    std::vector<ni_work> work;
    std::vector<uint32_t> ctx, admitted, retired, pending_retired;
    bool planned = false;
    // summary of the current stats window (ni_serve_get_stats)
    uint32_t iters = 0, snaps = 0, peak = 0;
    uint64_t rows = 0, generated = 0, pages_sum = 0, snap_seqs = 0, snap_len = 0, snap_slots = 0;
};

struct ni_spec {
    ni_kv* kv;
    std::vector<uint32_t> seqs, base, tlen, ctx, accepted;
    std::vector<ni_work> work;
    uint32_t k;
    uint32_t window;  // 0: no restart
    XorShift rng;
    bool planned = false;
};

extern "C" {

const char* ni_drive_last_error(void) { return g_drive_error.c_str(); }

int ni_serve_create(ni_kv* kv, const ni_serve_opts* o, ni_serve** out) {
    if (!kv || !o || !out) return NI_ERR_BAD_ARG;
    if (o->prompt_min < 1 || o->prompt_min > o->prompt_max || o->out_min < 1 || o->out_min > o->out_max ||
        o->max_batch == 0 || o->budget == 0 || o->max_rows == 0 || o->n_requests == 0)
        return drive_fail(NI_ERR_BAD_ARG, "bad serve options");
    auto* s = new ni_serve();
    s->kv = kv;
    s->o = *o;
    s->reqs = requests(*o);
    *out = s;
    return NI_OK;
}

void ni_serve_destroy(ni_serve* s) { delete s; }

uint32_t ni_serve_done(const ni_serve* s) { return s ? s->done : 0; }

// metal_serve.rs:271-307.
int ni_serve_plan(ni_serve* s, ni_serve_iter* it) {
    if (!s || !it) return NI_ERR_BAD_ARG;
    s->retired.swap(s->pending_retired);
    s->pending_retired.clear();
    s->admitted.clear();
    s->work.clear();
    s->ctx.clear();
    s->kinds.clear();
    const auto& reqs = s->reqs;
    for (;;) {
        while (s->next < reqs.size() && reqs[s->next].arrival <= s->clock) s->waiting.push_back((uint32_t)s->next++);
        if (s->live.empty() && s->waiting.empty()) {
            if (s->next >= reqs.size()) return drive_fail(NI_ERR_BAD_ARG, "every request has finished");
            s->clock = reqs[s->next].arrival;
            continue;
        }
        break;
    }
    // Admit while a slot is free and the pool holds the prompt plus one page
    // of headroom per running sequence.
    while (s->live.size() < s->o.max_batch && !s->waiting.empty()) {
        const uint32_t i = s->waiting.front();
        const uint32_t need = pages(reqs[i].prompt_len + 1) + (uint32_t)s->live.size();
        if (ni_kv_free_block_count(s->kv) < need) break;
        s->waiting.pop_front();
        uint32_t seq = 0;
        if (int rc = ni_kv_add_seq(s->kv, &seq)) return drive_fail(rc, "no sequence slot");
        s->admitted.push_back(seq);
        s->live.push_back({i, seq, 0, 0});
    }
    // One decode row per running sequence, then prefill chunks, oldest
    // first, under the token budget.
    uint32_t decode_rows = 0;
    for (uint32_t j = 0; j < s->live.size(); j++) {
        const auto& l = s->live[j];
        if (l.prefilled == reqs[l.req].prompt_len) {
            s->work.push_back({l.seq, 1, 1});
            s->kinds.push_back({j, false, 1});
            decode_rows++;
        }
    }
    uint32_t budget_left = std::min(s->o.budget, s->o.max_rows > decode_rows ? s->o.max_rows - decode_rows : 0u);
    for (uint32_t j = 0; j < s->live.size(); j++) {
        const auto& l = s->live[j];
        const uint32_t p = reqs[l.req].prompt_len;
        if (l.prefilled < p && budget_left > 0) {
            const uint32_t n = std::min(p - l.prefilled, budget_left);
            const bool last = l.prefilled + n == p;
            const uint32_t nq = s->o.query_all_prompt_rows ? n : (last ? 1u : 0u);
            s->work.push_back({l.seq, n, nq});
            s->kinds.push_back({j, true, n});
            budget_left -= n;
        }
    }
    for (const auto& w : s->work) {
        uint32_t len = 0;
        ni_kv_seq_len(s->kv, w.seq, &len);
        s->ctx.push_back(len + w.n_new);
    }
    s->planned = true;
    it->work = s->work.data();
    it->n_work = (uint32_t)s->work.size();
    it->ctx_after = s->ctx.data();
    it->admitted = s->admitted.data();
    it->n_admitted = (uint32_t)s->admitted.size();
    it->retired = s->retired.data();
    it->n_retired = (uint32_t)s->retired.size();
    return NI_OK;
}

// metal_serve.rs:331-357.
int ni_serve_commit(ni_serve* s) {
    if (!s) return NI_ERR_BAD_ARG;
    if (!s->planned) return drive_fail(NI_ERR_BAD_ARG, "commit without a planned iteration");
    s->planned = false;
    const auto& reqs = s->reqs;
    for (const auto& kd : s->kinds) {
        auto& l = s->live[kd.j];
        if (kd.prefill) {
            l.prefilled += kd.n;
            if (l.prefilled < reqs[l.req].prompt_len) continue;  // mid-prompt chunk: no token yet
        }
        l.generated++;
        s->generated++;
    }
    s->clock += 1.0;
    // metal_serve.rs:320-331: blocks in use after the step, and every
    // KV_SNAP_EVERY iterations the running sequences' lengths and pages,
    // before this iteration's retirements.
    const uint32_t used = ni_kv_blocks_used(s->kv);
    s->peak = std::max(s->peak, used);
    s->pages_sum += used;
    for (const auto& w : s->work) s->rows += w.n_new;
    if (s->iters % 10 == 0) {
        for (const auto& l : s->live) {
            uint32_t len = 0;
            const uint32_t* pg = nullptr;
            uint32_t np = 0;
            if (int rc = ni_kv_seq_len(s->kv, l.seq, &len)) return rc;
            if (int rc = ni_kv_block_table(s->kv, l.seq, &pg, &np)) return rc;
            s->snap_len += len;
            s->snap_slots += (uint64_t)np * NI_KV_BLOCK;
            s->snap_seqs++;
        }
        s->snaps++;
    }
    s->iters++;
    size_t k = 0;
    while (k < s->live.size()) {
        const auto& l = s->live[k];
        if (l.generated == reqs[l.req].out_len) {
            if (int rc = ni_kv_free_seq(s->kv, l.seq)) return rc;
            s->pending_retired.push_back(l.seq);
            s->live[k] = s->live.back();  // swap_remove
            s->live.pop_back();
            s->done++;
        } else {
            k++;
        }
    }
    return NI_OK;
}

int ni_serve_get_stats(const ni_serve* s, ni_serve_stats* out) {
    if (!s || !out) return NI_ERR_BAD_ARG;
    ni_serve_stats r{};
    r.iterations = s->iters;
    r.rows = s->rows;
    r.generated = s->generated;
    r.kv_pages_peak = s->peak;
    r.kv_pages_avg_used = s->iters ? (double)s->pages_sum / s->iters : 0.0;
    r.snapshots = s->snaps;
    r.avg_live_seqs = s->snaps ? (double)s->snap_seqs / s->snaps : 0.0;
    r.avg_pages_per_seq = s->snap_seqs ? (double)s->snap_slots / NI_KV_BLOCK / s->snap_seqs : 0.0;
    r.internal_fragmentation = s->snap_slots ? 1.0 - (double)s->snap_len / (double)s->snap_slots : 0.0;
    *out = r;
    return NI_OK;
}

int ni_serve_reset_stats(ni_serve* s) {
    if (!s) return NI_ERR_BAD_ARG;
    s->iters = s->snaps = s->peak = 0;
    s->rows = s->generated = s->pages_sum = s->snap_seqs = s->snap_len = s->snap_slots = 0;
    return NI_OK;
}

int ni_spec_create(ni_kv* kv, const uint32_t* seqs, uint32_t n, uint32_t draft_k, uint64_t seed, ni_spec** out) {
    if (!kv || (!seqs && n) || !out || draft_k == 0) return NI_ERR_BAD_ARG;
    auto* s = new ni_spec();
    s->kv = kv;
    s->seqs.assign(seqs, seqs + n);
    s->k = draft_k;
    s->window = 0;
    s->rng = XorShift::seeded(seed);
    for (uint32_t q : s->seqs) {
        uint32_t len = 0;
        if (int rc = ni_kv_seq_len(kv, q, &len)) {
            delete s;
            return rc;
        }
        s->base.push_back(len);
    }
    *out = s;
    return NI_OK;
}

void ni_spec_destroy(ni_spec* s) { delete s; }

int ni_spec_set_window(ni_spec* s, uint32_t window) {
    if (!s) return NI_ERR_BAD_ARG;
    s->window = window;
    return NI_OK;
}

// metal_spec.rs:137-143: the target appends [g, d1..dk] with a greedy
// prediction (here: a query) after every position.
int ni_spec_plan(ni_spec* s, const ni_work** work, uint32_t* n_work, const uint32_t** ctx_after) {
    if (!s || !work || !n_work) return NI_ERR_BAD_ARG;
    s->tlen.clear();
    s->work.clear();
    s->ctx.clear();
    for (uint32_t q : s->seqs) {
        uint32_t len = 0;
        if (int rc = ni_kv_seq_len(s->kv, q, &len)) return rc;
        s->tlen.push_back(len);
        s->work.push_back({q, s->k + 1, s->k + 1});
        s->ctx.push_back(len + s->k + 1);
    }
    s->planned = true;
    *work = s->work.data();
    *n_work = (uint32_t)s->work.size();
    if (ctx_after) *ctx_after = s->ctx.data();
    return NI_OK;
}

// metal_spec.rs:146-163: accept a prefix of the drafts, truncate the rest.
int ni_spec_commit(ni_spec* s, const uint32_t** accepted) {
    if (!s) return NI_ERR_BAD_ARG;
    if (!s->planned) return drive_fail(NI_ERR_BAD_ARG, "commit without a planned round");
    s->planned = false;
    s->accepted.clear();
    for (size_t i = 0; i < s->seqs.size(); i++) {
        const uint32_t acc = s->rng.range(0, s->k);
        const uint32_t keep = s->tlen[i] + 1 + acc;
        if (int rc = ni_kv_truncate(s->kv, s->seqs[i], keep)) return rc;
        if (s->window && keep > s->base[i] + s->window)
            if (int rc = ni_kv_truncate(s->kv, s->seqs[i], s->base[i])) return rc;
        s->accepted.push_back(acc);
    }
    if (accepted) *accepted = s->accepted.data();
    return NI_OK;
}

}  // extern "C"

// ------------------------------------------------------------------ runner

namespace {

struct DeviceBufs {
    float* q = nullptr;
    float* k = nullptr;
    float* v = nullptr;
    float* out = nullptr;
    ~DeviceBufs() {
        for (float* p : {q, k, v, out})
            if (p) (void)hipFree(p);
    }
};

// Algorithmic bytes of one step: each KV byte once, append and q/out rows.
// kvb = stored bytes of one position's K (or V) in one layer: 2C for f16,
// C + 4 * n_head for Q8 (int8 values and a scale per head).
double step_bytes(const ni_work* w, uint32_t n, const uint32_t* ctx, uint32_t n_layer, uint32_t c, double kvb) {
    double b = 0;
    for (uint32_t i = 0; i < n; i++) {
        b += (double)w[i].n_new * (c * 8.0 + 2 * kvb);
        if (w[i].n_query) b += (double)w[i].n_query * c * 8 + 2.0 * ctx[i] * kvb + pages(ctx[i]) * 4.0;
    }
    return b * n_layer;
}

struct Runner {
    const ni_drive_opts& o;
    ni_kv* kv = nullptr;
    hipStream_t stream = nullptr;
    DeviceBufs d;
    uint32_t C, L;
    int64_t ls;  // layer stride of the q/k/v/out buffers (floats)
    std::vector<ni_row> rows, qrows;
    uint64_t calls = 0;
    // With time_calls set: host seconds of each planning call (ni_kv_step,
    // ni_kv_step_begin) and each per-layer call (ni_kv_step_layer).
    bool time_calls = false;
    std::vector<double> plan_t, layer_t;

    double kvb;  // stored bytes of one position's K (or V) in one layer

    explicit Runner(const ni_drive_opts& opts) : o(opts), C(opts.kv.n_head * opts.kv.head_dim), L(opts.kv.n_layer) {
        ls = (int64_t)opts.kv.max_rows * C;
        kvb = (opts.kv.flags & NI_KV_Q8) ? (double)C + 4.0 * opts.kv.n_head : 2.0 * C;
    }
    ~Runner() {
        if (stream) (void)hipStreamDestroy(stream);
        if (kv) ni_kv_destroy(kv);
    }
    int kv_fail(int rc, const char* what) {
        return drive_fail(rc, "%s: %s", what, ni_kv_last_error(kv));
    }

    int setup() {
        if (int rc = ni_kv_create(&o.kv, &kv)) return drive_fail(rc, "ni_kv_create: %s", ni_kv_last_error(nullptr));
        if (hipStreamCreate(&stream) != hipSuccess) return drive_fail(NI_ERR_HIP, "hipStreamCreate failed");
        const size_t n = (size_t)L * ls;
        std::vector<float> host(n);
        XorShift g = XorShift::seeded(o.data_seed);
        const float kv_std = o.kv_std > 0 ? o.kv_std : 1.f;
        for (float** p : {&d.q, &d.k, &d.v, &d.out}) {
            if (hipMalloc(p, n * sizeof(float)) != hipSuccess) return drive_fail(NI_ERR_HIP, "hipMalloc failed");
            const float scale = (p == &d.k || p == &d.v) ? kv_std : 1.f;
            for (auto& x : host) x = g.normal() * scale;
            if (hipMemcpy(*p, host.data(), n * sizeof(float), hipMemcpyHostToDevice) != hipSuccess)
                return drive_fail(NI_ERR_HIP, "hipMemcpy failed");
        }
        return NI_OK;
    }

    // Fill positions 0..len-1 of seq (untimed set-up), max_rows at a time.
    int fill(uint32_t seq, uint32_t len) {
        if (int rc = ni_kv_reserve(kv, seq, len)) return kv_fail(rc, "reserve");
        for (uint32_t p0 = 0; p0 < len; p0 += o.kv.max_rows) {
            const uint32_t n = std::min(o.kv.max_rows, len - p0);
            rows.resize(n);
            for (uint32_t i = 0; i < n; i++) rows[i] = {seq, p0 + i};
            if (int rc = ni_kv_append(kv, NI_ALL_LAYERS, rows.data(), n, d.k, d.v, C, ls, stream))
                return kv_fail(rc, "append");
        }
        if (int rc = ni_kv_commit(kv, seq, len)) return kv_fail(rc, "commit");
        return NI_OK;
    }

    // A ramp iteration: the work's rows reserved, appended for every layer in
    // one call and committed, in work order (ni_kv_step's page order and
    // row numbering), with no attention.
    int append_only(const ni_work* w, uint32_t n) {
        rows.clear();
        for (uint32_t i = 0; i < n; i++) {
            uint32_t len = 0;
            ni_kv_seq_len(kv, w[i].seq, &len);
            if (int rc = ni_kv_reserve(kv, w[i].seq, len + w[i].n_new)) return kv_fail(rc, "reserve");
            for (uint32_t j = 0; j < w[i].n_new; j++) rows.push_back({w[i].seq, len + j});
        }
        if (!rows.empty())
            if (int rc = ni_kv_append(kv, NI_ALL_LAYERS, rows.data(), (uint32_t)rows.size(), d.k, d.v, C, ls, stream))
                return kv_fail(rc, "append");
        for (uint32_t i = 0; i < n; i++)
            if (int rc = ni_kv_commit(kv, w[i].seq, w[i].n_new)) return kv_fail(rc, "commit");
        return NI_OK;
    }

    // One iteration's KV work through the chosen launch path (append_only:
    // a ramp iteration).
    int launch(const ni_work* w, uint32_t n, bool ramp = false) {
        if (ramp) return append_only(w, n);
        using clk = std::chrono::steady_clock;
        auto since = [](clk::time_point t) { return std::chrono::duration<double>(clk::now() - t).count(); };
        if (o.launch == NI_DRIVE_STEP) {
            calls++;
            const auto t0 = clk::now();
            if (int rc = ni_kv_step(kv, w, n, d.q, d.k, d.v, C, ls, d.out, C, ls, o.split_tokens, stream))
                return kv_fail(rc, "ni_kv_step");
            if (time_calls) plan_t.push_back(since(t0));
            return NI_OK;
        }
        if (o.launch == NI_DRIVE_STEP_LAYERS) {
            // The step planned once, then one append + attention launch per
            // layer, as a model's forward would call it between layers.
            const auto t0 = clk::now();
            if (int rc = ni_kv_step_begin(kv, w, n, o.split_tokens)) return kv_fail(rc, "ni_kv_step_begin");
            if (time_calls) plan_t.push_back(since(t0));
            for (uint32_t l = 0; l < L; l++) {
                calls++;
                const auto t1 = clk::now();
                if (int rc = ni_kv_step_layer(kv, (int32_t)l, d.q + l * ls, d.k + l * ls, d.v + l * ls, C,
                                              d.out + l * ls, C, stream)) {
                    (void)ni_kv_step_end(kv);
                    return kv_fail(rc, "ni_kv_step_layer");
                }
                if (time_calls) layer_t.push_back(since(t1));
            }
            if (int rc = ni_kv_step_end(kv)) return kv_fail(rc, "ni_kv_step_end");
            return NI_OK;
        }
        // Per layer, as the reference's forward dispatches: reserve, then for
        // each layer append its rows and attend its queried rows, then commit.
        rows.clear();
        qrows.clear();
        for (uint32_t i = 0; i < n; i++) {
            uint32_t len = 0;
            ni_kv_seq_len(kv, w[i].seq, &len);
            if (int rc = ni_kv_reserve(kv, w[i].seq, len + w[i].n_new)) return kv_fail(rc, "reserve");
            for (uint32_t j = 0; j < w[i].n_new; j++) {
                rows.push_back({w[i].seq, len + j});
                if (j >= w[i].n_new - w[i].n_query) qrows.push_back({w[i].seq, len + j});
            }
        }
        for (uint32_t l = 0; l < L; l++) {
            calls += 1 + !qrows.empty();
            if (int rc = ni_kv_append(kv, (int32_t)l, rows.data(), (uint32_t)rows.size(), d.k + l * ls, d.v + l * ls, C,
                                      0, stream))
                return kv_fail(rc, "ni_kv_append");
            if (!qrows.empty())
                if (int rc = ni_paged_decode_attention(kv, (int32_t)l, d.q + l * ls, C, 0, qrows.data(),
                                                       (uint32_t)qrows.size(), d.out + l * ls, C, 0, o.split_tokens,
                                                       stream))
                    return kv_fail(rc, "ni_paged_decode_attention");
        }
        for (uint32_t i = 0; i < n; i++)
            if (int rc = ni_kv_commit(kv, w[i].seq, w[i].n_new)) return kv_fail(rc, "commit");
        return NI_OK;
    }
};

using Clock = std::chrono::steady_clock;

double seconds_since(Clock::time_point t) { return std::chrono::duration<double>(Clock::now() - t).count(); }

enum Phase { RAMP, WARMUP, TIMED };

// Run `iterate(phase)` over ramp + warmup + steps iterations; time the last
// `steps`.
template <typename Fn>
int timed_run(Runner& r, ni_drive_result* res, Fn&& iterate) {
    for (uint32_t i = 0; i < r.o.ramp; i++)
        if (int rc = iterate(RAMP)) return rc;
    for (uint32_t i = 0; i < r.o.warmup; i++)
        if (int rc = iterate(WARMUP)) return rc;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    if (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess)
        return drive_fail(NI_ERR_HIP, "hipEventCreate failed");
    if (hipStreamSynchronize(r.stream) != hipSuccess) return drive_fail(NI_ERR_HIP, "hipStreamSynchronize failed");
    if (r.o.profile_mask) {
        if (int rc = ni_kv_profile(r.kv, r.o.profile_mask)) return r.kv_fail(rc, "ni_kv_profile");
        for (int k = 0; k < NI_K_COUNT; k++) ni_kv_profile_read(r.kv, k, nullptr, nullptr);
    }
    r.calls = 0;
    double host = 0;
    const auto t0 = Clock::now();
    (void)hipEventRecord(e0, r.stream);
    for (uint32_t i = 0; i < r.o.steps; i++) {
        const auto h0 = Clock::now();
        if (int rc = iterate(TIMED)) return rc;
        host += seconds_since(h0);
    }
    (void)hipEventRecord(e1, r.stream);
    if (hipStreamSynchronize(r.stream) != hipSuccess) return drive_fail(NI_ERR_HIP, "hipStreamSynchronize failed");
    res->seconds = seconds_since(t0);
    float ms = 0;
    (void)hipEventElapsedTime(&ms, e0, e1);
    res->gpu_seconds = ms / 1e3;
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    res->host_us_per_step = host / std::max(1u, r.o.steps) * 1e6;
    res->steps = r.o.steps;
    res->launches = r.calls;
    if (r.o.profile_mask) {
        for (int k = 0; k < NI_K_COUNT; k++)
            if (int rc = ni_kv_profile_read(r.kv, k, &res->kernel_ms[k], &res->kernel_launches[k]))
                return r.kv_fail(rc, "ni_kv_profile_read");
        ni_kv_profile(r.kv, 0);
    }
    // The host cost of the calls themselves: a few more iterations, each
    // after the stream has drained, so no call waits for room in the
    // device's queue (in the timed loop the host runs ahead until it does).
    // The median of the calls, so that one stall of the host does not move it.
    r.plan_t.clear();
    r.layer_t.clear();
    r.time_calls = true;
    const uint32_t n_idle = std::min<uint32_t>(r.o.steps, 20);
    for (uint32_t i = 0; i < n_idle; i++) {
        if (hipStreamSynchronize(r.stream) != hipSuccess) return drive_fail(NI_ERR_HIP, "hipStreamSynchronize failed");
        if (int rc = iterate(WARMUP)) return rc;
    }
    r.time_calls = false;
    if (hipStreamSynchronize(r.stream) != hipSuccess) return drive_fail(NI_ERR_HIP, "hipStreamSynchronize failed");
    auto median_us = [](std::vector<double>& t) {
        if (t.empty()) return 0.0;
        std::nth_element(t.begin(), t.begin() + t.size() / 2, t.end());
        return t[t.size() / 2] * 1e6;
    };
    res->idle_us_plan_call = median_us(r.plan_t);
    res->idle_us_layer_call = median_us(r.layer_t);
    return NI_OK;
}

int run_serve(Runner& r, ni_drive_result* res) {
    ni_serve* sv = nullptr;
    if (int rc = ni_serve_create(r.kv, &r.o.serve, &sv)) return rc;
    double live = 0, ctx = 0;
    uint32_t timed = 0;
    int rc = timed_run(r, res, [&](Phase ph) -> int {
        ni_serve_iter it{};
        if (int e = ni_serve_plan(sv, &it)) return e;
        if (int e = r.launch(it.work, it.n_work, ph == RAMP)) return e;
        if (ph == TIMED) {
            res->bytes += step_bytes(it.work, it.n_work, it.ctx_after, r.L, r.C, r.kvb);
            for (uint32_t i = 0; i < it.n_work; i++)
                if (it.work[i].n_query) {
                    res->seq_tokens += 1;
                    live += 1;
                    ctx += it.ctx_after[i];
                }
        }
        if (int e = ni_serve_commit(sv)) return e;
        // the summary over every iteration up to the last timed one
        if (ph == TIMED && ++timed == r.o.steps) return ni_serve_get_stats(sv, &res->serve_stats);
        return NI_OK;
    });
    ni_serve_destroy(sv);
    res->mean_live = live / std::max(1u, r.o.steps);
    res->mean_context = ctx / std::max(1.0, live);
    return rc;
}

int run_spec(Runner& r, ni_drive_result* res) {
    XorShift rng = XorShift::seeded(r.o.spec_seed);
    std::vector<uint32_t> seqs;
    for (uint32_t i = 0; i < r.o.spec_seqs; i++) {
        const uint32_t len = rng.range(r.o.spec_ctx_min, r.o.spec_ctx_max);
        uint32_t s = 0;
        if (int rc = ni_kv_add_seq(r.kv, &s)) return r.kv_fail(rc, "add_seq");
        if (int rc = r.fill(s, len)) return rc;
        seqs.push_back(s);
    }
    ni_spec* sp = nullptr;
    if (int rc = ni_spec_create(r.kv, seqs.data(), (uint32_t)seqs.size(), r.o.spec_k, r.o.data_seed, &sp)) return rc;
    ni_spec_set_window(sp, r.o.spec_window);
    double ctx = 0;
    int rc = timed_run(r, res, [&](Phase ph) -> int {
        const ni_work* w = nullptr;
        const uint32_t* ca = nullptr;
        uint32_t n = 0;
        if (int e = ni_spec_plan(sp, &w, &n, &ca)) return e;
        if (int e = r.launch(w, n, ph == RAMP)) return e;
        const uint32_t* acc = nullptr;
        if (int e = ni_spec_commit(sp, &acc)) return e;
        if (ph == TIMED) {
            res->bytes += step_bytes(w, n, ca, r.L, r.C, r.kvb);
            for (uint32_t i = 0; i < n; i++) {
                res->seq_tokens += acc[i] + 1;  // tokens a verify round yields
                ctx += ca[i];
            }
        }
        return NI_OK;
    });
    ni_spec_destroy(sp);
    res->mean_live = r.o.spec_seqs;
    res->mean_context = ctx / std::max(1.0, (double)r.o.spec_seqs * r.o.steps);
    return rc;
}

int run_fixed(Runner& r, ni_drive_result* res) {
    if (!r.o.fixed_ctx || r.o.fixed_n == 0) return drive_fail(NI_ERR_BAD_ARG, "fixed workload without contexts");
    const uint32_t R = r.o.fixed_rows ? r.o.fixed_rows : 1;
    std::vector<uint32_t> seqs;
    std::vector<ni_work> work;
    double flops = 0;
    for (uint32_t i = 0; i < r.o.fixed_n; i++) {
        const uint32_t ctx = r.o.fixed_ctx[i];
        if (ctx < R) return drive_fail(NI_ERR_BAD_ARG, "fixed context %u < %u rows", ctx, R);
        uint32_t s = 0;
        if (int rc = ni_kv_add_seq(r.kv, &s)) return r.kv_fail(rc, "add_seq");
        if (ctx > R)
            if (int rc = r.fill(s, ctx - R)) return rc;
        seqs.push_back(s);
        work.push_back({s, R, R});
        // Row j (position ctx - R + j) sees ctx - R + j + 1 keys.
        flops += 4.0 * r.C * r.L * ((double)R * (ctx - R) + (double)R * (R + 1) / 2);
    }
    const double bytes = step_bytes(work.data(), (uint32_t)work.size(), r.o.fixed_ctx, r.L, r.C, r.kvb);
    int rc = timed_run(r, res, [&](Phase ph) -> int {
        if (int e = r.launch(work.data(), (uint32_t)work.size(), ph == RAMP)) return e;
        // Roll back, so the next iteration appends the same positions.
        for (uint32_t i = 0; i < r.o.fixed_n; i++)
            if (int e = ni_kv_truncate(r.kv, seqs[i], r.o.fixed_ctx[i] - R)) return r.kv_fail(e, "truncate");
        if (ph == TIMED) {
            res->bytes += bytes;
            res->flops += flops;
            res->seq_tokens += (double)r.o.fixed_n * R;
        }
        return NI_OK;
    });
    double ctx = 0;
    for (uint32_t i = 0; i < r.o.fixed_n; i++) ctx += r.o.fixed_ctx[i];
    res->mean_live = r.o.fixed_n;
    res->mean_context = ctx / r.o.fixed_n;
    return rc;
}

// The reference's weight upload in the formats it serves with
// (crates/metal/src/weights.rs:12-27 quantize_q8_0, :54-72 quantize_q4_0,
// :115-118 f16), over one row-major matrix: quants, then one f16 scale per
// block of 32.  The f16 conversion is the library's (round to nearest even).
uint16_t to_f16(float x) {
    const _Float16 h = static_cast<_Float16>(x);
    uint16_t b;
    std::memcpy(&b, &h, 2);
    return b;
}
std::vector<uint8_t> upload_weights(const std::vector<float>& w, uint32_t fmt) {
    const size_t n = w.size();
    std::vector<uint8_t> out;
    if (fmt == NI_W_F32) {
        out.resize(4 * n);
        std::memcpy(out.data(), w.data(), 4 * n);
        return out;
    }
    if (fmt == NI_W_F16) {
        out.resize(2 * n);
        for (size_t i = 0; i < n; i++) {
            const uint16_t h = to_f16(w[i]);
            std::memcpy(&out[2 * i], &h, 2);
        }
        return out;
    }
    const bool q8 = fmt == NI_W_Q8_0;
    const size_t qb = q8 ? n : n / 2;
    out.assign(qb + n / 16, 0);
    for (size_t b = 0; b < n / 32; b++) {
        const float* blk = &w[32 * b];
        float d;
        if (q8) {
            float amax = 0.f;
            for (int i = 0; i < 32; i++) amax = std::max(amax, std::fabs(blk[i]));
            d = amax / 127.f;
            const float id = d > 0.f ? 1.f / d : 0.f;
            for (int i = 0; i < 32; i++) {
                const float r = std::round(blk[i] * id);
                out[32 * b + i] = (uint8_t)(int8_t)std::max(-128.f, std::min(127.f, r));
            }
        } else {
            float mx = 0.f;
            for (int i = 0; i < 32; i++)
                if (std::fabs(blk[i]) > std::fabs(mx)) mx = blk[i];
            d = mx / -8.f;
            const float id = d != 0.f ? 1.f / d : 0.f;
            auto q = [&](float v) { return (uint8_t)std::max(0, std::min(15, (int)(v * id + 8.5f))); };
            for (int i = 0; i < 16; i++) out[16 * b + i] = (uint8_t)(q(blk[i]) | (q(blk[i + 16]) << 4));
        }
        const uint16_t h = to_f16(d);
        std::memcpy(&out[qb + 2 * b], &h, 2);
    }
    return out;
}

double weight_bytes(uint32_t fmt, double n) {
    return fmt == NI_W_F32 ? 4 * n : fmt == NI_W_F16 ? 2 * n : fmt == NI_W_Q8_0 ? n + n / 16 : n / 2 + n / 16;
}

int run_qkv(Runner& r, ni_drive_result* res) {
    const uint32_t n = r.o.qkv_rows, C = r.C, L = r.L, d_in = C, F = 3 * C;
    if (n == 0 || n > r.o.kv.max_rows) return drive_fail(NI_ERR_BAD_ARG, "qkv_rows must be 1..max_rows");
    if (L < 3) return drive_fail(NI_ERR_BAD_ARG, "the unfused path keeps [n][3C] in the k buffer: n_layer >= 3");
    // Rows spread over the sequences, one page-aligned position block each.
    const uint32_t S = std::min(n, r.o.kv.max_seqs);
    std::vector<uint32_t> seqs(S);
    for (uint32_t i = 0; i < S; i++) {
        if (int rc = ni_kv_add_seq(r.kv, &seqs[i])) return r.kv_fail(rc, "add_seq");
        if (int rc = ni_kv_reserve(r.kv, seqs[i], (n + S - 1) / S)) return r.kv_fail(rc, "reserve");
    }
    std::vector<ni_row> rows(n);
    for (uint32_t i = 0; i < n; i++) rows[i] = {seqs[i % S], i / S};
    const uint32_t fmt = r.o.qkv_wformat;
    if (fmt > NI_W_Q4_0) return drive_fail(NI_ERR_BAD_ARG, "qkv_wformat must be one of NI_W_*");
    if (fmt != NI_W_F32 && r.o.launch != NI_DRIVE_STEP)
        return drive_fail(NI_ERR_BAD_ARG, "the unfused comparison runs f32 weights only");
    // W [L][3C][d_in] ~ N(0, 1/d_in) in format fmt (each layer's matrix
    // quantised on its own), bias [L][3C] ~ N(0, 0.01).
    const size_t wn = (size_t)L * F * d_in;
    const size_t wl_bytes = (size_t)weight_bytes(fmt, (double)F * d_in);  // one layer's matrix
    uint8_t* w = nullptr;
    float* bias = nullptr;
    if (hipMalloc(&w, (size_t)L * wl_bytes) != hipSuccess || hipMalloc(&bias, (size_t)L * F * sizeof(float)) != hipSuccess)
        return drive_fail(NI_ERR_HIP, "hipMalloc(weights) failed");
    struct Free {
        void* p[2];
        ~Free() {
            for (void* q : p)
                if (q) (void)hipFree(q);
        }
    } guard{{w, bias}};
    {
        XorShift g = XorShift::seeded(r.o.data_seed + 1);
        std::vector<float> host(wn);
        const float sc = 1.f / std::sqrt((float)d_in);
        for (auto& x : host) x = g.normal() * sc;
        for (uint32_t l = 0; l < L; l++) {
            std::vector<float> one(host.begin() + (size_t)l * F * d_in, host.begin() + (size_t)(l + 1) * F * d_in);
            const std::vector<uint8_t> up = upload_weights(one, fmt);
            if (up.size() != wl_bytes ||
                hipMemcpy(w + (size_t)l * wl_bytes, up.data(), wl_bytes, hipMemcpyHostToDevice) != hipSuccess)
                return drive_fail(NI_ERR_HIP, "hipMemcpy(weights) failed");
        }
        host.resize((size_t)L * F);
        for (auto& x : host) x = g.normal() * 0.1f;
        if (hipMemcpy(bias, host.data(), host.size() * sizeof(float), hipMemcpyHostToDevice) != hipSuccess)
            return drive_fail(NI_ERR_HIP, "hipMemcpy(bias) failed");
    }
    const double bytes = (double)L * ((double)wl_bytes + F * 4.0 + (double)n * d_in * 4 + (double)n * C * 4 +
                                      (double)n * 2 * C * 2);
    const double flops = 2.0 * L * n * (double)d_in * F;
    float* x = r.d.q;    // [n][d_in]
    float* y = r.d.k;    // unfused: [n][3C]
    // The projection has no append-only form: ramp iterations run whole.
    int rc = timed_run(r, res, [&](Phase ph) -> int {
        for (uint32_t l = 0; l < L; l++) {
            const void* wl = w + (size_t)l * wl_bytes;
            const float* bl = bias + (size_t)l * F;
            if (r.o.launch == NI_DRIVE_STEP) {
                r.calls++;
                if (int e = ni_kv_qkv_append_w(r.kv, (int32_t)l, rows.data(), n, x, d_in, d_in, wl, fmt, bl,
                                               r.d.out, C, r.stream))
                    return r.kv_fail(e, "ni_kv_qkv_append_w");
            } else {
                r.calls += 2;
                if (int e = ni_kv_qkv_project(r.kv, x, d_in, n, d_in, static_cast<const float*>(wl), bl, y, F,
                                              r.stream))
                    return r.kv_fail(e, "ni_kv_qkv_project");
                if (int e = ni_kv_append(r.kv, (int32_t)l, rows.data(), n, y + C, y + 2 * C, F, 0, r.stream))
                    return r.kv_fail(e, "ni_kv_append");
            }
        }
        if (ph == TIMED) {
            res->bytes += bytes;
            res->flops += flops;
            res->seq_tokens += n;
        }
        return NI_OK;
    });
    res->mean_live = n;
    return rc;
}

}  // namespace

extern "C" int ni_drive_device_memory(int device, int* mem_clock_khz, int* bus_width_bits) {
    if (!mem_clock_khz || !bus_width_bits) return drive_fail(NI_ERR_BAD_ARG, "NULL argument");
    if (hipDeviceGetAttribute(mem_clock_khz, hipDeviceAttributeMemoryClockRate, device) != hipSuccess ||
        hipDeviceGetAttribute(bus_width_bits, hipDeviceAttributeMemoryBusWidth, device) != hipSuccess)
        return drive_fail(NI_ERR_HIP, "hipDeviceGetAttribute failed for device %d", device);
    return NI_OK;
}

extern "C" int ni_drive_run(const ni_drive_opts* o, ni_drive_result* res) {
    if (!o || !res) return drive_fail(NI_ERR_BAD_ARG, "NULL argument");
    if (o->launch > NI_DRIVE_STEP_LAYERS) return drive_fail(NI_ERR_BAD_ARG, "unknown launch mode %u", o->launch);
    if (o->workload == NI_DRIVE_QKV && o->launch == NI_DRIVE_STEP_LAYERS)
        return drive_fail(NI_ERR_BAD_ARG, "the qkv workload runs NI_DRIVE_STEP or NI_DRIVE_PER_LAYER");
    if (o->kv.flags & NI_KV_HOST_ONLY) return drive_fail(NI_ERR_BAD_ARG, "ni_drive_run needs a device handle");
    *res = ni_drive_result{};
    Runner r(*o);
    if (int rc = r.setup()) return rc;
    switch (o->workload) {
        case NI_DRIVE_SERVE: return run_serve(r, res);
        case NI_DRIVE_SPEC: return run_spec(r, res);
        case NI_DRIVE_FIXED: return run_fixed(r, res);
        case NI_DRIVE_QKV: return run_qkv(r, res);
        default: return drive_fail(NI_ERR_BAD_ARG, "unknown workload %u", o->workload);
    }
}
