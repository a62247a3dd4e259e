/*
 * nanoinfer_drivers.h -- C++ serving drivers over the KV C ABI (nanoinfer_kv.h).
 *
 * The reference's serving harnesses restated as callers of the ABI, the way a
 * HIP build of the CLI would drive it:
 *   - ni_serve_*: the continuous-batching scheduler of `metal-serve`
 *     (crates/cli/src/metal_serve.rs:97-126 request stream and RNG,
 *     :255-363 admission, iteration and retirement), on a step clock: the
 *     clock advances one unit per iteration instead of by measured seconds,
 *     so a trace is the same on every machine.
 *   - ni_spec_*: the verify side of `metal-spec` (metal_spec.rs:118-169):
 *     append [g, d1..dk] with a causal query at every row, accept a prefix,
 *     truncate the rejected drafts.  Acceptance is drawn from the seeded RNG
 *     (the KV path sees no tokens).
 *   - ni_drive_run: a whole synthetic run of either driver on the device
 *     (q/k/v N(0,1) in HBM), timed with HIP events, launching through
 *     ni_kv_step (all layers in one launch) or per layer through
 *     ni_kv_append + ni_paged_decode_attention (the reference's per-layer
 *     dispatch, batch.rs:393-416,577-616).
 *
 * Drivers own no device memory of the KV cache; they call only the ABI.
 * Status codes are ni_status values; the message is ni_kv_last_error() of
 * the handle, or ni_drive_last_error() for ni_drive_run.
 */
#ifndef NANOINFER_DRIVERS_H
#define NANOINFER_DRIVERS_H

#include <stdint.h>

#include "nanoinfer_kv.h"

#ifdef __cplusplus
extern "C" {
#endif

/* ServeArgs fields used by the scheduler (metal_serve.rs:35-70, 470-486). */
typedef struct ni_serve_opts {
    uint64_t seed;         /* Rng(seed * 0x9e3779b97f4a7c15 | 1), metal_serve.rs:114 */
    double rate;           /* arrivals per step (per second in the reference); 0 = all at once */
    uint32_t n_requests;
    uint32_t max_batch;    /* concurrent sequences (slots) */
    uint32_t prompt_min, prompt_max;
    uint32_t out_min, out_max;
    uint32_t budget;       /* prefill rows per iteration (metal_serve.rs:299) */
    uint32_t max_rows;     /* rows per step at most (BatchOpts::max_rows) */
    /* 0: only the row that completes a prompt is queried (the reference's
     * all_logits = false); 1: every prompt row is queried. */
    uint32_t query_all_prompt_rows;
} ni_serve_opts;

typedef struct ni_serve ni_serve;

/* One iteration of the scheduler.  Arrays stay valid until the next call on
 * the driver.  `retired` lists sequences freed after the previous iteration
 * (already freed on the handle), `admitted` the sequences added for this
 * one (already added); `work` is what ni_kv_step takes; ctx_after[i] is
 * work[i]'s context after the step. */
typedef struct ni_serve_iter {
    const ni_work* work;
    uint32_t n_work;
    const uint32_t* ctx_after;
    const uint32_t* admitted;
    uint32_t n_admitted;
    const uint32_t* retired;
    uint32_t n_retired;
} ni_serve_iter;

int ni_serve_create(ni_kv* kv, const ni_serve_opts* opts, ni_serve** out);
void ni_serve_destroy(ni_serve* s);
/* Admit and build the next iteration (metal_serve.rs:271-307). */
int ni_serve_plan(ni_serve* s, ni_serve_iter* it);
/* After the step ran: advance prompts and outputs, retire finished
 * sequences with free_seq (metal_serve.rs:331-357). */
int ni_serve_commit(ni_serve* s);
/* Requests finished so far. */
uint32_t ni_serve_done(const ni_serve* s);

/* The serving summary of the reference's KV figures (metal_serve.rs:320-331,
 * 361, 440-464), taken in ni_serve_commit after each iteration's step and
 * before its retirements, as the reference takes them after b.step:
 * blocks in use (peak and mean), and every KV_SNAP_EVERY = 10 iterations a
 * snapshot of the running sequences' lengths and pages.  Internal
 * fragmentation = 1 - sum(len) / sum(pages * 16) over every snapshot.  On
 * the step clock every iteration weighs the same in the mean (the reference
 * weighs it by its measured GPU time).  ni_serve_reset_stats starts a new
 * window (the next iteration is snapshot 0 of it). */
typedef struct ni_serve_stats {
    uint32_t iterations;
    uint64_t rows;             /* rows appended (decode rows + prompt rows) */
    uint64_t generated;        /* tokens produced: decode rows + prompts completed */
    uint32_t kv_pages_peak;
    double kv_pages_avg_used;
    uint32_t snapshots;
    double avg_live_seqs;
    double avg_pages_per_seq;
    double internal_fragmentation;
} ni_serve_stats;
int ni_serve_get_stats(const ni_serve* s, ni_serve_stats* out);
int ni_serve_reset_stats(ni_serve* s);

typedef struct ni_spec ni_spec;
/* Verify driver over sequences that are live and filled: each round appends
 * draft_k + 1 rows to every sequence, all queried. */
int ni_spec_create(ni_kv* kv, const uint32_t* seqs, uint32_t n_seqs, uint32_t draft_k, uint64_t seed, ni_spec** out);
void ni_spec_destroy(ni_spec* s);
/* The round's work (metal_spec.rs:137-143) and contexts after it. */
int ni_spec_plan(ni_spec* s, const ni_work** work, uint32_t* n_work, const uint32_t** ctx_after);
/* After the step ran: accept acc ~ U[0, draft_k] per sequence and
 * truncate(seq, tlen + 1 + acc) (metal_spec.rs:146-163). */
int ni_spec_commit(ni_spec* s, const uint32_t** accepted);
/* Restart rule for long runs: a sequence that has grown more than `window`
 * rows past its length at ni_spec_create is truncated back to that length
 * after the round (a request ends; the next, with the same prompt length,
 * takes its slot).  0 (the default) = sequences grow without bound. */
int ni_spec_set_window(ni_spec* s, uint32_t window);

/* ---- a whole synthetic run on the device ---- */
enum ni_drive_workload {
    NI_DRIVE_SERVE = 0, /* ni_serve over the trace (config 3) */
    NI_DRIVE_SPEC = 1,  /* ni_spec verify rounds (config 5) */
    /* Fixed contexts (configs 2 and 4, and prefill): sequence i holds
     * fixed_ctx[i] - R positions (R = fixed_rows, default 1); every
     * iteration appends R rows to each and attends all of them, then
     * truncates back, so every iteration does the same work. */
    NI_DRIVE_FIXED = 2,
    /* The QKV projection of qkv_rows rows (d_in = C, random W and bias per
     * layer) with K/V appended, every layer per iteration: launch
     * NI_DRIVE_STEP runs ni_kv_qkv_append (the fused epilogue),
     * NI_DRIVE_PER_LAYER ni_kv_qkv_project + ni_kv_append (f32 K/V through
     * memory).  Rows i of qkv_rows go to sequence i % max_seqs. */
    NI_DRIVE_QKV = 3
};
enum ni_drive_launch {
    NI_DRIVE_STEP = 0,     /* one ni_kv_step per iteration (all layers per launch) */
    NI_DRIVE_PER_LAYER = 1, /* ni_kv_append + ni_paged_decode_attention per layer */
    NI_DRIVE_STEP_LAYERS = 2 /* ni_kv_step_begin, one ni_kv_step_layer per layer, ni_kv_step_end */
};

typedef struct ni_drive_opts {
    uint32_t workload;      /* ni_drive_workload */
    uint32_t launch;        /* ni_drive_launch */
    ni_kv_opts kv;          /* pool and shape */
    ni_serve_opts serve;    /* NI_DRIVE_SERVE */
    uint32_t spec_seqs;     /* NI_DRIVE_SPEC: sequences, contexts U[ctx_min, ctx_max] */
    uint32_t spec_ctx_min, spec_ctx_max;
    uint32_t spec_k;        /* drafts per round */
    uint64_t spec_seed;     /* contexts; acceptance draws use data_seed */
    uint32_t spec_window;   /* see ni_spec_set_window (0 = none) */
    /* untimed iterations before the warmup that only append (each
     * iteration's rows reserved, appended for every layer and committed in
     * work order, as ni_kv_step would: the same pages and bytes) and run no
     * attention: they bring a trace to its steady state cheaply */
    uint32_t ramp;
    uint32_t warmup;        /* untimed iterations (full steps) */
    uint32_t steps;         /* timed iterations */
    uint32_t split_tokens;  /* 0 = automatic */
    uint64_t data_seed;     /* q/k/v contents */
    const uint32_t* fixed_ctx; /* NI_DRIVE_FIXED: context of each sequence after the append */
    uint32_t fixed_n;
    float kv_std;           /* k/v data ~ N(0, kv_std^2); 0 = 1 (q is always N(0,1)) */
    uint32_t profile_mask;  /* ni_kv_profile mask over the timed iterations; 0 = none */
    uint32_t qkv_rows;      /* NI_DRIVE_QKV: rows per projection */
    uint32_t fixed_rows;    /* NI_DRIVE_FIXED: rows appended and queried per sequence and iteration (0 = 1) */
    uint32_t qkv_wformat;   /* NI_DRIVE_QKV: weight format (NI_W_*), quantised on the host as the reference's
                               upload does (crates/metal/src/weights.rs:12-72) */
} ni_drive_opts;

typedef struct ni_drive_result {
    double seconds;         /* host wall clock over the timed iterations (synchronised both ends) */
    double gpu_seconds;     /* HIP events on the stream around the timed iterations */
    double bytes;           /* algorithmic bytes of the timed iterations */
    double seq_tokens;      /* serve: queried sequences; spec: tokens yielded (accepted + 1); summed */
    double host_us_per_step;/* host time to plan and enqueue one iteration */
    uint32_t steps;
    uint64_t launches;      /* data-path ABI calls in the timed region */
    double mean_live;       /* mean queried sequences per iteration */
    double mean_context;    /* mean context of queried sequences */
    double flops;           /* NI_DRIVE_QKV: matrix flops; NI_DRIVE_FIXED: attention flops (causal, 4 per
                             * query, key and element of C: q.k and p.v), of the timed iterations */
    double kernel_ms[NI_K_COUNT]; /* per ni_kernel_id over the timed iterations, when profiled */
    uint64_t kernel_launches[NI_K_COUNT];
    /* Host microseconds per call with the device idle, the median over up to
     * 20 more iterations after the timed ones, each after the stream drains:
     * the planning call (ni_kv_step, or ni_kv_step_begin) and
     * ni_kv_step_layer; 0 where the launch path makes no such call. */
    double idle_us_plan_call;
    double idle_us_layer_call;
    /* NI_DRIVE_SERVE: the scheduler's KV summary (ni_serve_get_stats) over
     * every iteration from the first (ramp included) to the last timed one */
    ni_serve_stats serve_stats;
} ni_drive_result;

int ni_drive_run(const ni_drive_opts* opts, ni_drive_result* result);
const char* ni_drive_last_error(void);

/* The device's memory interface as HIP reports it (hipDeviceGetAttribute:
 * peak memory clock in kHz and bus width in bits), for a harness that
 * states the HBM peak it measures against. */
int ni_drive_device_memory(int device, int* mem_clock_khz, int* bus_width_bits);

#ifdef __cplusplus
}
#endif
#endif /* NANOINFER_DRIVERS_H */
