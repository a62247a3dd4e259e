// ni_drive -- command-line front end of ni_drive_run (nanoinfer_drivers.h):
// the config-3 continuous-batching trace (`serve`) or the config-5 verify
// loop (`spec`) on the device, launched per step or per layer, printed as
// one JSON line.
//
//   ni_drive [serve|spec|qkv|prefill] [--per-layer|--step-layers] [--steps K] [--warmup W]
//            [--ramp R] [--split T] [--all-prompt-rows] [--seed S] [--rows N] [--q8]
//            [--wfmt f32|f16|q8_0|q4_0]
//
// --ramp: R append-only iterations (no attention) before the warmup.
//
// --per-layer: ni_kv_append + ni_paged_decode_attention per layer;
// --step-layers: ni_kv_step_begin, one ni_kv_step_layer per layer,
// ni_kv_step_end; neither: one ni_kv_step per iteration (all layers).
//
// prefill: 16 sequences append and attend N-row prompts (default 512) from
// empty, every row queried, rolled back each iteration.
//
// qkv: the QKV projection of N rows per layer with K/V appended in its
// epilogue, weights in --wfmt; --per-layer runs the unfused path (f32
// projection + append).
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <algorithm>
#include <string>

#include "nanoinfer_drivers.h"

static uint32_t pages(uint32_t n) { return (n + NI_KV_BLOCK - 1) / NI_KV_BLOCK; }

int main(int argc, char** argv) {
    ni_drive_opts o{};
    std::string workload = "serve";
    bool q8 = false;  // the Q8 cache (NI_KV_Q8)
    o.launch = NI_DRIVE_STEP;
    o.steps = 2000;
    o.warmup = 300;
    o.data_seed = 7;
    o.serve = ni_serve_opts{7, 1.0, 100000, 64, 32, 512, 16, 256, 256, 512, 0};
    for (int i = 1; i < argc; i++) {
        const char* a = argv[i];
        auto val = [&](const char* name) -> const char* {
            if (i + 1 >= argc) {
                fprintf(stderr, "ni_drive: %s needs a value\n", name);
                exit(2);
            }
            return argv[++i];
        };
        if (!strcmp(a, "serve") || !strcmp(a, "spec") || !strcmp(a, "qkv") || !strcmp(a, "prefill")) workload = a;
        else if (!strcmp(a, "--rows")) o.qkv_rows = (uint32_t)atoi(val(a));
        else if (!strcmp(a, "--q8")) q8 = true;
        else if (!strcmp(a, "--wfmt")) {  // qkv: f32 (default), f16, q8_0, q4_0
            const char* f = val(a);
            if (!strcmp(f, "f32")) o.qkv_wformat = NI_W_F32;
            else if (!strcmp(f, "f16")) o.qkv_wformat = NI_W_F16;
            else if (!strcmp(f, "q8_0")) o.qkv_wformat = NI_W_Q8_0;
            else if (!strcmp(f, "q4_0")) o.qkv_wformat = NI_W_Q4_0;
            else {
                fprintf(stderr, "ni_drive: --wfmt must be f32, f16, q8_0 or q4_0 (got \"%s\")\n", f);
                return 2;
            }
        }
        else if (!strcmp(a, "--per-layer")) o.launch = NI_DRIVE_PER_LAYER;
        else if (!strcmp(a, "--step-layers")) o.launch = NI_DRIVE_STEP_LAYERS;
        else if (!strcmp(a, "--all-prompt-rows")) o.serve.query_all_prompt_rows = 1;
        else if (!strcmp(a, "--steps")) o.steps = (uint32_t)atoi(val(a));
        else if (!strcmp(a, "--warmup")) o.warmup = (uint32_t)atoi(val(a));
        else if (!strcmp(a, "--ramp")) o.ramp = (uint32_t)atoi(val(a));
        else if (!strcmp(a, "--split")) o.split_tokens = (uint32_t)atoi(val(a));
        else if (!strcmp(a, "--seed")) o.data_seed = o.serve.seed = strtoull(val(a), nullptr, 10);
        else {
            fprintf(stderr, "usage: ni_drive [serve|spec|qkv|prefill] [--per-layer|--step-layers] [--steps K] [--warmup W] "
                            "[--ramp R] [--split T] [--all-prompt-rows] [--seed S] [--rows N] [--q8] [--wfmt F]\n");
            return 2;
        }
    }
    o.kv.n_layer = 12;
    o.kv.n_head = 12;
    o.kv.head_dim = 64;
    if (workload == "serve") {
        // metal_serve.rs:485: max_batch * pages(prompt_max + out_max) + 8 pages.
        o.workload = NI_DRIVE_SERVE;
        o.kv.kv_pages = o.serve.max_batch * pages(o.serve.prompt_max + o.serve.out_max) + 8;
        o.kv.max_seqs = o.serve.max_batch;
        o.kv.max_ctx = 1024;
        o.kv.max_rows = o.serve.max_rows;
    } else if (workload == "prefill") {
        static uint32_t ctx[16];
        const uint32_t P = o.qkv_rows ? o.qkv_rows : 512;
        for (uint32_t& c : ctx) c = P;
        o.qkv_rows = 0;
        o.workload = NI_DRIVE_FIXED;
        o.fixed_ctx = ctx;
        o.fixed_n = 16;
        o.fixed_rows = P;
        o.kv.kv_pages = 16 * pages(P) + 8;
        o.kv.max_seqs = 16;
        o.kv.max_ctx = std::max<uint32_t>(1024, P);
        o.kv.max_rows = 16 * P;
    } else if (workload == "qkv") {
        o.workload = NI_DRIVE_QKV;
        if (o.qkv_rows == 0) o.qkv_rows = 64;
        o.kv.kv_pages = 64 * 64;
        o.kv.max_seqs = 64;
        o.kv.max_ctx = 1024;
        o.kv.max_rows = 512;
    } else {
        o.workload = NI_DRIVE_SPEC;
        o.spec_seqs = 32;
        o.spec_ctx_min = 128;
        o.spec_ctx_max = 1024;
        o.spec_k = 4;
        o.spec_seed = 5;
        o.spec_window = 64;
        o.kv.max_ctx = 2048;
        o.kv.kv_pages = o.spec_seqs * pages(o.kv.max_ctx);
        o.kv.max_seqs = o.spec_seqs;
        o.kv.max_rows = 512;
    }
    if (q8) o.kv.flags |= NI_KV_Q8;
    ni_drive_result r{};
    if (int rc = ni_drive_run(&o, &r)) {
        fprintf(stderr, "ni_drive: %s (status %d)\n", ni_drive_last_error(), rc);
        return 1;
    }
    const double gbs = r.bytes / r.seconds / 1e9;
    if (workload == "qkv")
        fprintf(stderr, "ni_drive: qkv %u rows: %.2f TFLOP/s, %.3f ms per iteration (12 layers)\n", o.qkv_rows,
                r.flops / r.seconds / 1e12, r.seconds / r.steps * 1e3);
    if (workload == "prefill")
        fprintf(stderr, "ni_drive: prefill 16 x %u rows: %.2f attention TFLOP/s over the whole step, %.3f ms per step\n",
                o.fixed_rows, r.flops / r.seconds / 1e12, r.seconds / r.steps * 1e3);
    printf("{\"driver\": \"ni_drive\", \"workload\": \"%s\", \"launch\": \"%s\", \"steps\": %u, \"ramp\": %u, \"warmup\": %u, "
           "\"value\": %.2f, \"unit\": \"GB/s\", \"pct_of_peak\": %.2f, \"ms_per_step\": %.5f, "
           "\"gpu_ms_per_step\": %.5f, \"host_us_per_step\": %.1f, \"abi_calls_per_step\": %.1f, "
           "\"seq_tokens_per_s\": %.1f, \"algorithmic_bytes_per_step\": %.0f, \"mean_live\": %.2f, "
           "\"mean_context\": %.1f, \"kv\": \"%s\", \"idle_us_plan_call\": %.2f, \"idle_us_layer_call\": %.2f}\n",
           workload.c_str(), o.launch == NI_DRIVE_STEP ? "step" : o.launch == NI_DRIVE_PER_LAYER ? "per-layer" : "step-layers", r.steps, o.ramp, o.warmup, gbs,
           100.0 * gbs / 8000.0, r.seconds / r.steps * 1e3, r.gpu_seconds / r.steps * 1e3, r.host_us_per_step,
           (double)r.launches / r.steps, r.seq_tokens / r.seconds, r.bytes / r.steps, r.mean_live, r.mean_context, q8 ? "q8" : "f16",
           r.idle_us_plan_call, r.idle_us_layer_call);
    return 0;
}
