/*
 * oracle.c -- CPU restatement of nanoinfer's paged f16 KV-cache path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (nanoinfer_amd/) links,
 * loads or calls this file.  It is used by tests/ (as the parity checker),
 * by __graft_entry__.smoke() (same) and by bench.py's cpu_baseline leg (the
 * reference's CPU path, timed beside the GPU).
 *
 * Every function restates one piece of the reference (Rust / MSL) and cites
 * the file:line it follows; paths are relative to the reference repository
 * (joshuaramkissoon/nanoinfer).  The arithmetic order is kept: sequential
 * f32 sums, separate multiply and add (build with -ffp-contract=off, Rust
 * never fuses), the same exp.
 *
 * Layout of the oracle's own paged pools is the reference's:
 *   pool[layer][kv_blocks][16][C] f16 bits  (crates/metal/src/batch.rs:166),
 *   slot(seq, pos) = table[seq*max_blocks + pos/16]*16 + pos%16
 *   (crates/metal/src/shaders/batch.metal:24-26).
 */
#include <math.h>
#include <pthread.h>
#include <stdatomic.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#if defined(__x86_64__)
#include <immintrin.h>
#endif

#define OR_KV_BLOCK 16u

/* ------------------------------------------------------------------------- */
/* f16 <-> f32                                                                */
/* ------------------------------------------------------------------------- */

/* crates/core/src/quant.rs:25-54 -- f32 -> f16 bits, round to nearest even,
 * subnormals, overflow to inf, NaN canonicalised to sign|0x7e00. */
uint16_t or_f32_to_f16(float x) {
    uint32_t b;
    memcpy(&b, &x, 4);
    uint16_t sign = (uint16_t)((b >> 16) & 0x8000u);
    int32_t exp = (int32_t)((b >> 23) & 0xffu);
    uint32_t man = b & 0x7fffffu;
    if (exp == 0xff) return (uint16_t)(sign | 0x7c00u | (man != 0 ? 0x200u : 0u));
    int32_t e = exp - 127 + 15;
    if (e >= 0x1f) return (uint16_t)(sign | 0x7c00u);
    if (e <= 0) {
        if (e < -10) return sign;
        uint32_t m = man | 0x800000u;
        uint32_t shift = (uint32_t)(14 - e);
        uint32_t half = 1u << (shift - 1);
        uint32_t rounded = (m + half - 1 + ((m >> shift) & 1u)) >> shift;
        return (uint16_t)(sign | rounded);
    }
    uint32_t v = ((uint32_t)e << 10) | (man >> 13);
    uint32_t rem = man & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (v & 1u))) v += 1;
    return (uint16_t)(sign | v);
}

/* crates/core/src/quant.rs:57-73 -- f16 bits -> f32, exact. */
float or_f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)(h & 0x8000u)) << 16;
    uint32_t exp = (h >> 10) & 0x1fu;
    uint32_t man = h & 0x3ffu;
    uint32_t bits;
    if (exp == 0 && man == 0) {
        bits = sign;
    } else if (exp == 0) {
        uint32_t lz = (uint32_t)__builtin_clz(man) - 22; /* zeros within the 10-bit field */
        uint32_t m = (man << (lz + 1)) & 0x3ffu;
        bits = sign | ((127u - 15u - lz) << 23) | (m << 13);
    } else if (exp == 0x1f) {
        bits = sign | 0x7f800000u | (man << 13);
    } else {
        bits = sign | ((exp + 127u - 15u) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* crates/core/src/stages/kv16.rs:61-82 (the non-aarch64 branch, :78-81). */
void or_narrow(const float* src, uint16_t* dst, size_t n) {
    for (size_t i = 0; i < n; i++) dst[i] = or_f32_to_f16(src[i]);
}

void or_widen(const uint16_t* src, float* dst, size_t n) {
    for (size_t i = 0; i < n; i++) dst[i] = or_f16_to_f32(src[i]);
}

/* Exhaustive pin of or_f32_to_f16 against an independent library routine:
 * x86 F16C (vcvtps2ph, round to nearest even) over the bit patterns
 * [start, start+count).  NaN inputs are excluded (F16C keeps payload bits,
 * the reference canonicalises) and counted separately; for those, the
 * canonical sign|0x7e00 is checked instead.  Returns mismatches. */
uint64_t or_f16_check_f16c(uint64_t start, uint64_t count, uint64_t* nan_seen) {
    uint64_t bad = 0, nans = 0;
#if defined(__x86_64__) && defined(__F16C__)
    for (uint64_t i = start; i < start + count; i++) {
        uint32_t b = (uint32_t)i;
        float f;
        memcpy(&f, &b, 4);
        uint16_t got = or_f32_to_f16(f);
        if ((b & 0x7fffffffu) > 0x7f800000u) {
            nans++;
            uint16_t want = (uint16_t)(((b >> 16) & 0x8000u) | 0x7e00u);
            if (got != want) bad++;
            continue;
        }
        uint16_t want = _cvtss_sh(f, _MM_FROUND_TO_NEAREST_INT);
        if (got != want) bad++;
    }
#else
    (void)start;
    (void)count;
    bad = (uint64_t)-1;
#endif
    if (nan_seen) *nan_seen = nans;
    return bad;
}

/* Compare device-produced f16 bits for the f32 bit patterns [start,
 * start+count) with or_f32_to_f16.  Returns mismatches; the first mismatching
 * pattern goes to *first_bad. */
uint64_t or_f16_compare_range(uint64_t start, uint64_t count, const uint16_t* got, uint64_t* first_bad) {
    uint64_t bad = 0;
    for (uint64_t i = 0; i < count; i++) {
        uint32_t b = (uint32_t)(start + i);
        float f;
        memcpy(&f, &b, 4);
        if (or_f32_to_f16(f) != got[i]) {
            if (bad == 0 && first_bad) *first_bad = start + i;
            bad++;
        }
    }
    return bad;
}

/* ------------------------------------------------------------------------- */
/* exp                                                                        */
/* ------------------------------------------------------------------------- */

/* crates/core/src/kernels/fastops.rs:55-63 -- Cody-Waite range reduction,
 * degree-6 Taylor polynomial, 2^n built in the exponent bits. */
float or_fast_exp(float x) {
    const float LN2_HI = 0.693359375f;
    const float LN2_LO = -2.1219444e-4f;
    const float LOG2_E = 1.44269504088896340736f;
    if (x != x) return x;                      /* Rust's clamp keeps NaN */
    x = x < -87.0f ? -87.0f : (x > 88.0f ? 88.0f : x);
    float n = nearbyintf(x * LOG2_E);          /* round_ties_even (default RNE mode) */
    float r = (x - n * LN2_HI) - n * LN2_LO;
    float p = 1.0f + r * (1.0f + r * (0.5f + r * (1.0f / 6.0f + r * (1.0f / 24.0f + r * (1.0f / 120.0f + r * (1.0f / 720.0f))))));
    uint32_t bits = ((uint32_t)((int32_t)n + 127)) << 23;
    float s;
    memcpy(&s, &bits, 4);
    return p * s;
}

/* ------------------------------------------------------------------------- */
/* contiguous attention (ground truth and the f16 CPU path)                   */
/* ------------------------------------------------------------------------- */

/* Rust's `Iterator::sum::<f32>()` folds from -0.0 left to right. */
static inline float dot_seq(const float* a, const float* b, size_t n) {
    float s = -0.0f;
    for (size_t i = 0; i < n; i++) s += a[i] * b[i];
    return s;
}

/* crates/core/src/kernels/reference.rs:65-76 -- softmax with std exp. */
void or_softmax(float* x, size_t n) {
    float max = -INFINITY;
    for (size_t i = 0; i < n; i++) max = fmaxf(max, x[i]);
    float sum = 0.0f;
    for (size_t i = 0; i < n; i++) {
        x[i] = expf(x[i] - max);
        sum += x[i];
    }
    float inv = 1.0f / sum;
    for (size_t i = 0; i < n; i++) x[i] *= inv;
}

/* crates/core/src/kernels/reference.rs:109-142 -- causal multi-head attention,
 * f32 rows with a stride (kernels/mod.rs:50-62), query i at q_pos0 + i sees
 * keys 0..=q_pos0+i.  `scores` holds >= q_pos0 + n_q floats. */
void or_reference_attention(float* out, const float* q, size_t q_stride, const float* k, size_t k_stride,
                            const float* v, size_t v_stride, size_t n_q, size_t q_pos0, size_t n_head,
                            size_t head_dim, float* scores) {
    size_t c = n_head * head_dim;
    float scale = 1.0f / sqrtf((float)head_dim);
    for (size_t i = 0; i < n_q; i++) {
        size_t n_kv = q_pos0 + i + 1;
        for (size_t h = 0; h < n_head; h++) {
            const float* qh = q + i * q_stride + h * head_dim;
            for (size_t j = 0; j < n_kv; j++) {
                scores[j] = dot_seq(qh, k + j * k_stride + h * head_dim, head_dim) * scale;
            }
            or_softmax(scores, n_kv);
            float* oh = out + i * c + h * head_dim;
            for (size_t d = 0; d < head_dim; d++) oh[d] = 0.0f;
            for (size_t j = 0; j < n_kv; j++) {
                const float* vh = v + j * v_stride + h * head_dim;
                for (size_t d = 0; d < head_dim; d++) oh[d] += scores[j] * vh[d];
            }
        }
    }
}

/* crates/core/src/kernels/unrolled.rs:26-46 -- 16 independent partial sums,
 * pairwise tree reduction, sequential remainder. */
static float dot_unrolled(const float* a, const float* b, size_t n) {
    float acc[16] = {0};
    size_t nc = n / 16 * 16;
    for (size_t i = 0; i < nc; i += 16)
        for (int j = 0; j < 16; j++) acc[j] += a[i + j] * b[i + j];
    for (int width = 8; width > 0; width /= 2)
        for (int j = 0; j < width; j++) acc[j] += acc[j + width];
    float s = acc[0];
    for (size_t i = nc; i < n; i++) s += a[i] * b[i];
    return s;
}

/* crates/core/src/kernels/fastops.rs:130-161 (attend_one) driven as
 * fastops.rs:167-213 with one thread. */
void or_fastops_attention(float* out, const float* q, size_t q_stride, const float* k, size_t k_stride,
                          const float* v, size_t v_stride, size_t n_q, size_t q_pos0, size_t n_head,
                          size_t head_dim, float* scores) {
    size_t c = n_head * head_dim;
    float scale = 1.0f / sqrtf((float)head_dim);
    for (size_t i = 0; i < n_q; i++) {
        size_t n_kv = q_pos0 + i + 1;
        for (size_t h = 0; h < n_head; h++) {
            const float* qh = q + i * q_stride + h * head_dim;
            float max = -INFINITY;
            for (size_t j = 0; j < n_kv; j++) {
                scores[j] = dot_unrolled(qh, k + j * k_stride + h * head_dim, head_dim) * scale;
                max = fmaxf(max, scores[j]);
            }
            float total = 0.0f;
            for (size_t j = 0; j < n_kv; j++) {
                scores[j] = or_fast_exp(scores[j] - max);
                total += scores[j];
            }
            float inv = 1.0f / total;
            float* oh = out + i * c + h * head_dim;
            for (size_t d = 0; d < head_dim; d++) oh[d] = 0.0f;
            for (size_t j = 0; j < n_kv; j++) {
                float p = scores[j] * inv;
                const float* vh = v + j * v_stride + h * head_dim;
                for (size_t d = 0; d < head_dim; d++) oh[d] += p * vh[d];
            }
        }
    }
}

/* crates/core/src/stages/kv16.rs:144-164 -- the portable (x86) f16 unit:
 * k, v are this head's n_kv contiguous hd-half rows. */
void or_attend_f16_portable(float* out, const float* q, const uint16_t* k, const uint16_t* v, size_t hd,
                            size_t n_kv, float* scores) {
    float scale = 1.0f / sqrtf((float)hd);
    float max = -INFINITY;
    for (size_t j = 0; j < n_kv; j++) {
        float s = -0.0f;
        for (size_t d = 0; d < hd; d++) s += q[d] * or_f16_to_f32(k[j * hd + d]);
        s = s * scale;
        scores[j] = s;
        max = fmaxf(max, s);
    }
    float total = 0.0f;
    for (size_t j = 0; j < n_kv; j++) {
        scores[j] = or_fast_exp(scores[j] - max);
        total += scores[j];
    }
    for (size_t d = 0; d < hd; d++) out[d] = 0.0f;
    for (size_t j = 0; j < n_kv; j++) {
        float p = scores[j] / total;
        for (size_t d = 0; d < hd; d++) out[d] += p * or_f16_to_f32(v[j * hd + d]);
    }
}

/* crates/core/src/stages/kv16.rs:168-204 with the cache of :33-58 -- causal
 * attention for n rows of qkv (stride 3C) at positions pos0.. over one layer
 * of a head-major f16 cache k/v [n_head][capacity][hd] (the caller passes the
 * layer's base).  Serial over units here; the threaded form is or_cpu_step. */
void or_kv16_attention(float* out, const float* qkv, const uint16_t* k, const uint16_t* v, size_t capacity,
                       size_t n, size_t pos0, size_t n_head, size_t hd, float* scores) {
    size_t c = n_head * hd;
    for (size_t u = 0; u < n * n_head; u++) {
        size_t i = u / n_head, h = u % n_head;
        size_t n_kv = pos0 + i + 1;
        size_t base = h * capacity * hd;
        or_attend_f16_portable(out + i * c + h * hd, qkv + i * 3 * c + h * hd, k + base, v + base, hd, n_kv, scores);
    }
}

/* ------------------------------------------------------------------------- */
/* paged KV: slot map, append, gather, attention                              */
/* ------------------------------------------------------------------------- */

/* crates/metal/src/shaders/batch.metal:24-26. */
uint32_t or_kv_slot(const uint32_t* table, uint32_t seq, uint32_t pos, uint32_t max_blocks) {
    return table[(size_t)seq * max_blocks + pos / OR_KV_BLOCK] * OR_KV_BLOCK + pos % OR_KV_BLOCK;
}

/* crates/metal/src/shaders/batch.metal:329-344 (b_kv_write), with half() as
 * quant.rs:25-54 and the layer offset of batch.rs:390.  One layer:
 * kp/vp point at that layer's pool [kv_blocks][16][C]; k/v rows at stride. */
void or_paged_append(uint16_t* kp, uint16_t* vp, const uint32_t* table, uint32_t max_blocks, const uint32_t* seqs,
                     const uint32_t* poss, size_t n, const float* k, const float* v, size_t stride, size_t c) {
    for (size_t t = 0; t < n; t++) {
        size_t slot = or_kv_slot(table, seqs[t], poss[t], max_blocks);
        for (size_t i = 0; i < c; i++) {
            kp[slot * c + i] = or_f32_to_f16(k[t * stride + i]);
            vp[slot * c + i] = or_f32_to_f16(v[t * stride + i]);
        }
    }
}

/* The reads of b_attn_split (batch.metal:377,392): K/V rows of (seq, pos)
 * through the table, copied out as f16 bits [n][C]. */
void or_paged_gather(uint16_t* k_out, uint16_t* v_out, const uint16_t* kp, const uint16_t* vp, const uint32_t* table,
                     uint32_t max_blocks, const uint32_t* seqs, const uint32_t* poss, size_t n, size_t c) {
    for (size_t t = 0; t < n; t++) {
        size_t slot = or_kv_slot(table, seqs[t], poss[t], max_blocks);
        memcpy(k_out + t * c, kp + slot * c, c * 2);
        memcpy(v_out + t * c, vp + slot * c, c * 2);
    }
}

/* kv16.rs:144-164 arithmetic with the keys found through kv_slot: identical
 * to or_attend_f16_portable on the gathered rows (tested), without the copy.
 * kp/vp: one layer's pool; head h of width hd; n_kv = pos + 1. */
static void attend_f16_paged(float* out, const float* q, const uint16_t* kp, const uint16_t* vp, size_t c, size_t h,
                             size_t hd, const uint32_t* table, uint32_t seq, uint32_t max_blocks, size_t n_kv,
                             float* scores) {
    float scale = 1.0f / sqrtf((float)hd);
    float max = -INFINITY;
    const uint32_t* trow = table + (size_t)seq * max_blocks;
    for (size_t j = 0; j < n_kv; j++) {
        size_t slot = (size_t)trow[j / OR_KV_BLOCK] * OR_KV_BLOCK + j % OR_KV_BLOCK;
        const uint16_t* kr = kp + slot * c + h * hd;
        float s = -0.0f;
        for (size_t d = 0; d < hd; d++) s += q[d] * or_f16_to_f32(kr[d]);
        s = s * scale;
        scores[j] = s;
        max = fmaxf(max, s);
    }
    float total = 0.0f;
    for (size_t j = 0; j < n_kv; j++) {
        scores[j] = or_fast_exp(scores[j] - max);
        total += scores[j];
    }
    for (size_t d = 0; d < hd; d++) out[d] = 0.0f;
    for (size_t j = 0; j < n_kv; j++) {
        size_t slot = (size_t)trow[j / OR_KV_BLOCK] * OR_KV_BLOCK + j % OR_KV_BLOCK;
        const uint16_t* vr = vp + slot * c + h * hd;
        float p = scores[j] / total;
        for (size_t d = 0; d < hd; d++) out[d] += p * or_f16_to_f32(vr[d]);
    }
}

/* Paged attention for n query rows of one layer: row t is (seqs[t], poss[t])
 * with n_kv = poss[t] + 1 (batch.metal:368), q row t at q + t*q_stride, out
 * row t at out + t*out_stride.  Each (row, head) is kv16.rs:144-164 over the
 * keys kv_slot finds.  `scores` holds >= max n_kv floats. */
void or_paged_attention(float* out, size_t out_stride, const float* q, size_t q_stride, const uint16_t* kp,
                        const uint16_t* vp, const uint32_t* table, uint32_t max_blocks, const uint32_t* seqs,
                        const uint32_t* poss, size_t n, size_t n_head, size_t hd, float* scores) {
    size_t c = n_head * hd;
    for (size_t t = 0; t < n; t++)
        for (size_t h = 0; h < n_head; h++)
            attend_f16_paged(out + t * out_stride + h * hd, q + t * q_stride + h * hd, kp, vp, c, h, hd, table,
                             seqs[t], max_blocks, (size_t)poss[t] + 1, scores);
}

/* ------------------------------------------------------------------------- */
/* split-K (flash-decoding) arithmetic                                        */
/* ------------------------------------------------------------------------- */

/* The split/merge of crates/metal/src/shaders/batch.metal:349-424 (and its
 * contiguous twin attn.metal:17-84), generalised to any head_dim and any
 * partition size P, in double precision: per partition s of keys
 * [sP, min(sP+P, n_kv)): m_s = max score, l_s = sum e^(x-m_s),
 * o_s = sum e^(x-m_s) v; then M = max m_s, L = sum l_s e^(m_s-M),
 * out = sum o_s e^(m_s-M) / L.  Scores are (q.k)/sqrt(hd).  K/V are f32
 * values (the caller widens f16).  P = 0 means one partition (unsplit
 * softmax).  Used to pin the log-sum-exp identity. */
void or_split_attention_f64(double* out, const float* q, const float* k, const float* v, size_t hd, size_t n_kv,
                            size_t part) {
    double scale = 1.0 / sqrt((double)hd);
    if (part == 0) part = n_kv;
    size_t n_parts = (n_kv + part - 1) / part;
    double* m = (double*)malloc(n_parts * sizeof(double));
    double* l = (double*)malloc(n_parts * sizeof(double));
    double* o = (double*)calloc(n_parts * hd, sizeof(double));
    for (size_t s = 0; s < n_parts; s++) {
        size_t j0 = s * part, j1 = j0 + part < n_kv ? j0 + part : n_kv;
        double mx = -INFINITY;
        for (size_t j = j0; j < j1; j++) {
            double x = 0;
            for (size_t d = 0; d < hd; d++) x += (double)q[d] * (double)k[j * hd + d];
            x *= scale;
            if (x > mx) mx = x;
        }
        double sum = 0;
        for (size_t j = j0; j < j1; j++) {
            double x = 0;
            for (size_t d = 0; d < hd; d++) x += (double)q[d] * (double)k[j * hd + d];
            double e = exp(x * scale - mx);
            sum += e;
            for (size_t d = 0; d < hd; d++) o[s * hd + d] += e * (double)v[j * hd + d];
        }
        m[s] = mx;
        l[s] = sum;
    }
    double M = -INFINITY;
    for (size_t s = 0; s < n_parts; s++)
        if (m[s] > M) M = m[s];
    double L = 0;
    for (size_t d = 0; d < hd; d++) out[d] = 0;
    for (size_t s = 0; s < n_parts; s++) {
        double w = exp(m[s] - M);
        L += l[s] * w;
        for (size_t d = 0; d < hd; d++) out[d] += o[s * hd + d] * w;
    }
    for (size_t d = 0; d < hd; d++) out[d] /= L;
    free(m);
    free(l);
    free(o);
}

/* ------------------------------------------------------------------------- */
/* page allocator (crates/metal/src/batch.rs:129-254)                          */
/* ------------------------------------------------------------------------- */

typedef struct {
    uint32_t kv_blocks, max_seqs, n_ctx, max_blocks;
    uint32_t* seq_len;   /* batch.rs:133 */
    uint8_t* live;       /* batch.rs:134 */
    uint32_t* blocks;    /* batch.rs:135, [max_seqs][max_blocks] */
    uint32_t* nblocks;
    uint32_t* free_list; /* batch.rs:136, a LIFO stack */
    uint32_t nfree;
} or_alloc;

/* batch.rs:159-194: free list (0..kv_blocks).rev(), so pop() yields 0, 1, 2...
 * `order` (optional) lists pages in the order pop() should yield them. */
or_alloc* or_alloc_new(uint32_t kv_blocks, uint32_t max_seqs, uint32_t n_ctx, const uint32_t* order) {
    or_alloc* a = (or_alloc*)calloc(1, sizeof(or_alloc));
    a->kv_blocks = kv_blocks;
    a->max_seqs = max_seqs;
    a->n_ctx = n_ctx;
    a->max_blocks = (n_ctx + OR_KV_BLOCK - 1) / OR_KV_BLOCK; /* batch.rs:164 */
    a->seq_len = (uint32_t*)calloc(max_seqs, 4);
    a->live = (uint8_t*)calloc(max_seqs, 1);
    a->blocks = (uint32_t*)calloc((size_t)max_seqs * a->max_blocks, 4);
    a->nblocks = (uint32_t*)calloc(max_seqs, 4);
    a->free_list = (uint32_t*)malloc((size_t)kv_blocks * 4);
    for (uint32_t i = 0; i < kv_blocks; i++) a->free_list[i] = order ? order[kv_blocks - 1 - i] : kv_blocks - 1 - i;
    a->nfree = kv_blocks;
    return a;
}

void or_alloc_free(or_alloc* a) {
    if (!a) return;
    free(a->seq_len);
    free(a->live);
    free(a->blocks);
    free(a->nblocks);
    free(a->free_list);
    free(a);
}

/* batch.rs:201-206 -- first non-live slot; -1 for None. */
int64_t or_alloc_add_seq(or_alloc* a) {
    for (uint32_t s = 0; s < a->max_seqs; s++) {
        if (!a->live[s]) {
            a->live[s] = 1;
            a->seq_len[s] = 0;
            return s;
        }
    }
    return -1;
}

/* batch.rs:220-227 -- returns -1 where the reference's assert fires. */
int or_alloc_truncate(or_alloc* a, uint32_t s, uint32_t len) {
    if (len > a->seq_len[s]) return -1;
    a->seq_len[s] = len;
    uint32_t keep = (len + OR_KV_BLOCK - 1) / OR_KV_BLOCK;
    while (a->nblocks[s] > keep) {
        a->nblocks[s]--;
        a->free_list[a->nfree++] = a->blocks[(size_t)s * a->max_blocks + a->nblocks[s]];
    }
    return 0;
}

/* batch.rs:209-212. */
void or_alloc_free_seq(or_alloc* a, uint32_t s) {
    or_alloc_truncate(a, s, 0);
    a->live[s] = 0;
}

/* batch.rs:243-254 -- 0 ok, 1 context full, 2 pool exhausted (pages popped
 * before the pool ran dry stay with the sequence, as in the reference). */
int or_alloc_ensure(or_alloc* a, uint32_t s, uint32_t len) {
    if (len > a->n_ctx) return 1;
    while (a->nblocks[s] * OR_KV_BLOCK < len) {
        if (a->nfree == 0) return 2;
        uint32_t b = a->free_list[--a->nfree];
        a->blocks[(size_t)s * a->max_blocks + a->nblocks[s]] = b;
        a->nblocks[s]++;
    }
    return 0;
}

/* batch.rs:270 -- seq_len += n once the forward has run. */
void or_alloc_commit(or_alloc* a, uint32_t s, uint32_t n) { a->seq_len[s] += n; }

uint32_t or_alloc_seq_len(const or_alloc* a, uint32_t s) { return a->seq_len[s]; }
int or_alloc_live(const or_alloc* a, uint32_t s) { return a->live[s]; }
/* batch.rs:230-240. */
uint32_t or_alloc_blocks_used(const or_alloc* a) { return a->kv_blocks - a->nfree; }
uint32_t or_alloc_free_block_count(const or_alloc* a) { return a->nfree; }
uint32_t or_alloc_block_table(const or_alloc* a, uint32_t s, uint32_t* out) {
    memcpy(out, a->blocks + (size_t)s * a->max_blocks, (size_t)a->nblocks[s] * 4);
    return a->nblocks[s];
}
/* The dense table [max_seqs][max_blocks] the GPU side of the reference
 * mirrors (batch.rs:178,250); unused entries are 0. */
const uint32_t* or_alloc_table(const or_alloc* a) { return a->blocks; }
uint32_t or_alloc_max_blocks(const or_alloc* a) { return a->max_blocks; }

/* ------------------------------------------------------------------------- */
/* threaded CPU step (the reported CPU baseline)                              */
/* ------------------------------------------------------------------------- */

/* A fixed pool of workers claiming chunk indices with one fetch_add each
 * (crates/core/src/fastpool.rs:1-19; lowlat.rs:35-40). */
typedef void (*or_job_fn)(void* ctx, size_t chunk);

typedef struct or_pool {
    int threads;
    pthread_t* tid;
    pthread_mutex_t mu;
    pthread_cond_t cv_go, cv_done;
    uint64_t generation;
    int active;      /* workers still running the current job */
    int quit;
    or_job_fn fn;
    void* ctx;
    size_t n_chunks;
    atomic_size_t next;
} or_pool;

static void pool_drain(or_pool* p) {
    for (;;) {
        size_t c = atomic_fetch_add(&p->next, 1);
        if (c >= p->n_chunks) break;
        p->fn(p->ctx, c);
    }
}

static void* pool_worker(void* arg) {
    or_pool* p = (or_pool*)arg;
    uint64_t seen = 0;
    pthread_mutex_lock(&p->mu);
    for (;;) {
        while (p->generation == seen && !p->quit) pthread_cond_wait(&p->cv_go, &p->mu);
        if (p->quit) break;
        seen = p->generation;
        pthread_mutex_unlock(&p->mu);
        pool_drain(p);
        pthread_mutex_lock(&p->mu);
        if (--p->active == 0) pthread_cond_signal(&p->cv_done);
    }
    pthread_mutex_unlock(&p->mu);
    return NULL;
}

or_pool* or_pool_new(int threads) {
    if (threads < 1) threads = 1;
    or_pool* p = (or_pool*)calloc(1, sizeof(or_pool));
    p->threads = threads;
    pthread_mutex_init(&p->mu, NULL);
    pthread_cond_init(&p->cv_go, NULL);
    pthread_cond_init(&p->cv_done, NULL);
    p->tid = (pthread_t*)calloc((size_t)threads, sizeof(pthread_t));
    for (int i = 1; i < threads; i++) pthread_create(&p->tid[i], NULL, pool_worker, p);
    return p;
}

int or_pool_threads(const or_pool* p) { return p->threads; }

/* lowlat::par_for: run fn(ctx, c) for c in 0..n_chunks on all threads (the
 * caller is worker 0) and return when every chunk is done. */
static void pool_run(or_pool* p, size_t n_chunks, or_job_fn fn, void* ctx) {
    if (p->threads == 1 || n_chunks <= 1) {
        for (size_t c = 0; c < n_chunks; c++) fn(ctx, c);
        return;
    }
    pthread_mutex_lock(&p->mu);
    p->fn = fn;
    p->ctx = ctx;
    p->n_chunks = n_chunks;
    atomic_store(&p->next, 0);
    p->active = p->threads - 1;
    p->generation++;
    pthread_cond_broadcast(&p->cv_go);
    pthread_mutex_unlock(&p->mu);
    pool_drain(p);
    pthread_mutex_lock(&p->mu);
    while (p->active > 0) pthread_cond_wait(&p->cv_done, &p->mu);
    pthread_mutex_unlock(&p->mu);
}

void or_pool_free(or_pool* p) {
    if (!p) return;
    pthread_mutex_lock(&p->mu);
    p->quit = 1;
    pthread_cond_broadcast(&p->cv_go);
    pthread_mutex_unlock(&p->mu);
    for (int i = 1; i < p->threads; i++) pthread_join(p->tid[i], NULL);
    free(p->tid);
    pthread_mutex_destroy(&p->mu);
    pthread_cond_destroy(&p->cv_go);
    pthread_cond_destroy(&p->cv_done);
    free(p);
}

typedef struct {
    float* out;
    size_t out_stride;
    const float* q;
    size_t q_stride;
    const uint16_t* kp;
    const uint16_t* vp;
    const uint32_t* table;
    uint32_t max_blocks;
    const uint32_t* seqs;
    const uint32_t* poss;
    const uint32_t* qrows; /* rows that get a query */
    size_t n_units, per, n_head, hd, scratch_len;
} attn_job;

static void attn_chunk(void* ctx, size_t ch) {
    attn_job* j = (attn_job*)ctx;
    float stack[1024];
    float* scratch = j->scratch_len <= 1024 ? stack : (float*)malloc(j->scratch_len * sizeof(float));
    size_t c = j->n_head * j->hd;
    size_t u1 = (ch + 1) * j->per < j->n_units ? (ch + 1) * j->per : j->n_units;
    for (size_t u = ch * j->per; u < u1; u++) {
        size_t i = u / j->n_head, h = u % j->n_head;
        size_t t = j->qrows[i];
        attend_f16_paged(j->out + t * j->out_stride + h * j->hd, j->q + t * j->q_stride + h * j->hd, j->kp, j->vp, c, h,
                         j->hd, j->table, j->seqs[t], j->max_blocks, (size_t)j->poss[t] + 1, scratch);
    }
    if (scratch != stack) free(scratch);
}

/* One step of the paged hot path on the CPU, restating the reference's x86
 * CPU path per layer (kv16.rs:214-263): append every row (narrow, serial,
 * :246-258), then attention over (query row, head) units split into
 * ceil(units / (threads * CHUNKS_PER_THREAD)) sized chunks (kv16.rs:189-203,
 * lowlat.rs:21) on the pool, each unit kv16.rs:144-164 over the keys the
 * table finds.
 *
 * Pools: kp/vp [n_layer][kv_blocks][16][C].  Row t: (seqs[t], poss[t]);
 * q/k/v/out row t of layer l at base + l*layer_stride + t*row_stride.
 * qrows[0..n_q) lists the rows that get attention. */
void or_cpu_step(or_pool* pool, uint16_t* kp, uint16_t* vp, size_t kv_blocks, const uint32_t* table,
                 uint32_t max_blocks, const uint32_t* seqs, const uint32_t* poss, size_t n, const uint32_t* qrows,
                 size_t n_q, const float* q, const float* k, const float* v, size_t row_stride, size_t layer_stride,
                 float* out, size_t out_row_stride, size_t out_layer_stride, size_t n_layer, size_t n_head,
                 size_t hd) {
    size_t c = n_head * hd;
    size_t layer_halves = kv_blocks * OR_KV_BLOCK * c;
    size_t max_kv = 0;
    for (size_t t = 0; t < n; t++)
        if ((size_t)poss[t] + 1 > max_kv) max_kv = (size_t)poss[t] + 1;
    for (size_t l = 0; l < n_layer; l++) {
        uint16_t* kl = kp + l * layer_halves;
        uint16_t* vl = vp + l * layer_halves;
        or_paged_append(kl, vl, table, max_blocks, seqs, poss, n, k + l * layer_stride, v + l * layer_stride,
                        row_stride, c);
        attn_job j;
        j.out = out + l * out_layer_stride;
        j.out_stride = out_row_stride;
        j.q = q + l * layer_stride;
        j.q_stride = row_stride;
        j.kp = kl;
        j.vp = vl;
        j.table = table;
        j.max_blocks = max_blocks;
        j.seqs = seqs;
        j.poss = poss;
        j.qrows = qrows;
        j.n_units = n_q * n_head;
        j.n_head = n_head;
        j.hd = hd;
        j.scratch_len = max_kv;
        size_t threads = (size_t)(pool ? pool->threads : 1);
        size_t per = (j.n_units + threads * 4 - 1) / (threads * 4);
        if (per == 0) per = 1;
        j.per = per;
        size_t chunks = (j.n_units + per - 1) / per;
        if (pool)
            pool_run(pool, chunks, attn_chunk, &j);
        else
            for (size_t ch = 0; ch < chunks; ch++) attn_chunk(&j, ch);
    }
}

/* ------------------------------------------------------------------------- */
/* QKV projection (the matvec whose epilogue appends K/V)                     */
/* ------------------------------------------------------------------------- */

/* crates/metal/src/shaders/batch.metal:94-165 (matvec_batch): for each token t
 * and output row f, s = sum_j w[f][j] * x[t][j] (+ bias[f]) with W stored
 * [d_out][d_in] row-major.  The reference sums in f32 in its lanes' order;
 * this restatement sums in double, the ground truth an f32 kernel is held to
 * within f32 rounding.  out [n][d_out]. */
void or_matvec_f64(double* out, const float* x, size_t x_stride, const float* w, const float* bias, size_t n,
                   size_t d_in, size_t d_out) {
    for (size_t t = 0; t < n; t++)
        for (size_t f = 0; f < d_out; f++) {
            double s = 0;
            for (size_t j = 0; j < d_in; j++) s += (double)w[f * d_in + j] * (double)x[t * x_stride + j];
            out[t * d_out + f] = s + (bias ? (double)bias[f] : 0.0);
        }
}

/* ------------------------------------------------------------------------- */
/* Weight formats of the projection (crates/metal/src/weights.rs)             */
/* ------------------------------------------------------------------------- */

/* quantize_q8_0, weights.rs:12-27, over n weights (n a multiple of 32), into
 * out: [n] int8 quants, then [n / 32] little-endian f16 scales.  Per block:
 * amax = max |w| (f32 max fold), d = amax / 127, id = d > 0 ? 1 / d : 0,
 * q = (w * id).round() as i8 -- Rust's round is half away from zero, `as`
 * saturates (and takes NaN to 0); the scale is f16::from_f32(d) (round to
 * nearest even, or_f32_to_f16).  Returns the bytes written, n + n / 16. */
size_t or_quantize_q8_0(const float* w, size_t n, uint8_t* out) {
    uint8_t* sc = out + n;
    for (size_t b = 0; b < n / 32; b++) {
        const float* blk = w + 32 * b;
        float amax = 0.0f;
        for (int i = 0; i < 32; i++) amax = fmaxf(amax, fabsf(blk[i]));
        volatile float d = amax / 127.0f;
        volatile float id = d > 0.0f ? 1.0f / d : 0.0f;
        for (int i = 0; i < 32; i++) {
            volatile float t = blk[i] * id;
            float r = roundf(t);
            int32_t q = r != r ? 0 : r >= 127.0f ? 127 : r <= -128.0f ? -128 : (int32_t)r;
            out[32 * b + i] = (uint8_t)(int8_t)q;
        }
        uint16_t h = or_f32_to_f16(d);
        sc[2 * b] = (uint8_t)(h & 0xff);
        sc[2 * b + 1] = (uint8_t)(h >> 8);
    }
    return n + n / 16;
}

/* quantize_q4_0, weights.rs:54-72 (GGML's rounding): per block of 32, max =
 * the value of largest magnitude (the first one on ties: replaced only when
 * |v| > |max|), d = max / -8, id = d != 0 ? 1 / d : 0, q(v) = ((v * id + 8.5)
 * as i32).clamp(0, 15) (`as` truncates toward zero, saturating, NaN to 0);
 * byte i of the block = q(w[i]) | q(w[i + 16]) << 4.  Then the [n / 32] f16
 * scales.  Returns the bytes written, n / 2 + n / 16. */
size_t or_quantize_q4_0(const float* w, size_t n, uint8_t* out) {
    uint8_t* sc = out + n / 2;
    for (size_t b = 0; b < n / 32; b++) {
        const float* blk = w + 32 * b;
        float mx = 0.0f;
        for (int i = 0; i < 32; i++)
            if (fabsf(blk[i]) > fabsf(mx)) mx = blk[i];
        volatile float d = mx / -8.0f;
        volatile float id = d != 0.0f ? 1.0f / d : 0.0f;
        uint8_t q[32];
        for (int i = 0; i < 32; i++) {
            volatile float t = blk[i] * id;
            volatile float u = t + 8.5f;
            float tr = truncf(u);
            int32_t v = u != u ? 0 : tr >= 2147483647.0f ? 2147483647 : tr <= -2147483648.0f ? (-2147483647 - 1) : (int32_t)tr;
            q[i] = (uint8_t)(v < 0 ? 0 : v > 15 ? 15 : v);
        }
        for (int i = 0; i < 16; i++) out[16 * b + i] = (uint8_t)(q[i] | (q[i + 16] << 4));
        uint16_t h = or_f32_to_f16(d);
        sc[2 * b] = (uint8_t)(h & 0xff);
        sc[2 * b + 1] = (uint8_t)(h >> 8);
    }
    return n / 2 + n / 16;
}

/* dequantize, weights.rs:29-52, for fmt 2 (Q8_0: q * d) and 3 (Q4_0:
 * (nibble - 8) * d, element j of a block in byte j % 16, low nibble for
 * j < 16), each product in f32; fmt 1 (F16) widens f16 bits; fmt 0 copies. */
void or_dequantize(const uint8_t* q, size_t n, int fmt, float* out) {
    if (fmt == 0) {
        memcpy(out, q, n * sizeof(float));
        return;
    }
    if (fmt == 1) {
        for (size_t i = 0; i < n; i++) out[i] = or_f16_to_f32((uint16_t)(q[2 * i] | (q[2 * i + 1] << 8)));
        return;
    }
    const size_t qbytes = fmt == 2 ? n : n / 2;
    for (size_t i = 0; i < n; i++) {
        const size_t b = i / 32, j = i % 32;
        const uint16_t h = (uint16_t)(q[qbytes + 2 * b] | (q[qbytes + 2 * b + 1] << 8));
        const float d = or_f16_to_f32(h);
        float v;
        if (fmt == 2) {
            v = (float)(int8_t)q[i];
        } else {
            const uint8_t byte = q[b * 16 + j % 16];
            v = (float)(j < 16 ? (byte & 15) : (byte >> 4)) - 8.0f;
        }
        volatile float r = v * d;
        out[i] = r;
    }
}

/* ------------------------------------------------------------------------- */
/* Q8 KV cache (crates/metal/src/shaders/kv8.metal)                           */
/* ------------------------------------------------------------------------- */

/* kv_quant8, kv8.metal:15-48, for one (position, head) of n values:
 * amax = max |x|, scale = amax / 127 (f32), inv = scale > 0 ? 1 / scale : 0,
 * q = clamp(rint(x * inv), -127, 127) with rint rounding half to even.
 * Returns the scale. */
float or_q8_quantize(const float* x, size_t n, int8_t* q) {
    float amax = 0.0f;
    for (size_t i = 0; i < n; i++) {
        float a = fabsf(x[i]);
        if (a > amax) amax = a;
    }
    volatile float scale = amax / 127.0f; /* volatile: keep both divisions in f32 */
    volatile float inv = scale > 0.0f ? 1.0f / scale : 0.0f;
    for (size_t i = 0; i < n; i++) {
        float y = nearbyintf(x[i] * inv);
        if (y < -127.0f) y = -127.0f;
        if (y > 127.0f) y = 127.0f;
        q[i] = (int8_t)y;
    }
    return scale;
}

/* The paged Q8 cache in the reference's row layout: values [kv_blocks*16][C]
 * int8 and scales [kv_blocks*16][n_head] f32 per layer (kv8.metal:11-12 with
 * the position replaced by kv_slot, batch.metal:24-26).  Appends rows of
 * f32 k/v at `stride`. */
void or_paged_q8_append(int8_t* kq, int8_t* vq, float* ks, float* vs, const uint32_t* table, uint32_t max_blocks,
                        const uint32_t* seqs, const uint32_t* poss, size_t n, const float* k, const float* v,
                        size_t stride, size_t n_head, size_t hd) {
    size_t c = n_head * hd;
    for (size_t t = 0; t < n; t++) {
        size_t slot = or_kv_slot(table, seqs[t], poss[t], max_blocks);
        for (size_t h = 0; h < n_head; h++) {
            ks[slot * n_head + h] = or_q8_quantize(k + t * stride + h * hd, hd, kq + slot * c + h * hd);
            vs[slot * n_head + h] = or_q8_quantize(v + t * stride + h * hd, hd, vq + slot * c + h * hd);
        }
    }
}

/* attn_decode_split_q8 (kv8.metal:50-95) over pages, in double: for row
 * (seq, pos) and head h, s_j = (sum_d q[d] k_j[d]) * ks_j / sqrt(hd) over
 * keys j = 0..pos, p = softmax(s), out[d] = sum_j p_j vs_j v_j[d]. */
void or_paged_q8_attention(float* out, size_t out_stride, const float* q, size_t q_stride, const int8_t* kq,
                           const int8_t* vq, const float* ks, const float* vs, const uint32_t* table,
                           uint32_t max_blocks, const uint32_t* seqs, const uint32_t* poss, size_t n, size_t n_head,
                           size_t hd, double* scores) {
    size_t c = n_head * hd;
    double scale = 1.0 / sqrt((double)hd);
    for (size_t t = 0; t < n; t++)
        for (size_t h = 0; h < n_head; h++) {
            size_t n_kv = (size_t)poss[t] + 1;
            const float* qr = q + t * q_stride + h * hd;
            double mx = -INFINITY;
            for (size_t j = 0; j < n_kv; j++) {
                size_t slot = or_kv_slot(table, seqs[t], (uint32_t)j, max_blocks);
                double s = 0;
                for (size_t d = 0; d < hd; d++) s += (double)qr[d] * (double)kq[slot * c + h * hd + d];
                s *= (double)ks[slot * n_head + h] * scale;
                scores[j] = s;
                if (s > mx) mx = s;
            }
            double sum = 0;
            for (size_t j = 0; j < n_kv; j++) {
                scores[j] = exp(scores[j] - mx);
                sum += scores[j];
            }
            for (size_t d = 0; d < hd; d++) {
                double acc = 0;
                for (size_t j = 0; j < n_kv; j++) {
                    size_t slot = or_kv_slot(table, seqs[t], (uint32_t)j, max_blocks);
                    acc += scores[j] * (double)vs[slot * n_head + h] * (double)vq[slot * c + h * hd + d];
                }
                out[t * out_stride + h * hd + d] = (float)(acc / sum);
            }
        }
}
