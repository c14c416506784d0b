/*
 * focr_oracle.c — CPU oracle (test infrastructure only; see focr_oracle.h).
 *
 * A plain-C restatement of franken_ocr's scalar semantics for the quantized
 * decoder hot path. Build flags: -O2 -ffp-contract=off (no FMA contraction;
 * every f32 operation rounds separately, as in Rust).
 */
#include "focr_oracle.h"

#include <float.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

/* checked_len (src/simd/scalar.rs:63-67): reject shape products that overflow */
static int mul_ok(size_t a, size_t b, size_t* out) {
    if (a != 0 && b > SIZE_MAX / a) return 0;
    *out = a * b;
    return 1;
}

/* Rust `f32 as i8` after a clamp into [lo, hi]: NaN -> 0 (saturating cast). */
static int8_t clamp_cast_i8(float r, float lo, float hi) {
    if (r != r) return 0;
    if (r < lo) r = lo;
    if (r > hi) r = hi;
    return (int8_t)(int)r;
}

/* ---- src/simd/scalar.rs:78-116 / :129-166 -------------------------------
 * out[i*N+o] += sum_p A[i*K+p] * B[o*K+p]; i32 accumulation; B is
 * output-channel-major. Wrapping add (release-mode Rust). */
int oracle_igemm_s8s8(const int8_t* a, const int8_t* b, size_t m, size_t k, size_t n,
                      int32_t* out) {
    size_t t;
    if (!mul_ok(m, k, &t) || !mul_ok(n, k, &t) || !mul_ok(m, n, &t)) return ORACLE_E_SHAPE;
    for (size_t i = 0; i < m; ++i) {
        for (size_t o = 0; o < n; ++o) {
            uint32_t acc = 0;
            for (size_t p = 0; p < k; ++p)
                acc += (uint32_t)((int32_t)a[i * k + p] * (int32_t)b[o * k + p]);
            out[i * n + o] = (int32_t)((uint32_t)out[i * n + o] + acc);
        }
    }
    return ORACLE_OK;
}

int oracle_igemm_u8s8(const uint8_t* a, const int8_t* b, size_t m, size_t k, size_t n,
                      int32_t* out) {
    size_t t;
    if (!mul_ok(m, k, &t) || !mul_ok(n, k, &t) || !mul_ok(m, n, &t)) return ORACLE_E_SHAPE;
    for (size_t i = 0; i < m; ++i) {
        for (size_t o = 0; o < n; ++o) {
            uint32_t acc = 0;
            for (size_t p = 0; p < k; ++p)
                acc += (uint32_t)((int32_t)a[i * k + p] * (int32_t)b[o * k + p]);
            out[i * n + o] = (int32_t)((uint32_t)out[i * n + o] + acc);
        }
    }
    return ORACLE_OK;
}

/* ---- src/simd/dispatch.rs:340-347 xs32, :352-368 SELFTEST_SHAPES -------- */
uint32_t oracle_xs32(uint32_t* state) {
    uint32_t s = *state;
    s ^= s << 13;
    s ^= s >> 17;
    s ^= s << 5;
    *state = s;
    return s;
}

typedef struct {
    const char* label;
    size_t m, k, n;
    uint32_t seed;
} selftest_shape;

static const selftest_shape k_shapes[] = {
    {"edge:1x1x1", 1, 1, 1, 0x11111111u},
    {"edge:1x7x3", 1, 7, 3, 0x22222222u},
    {"edge:2x3x2", 2, 3, 2, 0x33333333u},
    {"ktail:1x15x8", 1, 15, 8, 0x44444444u},
    {"ktail:1x16x8", 1, 16, 8, 0x55555555u},
    {"ktail:1x17x8", 1, 17, 8, 0x66666666u},
    {"ktail:4x33x5", 4, 33, 5, 0x77777777u},
    {"model:attn_proj_gemv", 1, 1280, 128, 0x0badc0deu},
    {"model:o_proj_gemv", 1, 1280, 1280, 0x12345678u},
    {"model:expert_down_gemv", 1, 6848, 256, 0x9abcdef0u},
    {"model:prefill_tile", 4, 1280, 64, 0x0f0f0f0fu},
    {"overflow:max_mag_k6848", 1, 6848, 4, 0u},
};

size_t oracle_selftest_n_shapes(void) { return sizeof(k_shapes) / sizeof(k_shapes[0]); }

int oracle_selftest_shape(size_t i, const char** label, size_t* m, size_t* k, size_t* n,
                          uint32_t* seed) {
    if (i >= oracle_selftest_n_shapes()) return ORACLE_E_SHAPE;
    if (label) *label = k_shapes[i].label;
    *m = k_shapes[i].m;
    *k = k_shapes[i].k;
    *n = k_shapes[i].n;
    if (seed) *seed = k_shapes[i].seed;
    return ORACLE_OK;
}

/* dispatch.rs:382-395: S8S8 operands; seed 0 = (i8::MAX, i8::MIN) extremes,
 * otherwise one xs32 stream (state seed|1) fills A then B, low byte each. */
int oracle_selftest_fill_s8(size_t i, int8_t* a, int8_t* b) {
    if (i >= oracle_selftest_n_shapes()) return ORACLE_E_SHAPE;
    const selftest_shape* s = &k_shapes[i];
    if (s->seed == 0) {
        for (size_t j = 0; j < s->m * s->k; ++j) a[j] = 127;
        for (size_t j = 0; j < s->n * s->k; ++j) b[j] = -128;
        return ORACLE_OK;
    }
    uint32_t st = s->seed | 1u;
    for (size_t j = 0; j < s->m * s->k; ++j) a[j] = (int8_t)(uint8_t)(oracle_xs32(&st) & 0xffu);
    for (size_t j = 0; j < s->n * s->k; ++j) b[j] = (int8_t)(uint8_t)(oracle_xs32(&st) & 0xffu);
    return ORACLE_OK;
}

/* dispatch.rs:403-413: U8S8 operands; seed 0 = (u8::MAX, i8::MIN); otherwise
 * the state is seed.rotate_left(7) | 1. */
int oracle_selftest_fill_u8(size_t i, uint8_t* a, int8_t* b) {
    if (i >= oracle_selftest_n_shapes()) return ORACLE_E_SHAPE;
    const selftest_shape* s = &k_shapes[i];
    if (s->seed == 0) {
        for (size_t j = 0; j < s->m * s->k; ++j) a[j] = 255;
        for (size_t j = 0; j < s->n * s->k; ++j) b[j] = -128;
        return ORACLE_OK;
    }
    uint32_t st = ((s->seed << 7) | (s->seed >> 25)) | 1u;
    for (size_t j = 0; j < s->m * s->k; ++j) a[j] = (uint8_t)(oracle_xs32(&st) & 0xffu);
    for (size_t j = 0; j < s->n * s->k; ++j) b[j] = (int8_t)(uint8_t)(oracle_xs32(&st) & 0xffu);
    return ORACLE_OK;
}

/* ---- src/native_engine/decoder.rs:1588-1597 quantize_row_i8 -------------
 * amax = fold(max, |x|) (f32::max ignores NaN); a_scale = amax/127 or 1.0;
 * inv = 1/a_scale; q = clamp(round_half_away(x*inv), -127, 127). */
float oracle_quantize_row_i8(const float* x, size_t k, int8_t* q) {
    float amax = 0.0f;
    for (size_t i = 0; i < k; ++i) amax = fmaxf(amax, fabsf(x[i]));
    float a_scale = amax > 0.0f ? amax / 127.0f : 1.0f;
    float inv = 1.0f / a_scale;
    for (size_t i = 0; i < k; ++i) q[i] = clamp_cast_i8(roundf(x[i] * inv), -127.0f, 127.0f);
    return a_scale;
}

/* decoder.rs:1647-1656 quantize_row_i8_te: same, rounding ties to even. */
float oracle_quantize_row_i8_te(const float* x, size_t k, int8_t* q) {
    float amax = 0.0f;
    for (size_t i = 0; i < k; ++i) amax = fmaxf(amax, fabsf(x[i]));
    float a_scale = amax > 0.0f ? amax / 127.0f : 1.0f;
    float inv = 1.0f / a_scale;
    for (size_t i = 0; i < k; ++i) q[i] = clamp_cast_i8(rintf(x[i] * inv), -127.0f, 127.0f);
    return a_scale;
}

/* decoder.rs:1636, :1737, :2734 dequant: y = ((f32)acc * a_scale) * w_scale,
 * two separately rounded multiplies, left to right. */
void oracle_dequant_i8(const int32_t* acc, size_t m, size_t n, const float* a_scales,
                       const float* w_scales, float* y) {
    for (size_t r = 0; r < m; ++r)
        for (size_t o = 0; o < n; ++o) {
            float t = (float)acc[r * n + o] * a_scales[r];
            y[r * n + o] = t * w_scales[o];
        }
}

/* decoder.rs:2703-2747 gemv_i8_batched (m=1 is gemv_i8, :1607-1640): each
 * row quantized on its own, one i32 contraction, dequant per row/channel.
 * xq/a_scales/acc are optional debug outputs (may be NULL). */
void oracle_gemv_i8_batched(const float* x, size_t m, const int8_t* w, const float* scales,
                            size_t n, size_t k, int8_t* xq, float* a_scales, int32_t* acc,
                            float* y) {
    int8_t* q = (int8_t*)malloc((m * k) > 0 ? m * k : 1);
    float* as = (float*)malloc((m ? m : 1) * sizeof(float));
    int32_t* ac = (int32_t*)calloc((m * n) > 0 ? m * n : 1, sizeof(int32_t));
    for (size_t r = 0; r < m; ++r) as[r] = oracle_quantize_row_i8(x + r * k, k, q + r * k);
    oracle_igemm_s8s8(q, w, m, k, n, ac);
    oracle_dequant_i8(ac, m, n, as, scales, y);
    if (xq) memcpy(xq, q, m * k);
    if (a_scales) memcpy(a_scales, as, m * sizeof(float));
    if (acc) memcpy(acc, ac, m * n * sizeof(int32_t));
    free(q);
    free(as);
    free(ac);
}

/* ---- src/native_engine/sampler.rs:168-186 argmax_row ----------------------
 * First index of the maximum; NaN skipped (`v <= best` keeps the earlier
 * index); an all-NaN row gives 0; an empty row is an error. */
int oracle_argmax_row(const float* logits, size_t n, uint32_t* idx) {
    if (n == 0) return ORACLE_E_SHAPE;
    int have = 0;
    size_t best = 0;
    float best_v = 0.0f;
    for (size_t i = 0; i < n; ++i) {
        float v = logits[i];
        if (v != v) continue;
        if (have && v <= best_v) continue;
        have = 1;
        best = i;
        best_v = v;
    }
    *idx = (uint32_t)(have ? best : 0);
    return ORACLE_OK;
}

/* decoder.rs:2943-2965 batched_lm_head_i8 (its input is the already-normed
 * row) + sampler argmax per row. */
int oracle_lm_head_i8(const float* x, size_t m, const int8_t* w, const float* scales, size_t n,
                      size_t k, float* logits, uint32_t* argmax) {
    oracle_gemv_i8_batched(x, m, w, scales, n, k, NULL, NULL, NULL, logits);
    for (size_t r = 0; r < m; ++r) {
        int st = oracle_argmax_row(logits + r * n, n, argmax + r);
        if (st) return st;
    }
    return ORACLE_OK;
}

/* ---- src/native_engine/sampler.rs no-repeat-ngram ban + greedy sample ------
 * sampler.rs:191-235 for_each_sliding_window_ngram_ban: nothing when ngram is
 * 0 or len < ngram; scan idx in [start, len - ngram + 1) with start =
 * len - window (saturating) or 0 for window 0; an n-gram whose first ngram-1
 * tokens equal the last ngram-1 tokens of seq bans its last token, unless
 * whitelisted or >= vocab. Writes the bans in scan order (repeats kept),
 * returns how many. */
size_t oracle_ngram_bans(const uint32_t* seq, size_t len, size_t ngram, size_t window, const uint32_t* white,
                         size_t n_white, size_t vocab, uint32_t* bans) {
    size_t nb = 0;
    if (ngram == 0 || len < ngram) return 0;
    size_t start = window == 0 ? 0 : (len > window ? len - window : 0);
    size_t end = len - ngram + 1;
    if (end <= start) return 0;
    const uint32_t* prefix = seq + (len - (ngram - 1));
    for (size_t idx = start; idx < end; ++idx) {
        int match = 1;
        for (size_t j = 0; j + 1 < ngram; ++j)
            if (seq[idx + j] != prefix[j]) {
                match = 0;
                break;
            }
        if (!match) continue;
        uint32_t banned = seq[idx + ngram - 1];
        int wl = 0;
        for (size_t j = 0; j < n_white; ++j) wl |= white[j] == banned;
        if (wl || banned >= vocab) continue;
        bans[nb++] = banned;
    }
    return nb;
}

/* sampler.rs:346-395 sample (greedy): the row with every banned id set to
 * -inf (the :245-257 masked copy; written to masked when non-NULL), then
 * argmax_row. */
int oracle_sample(const float* row, size_t n, const uint32_t* seq, size_t len, size_t ngram, size_t window,
                  const uint32_t* white, size_t n_white, float* masked, uint32_t* token) {
    if (n == 0) return ORACLE_E_SHAPE;
    float* m = (float*)malloc(n * sizeof(float));
    uint32_t* bans = (uint32_t*)malloc((len + 1) * sizeof(uint32_t));
    memcpy(m, row, n * sizeof(float));
    size_t nb = oracle_ngram_bans(seq, len, ngram, window, white, n_white, n, bans);
    for (size_t i = 0; i < nb; ++i) m[bans[i]] = -INFINITY;
    int st = oracle_argmax_row(m, n, token);
    if (masked) memcpy(masked, m, n * sizeof(float));
    free(m);
    free(bans);
    return st;
}

/* ---- src/native_engine/moe.rs:181-266 route --------------------------------
 * logits = x . G^T, softmax over experts, greedy top-k by descending prob
 * (strict >, lower index on ties, NaN skipped, error if no finite score),
 * optional renormalisation w /= (sum_f32(w) + 1e-20), then w *= scale.
 * Router numerics (documented definition of this build): each logit is an
 * f64 dot product rounded to f32; the softmax is computed in f64 from those
 * f32 logits (max-subtracted, exp, the sum taken in the order of the GPU's
 * full-wave DPP reduction, wave_tree_sum64 below, divide) and each probability rounded
 * to f32. Any f64 summation order of a 1280-term dot product or a 64-term sum
 * rounds to the same f32 except when the f64 value lies within ~2^-29
 * (relative) of an f32 rounding boundary, so the increasing-q dot order here
 * and the GPU's strided partial sums agree bit for bit in practice; the
 * softmax sum order is fixed exactly. `probs` (optional) receives the f32
 * probabilities [t][n_experts]. */
/* Sum of v[0..n), n <= 64, in the order of the GPU's full-wave DPP
 * reduction (lane i holds v[i], lanes i >= n hold +0): within each 16-lane
 * row the pairs (i, i+1), then the two pairs of each quad, then the two quads
 * of each 8-lane half, then the two halves (each step adds the same two
 * operands in both lanes that meet, and f64 addition is commutative, so every
 * lane of a row ends with the same value), then the four rows as
 * ((row0 + row1) + row2) + row3. */
static double wave_tree_sum64(const double* v, size_t n) {
    double a[64], row[4];
    for (size_t i = 0; i < 64; ++i) a[i] = i < n ? v[i] : 0.0;
    for (size_t r = 0; r < 4; ++r) {
        double q[4];
        for (size_t k = 0; k < 4; ++k) {
            const double* b = a + 16 * r + 4 * k;
            q[k] = (b[0] + b[1]) + (b[2] + b[3]);
        }
        row[r] = (q[0] + q[1]) + (q[2] + q[3]);
    }
    return ((row[0] + row[1]) + row[2]) + row[3];
}

int oracle_route(const float* hidden, size_t t, size_t h, const float* gate, size_t n_experts,
                 size_t top_k, int norm_topk, float routed_scale, uint32_t* idx, float* w,
                 float* probs) {
    if (n_experts < top_k || top_k == 0 || n_experts > 64) return ORACLE_E_SHAPE;
    float* logit = (float*)malloc(n_experts * sizeof(float));
    double* ex = (double*)malloc(n_experts * sizeof(double));
    float* p = (float*)malloc(n_experts * sizeof(float));
    unsigned char* taken = (unsigned char*)malloc(n_experts);
    int status = ORACLE_OK;
    for (size_t tok = 0; tok < t && status == ORACLE_OK; ++tok) {
        const float* x = hidden + tok * h;
        for (size_t e = 0; e < n_experts; ++e) {
            double acc = 0.0;
            for (size_t q = 0; q < h; ++q) acc += (double)x[q] * (double)gate[e * h + q];
            logit[e] = (float)acc;
        }
        double mx = -INFINITY;
        for (size_t e = 0; e < n_experts; ++e)
            if ((double)logit[e] > mx) mx = (double)logit[e];
        for (size_t e = 0; e < n_experts; ++e) ex[e] = exp((double)logit[e] - mx);
        const double sum = wave_tree_sum64(ex, n_experts);
        for (size_t e = 0; e < n_experts; ++e) p[e] = (float)(ex[e] / sum);
        if (probs) memcpy(probs + tok * n_experts, p, n_experts * sizeof(float));

        memset(taken, 0, n_experts);
        for (size_t slot = 0; slot < top_k; ++slot) {
            int have = 0;
            size_t best = 0;
            float best_v = 0.0f;
            for (size_t e = 0; e < n_experts; ++e) {
                float v = p[e];
                if (taken[e] || v != v) continue;
                if (have && v <= best_v) continue;
                have = 1;
                best = e;
                best_v = v;
            }
            if (!have) {
                status = ORACLE_E_ROUTE;
                break;
            }
            taken[best] = 1;
            idx[tok * top_k + slot] = (uint32_t)best;
            w[tok * top_k + slot] = best_v;
        }
        if (status) break;
        float* wt = w + tok * top_k;
        if (norm_topk) {
            float s = 0.0f;
            for (size_t j = 0; j < top_k; ++j) s += wt[j];
            float denom = s + 1e-20f;
            for (size_t j = 0; j < top_k; ++j) wt[j] /= denom;
        }
        for (size_t j = 0; j < top_k; ++j) wt[j] *= routed_scale;
    }
    free(logit);
    free(ex);
    free(p);
    free(taken);
    return status;
}

/* decoder.rs:1079-1083 silu(x) = x / (1 + e^-x) */
float oracle_silu(float x) { return x / (1.0f + expf(-x)); }

/* decoder.rs:1744-1755 expert_gemv_i8_serial (+ gemv_i8_serial :1729-1740):
 * quantize x once, gate/up GEMV with dequant, act = silu(g)*u, re-quantize
 * act, down GEMV with dequant. act/aq/a_scale2 are optional debug outputs. */
void oracle_expert_i8(const float* x, size_t h, size_t inter, const int8_t* wg, const float* sg,
                      const int8_t* wu, const float* su, const int8_t* wd, const float* sd,
                      float* y, float* act, int8_t* aq, float* a_scale2) {
    int8_t* xq = (int8_t*)malloc(h);
    int32_t* acc = (int32_t*)malloc((inter > h ? inter : h) * sizeof(int32_t));
    float* g = (float*)malloc(inter * sizeof(float));
    float* u = (float*)malloc(inter * sizeof(float));
    float* a = (float*)malloc(inter * sizeof(float));
    int8_t* q2 = (int8_t*)malloc(inter);
    float as = oracle_quantize_row_i8(x, h, xq);
    memset(acc, 0, inter * sizeof(int32_t));
    oracle_igemm_s8s8(xq, wg, 1, h, inter, acc);
    oracle_dequant_i8(acc, 1, inter, &as, sg, g);
    memset(acc, 0, inter * sizeof(int32_t));
    oracle_igemm_s8s8(xq, wu, 1, h, inter, acc);
    oracle_dequant_i8(acc, 1, inter, &as, su, u);
    for (size_t i = 0; i < inter; ++i) a[i] = oracle_silu(g[i]) * u[i];
    float as2 = oracle_quantize_row_i8(a, inter, q2);
    memset(acc, 0, h * sizeof(int32_t));
    oracle_igemm_s8s8(q2, wd, 1, inter, h, acc);
    oracle_dequant_i8(acc, 1, h, &as2, sd, y);
    if (act) memcpy(act, a, inter * sizeof(float));
    if (aq) memcpy(aq, q2, inter);
    if (a_scale2) *a_scale2 = as2;
    free(xq);
    free(acc);
    free(g);
    free(u);
    free(a);
    free(q2);
}

/* decoder.rs:2199-2268 decode_mlp_i8 (MoE arm), applied per token as the
 * batched spine does (decoder.rs:2924-2930): route, then for each slot j in
 * order y_j = expert(x) * w_j (elementwise f32 multiply), out = ((0 + y_0) +
 * y_1) ... + y_5, then + shared expert output when one is given. Expert e's
 * weights: wg/wu [e][inter][h], wd [e][h][inter], scales sg/su [e][inter],
 * sd [e][h]. */
int oracle_moe_decode(const float* hidden, size_t t, size_t h, size_t inter, size_t n_experts,
                      size_t top_k, const float* router, const int8_t* wg, const float* sg,
                      const int8_t* wu, const float* su, const int8_t* wd, const float* sd,
                      int norm_topk, float routed_scale, const int8_t* shared_wg,
                      const float* shared_sg, const int8_t* shared_wu, const float* shared_su,
                      const int8_t* shared_wd, const float* shared_sd, size_t shared_inter,
                      float* out, uint32_t* idx, float* gates) {
    int st = oracle_route(hidden, t, h, router, n_experts, top_k, norm_topk, routed_scale, idx,
                          gates, NULL);
    if (st) return st;
    float* y = (float*)malloc(h * sizeof(float));
    for (size_t tok = 0; tok < t; ++tok) {
        const float* x = hidden + tok * h;
        float* o = out + tok * h;
        for (size_t c = 0; c < h; ++c) o[c] = 0.0f;
        for (size_t j = 0; j < top_k; ++j) {
            size_t e = idx[tok * top_k + j];
            float wj = gates[tok * top_k + j];
            oracle_expert_i8(x, h, inter, wg + e * inter * h, sg + e * inter, wu + e * inter * h,
                             su + e * inter, wd + e * h * inter, sd + e * h, y, NULL, NULL,
                             NULL);
            for (size_t c = 0; c < h; ++c) y[c] *= wj;
            for (size_t c = 0; c < h; ++c) o[c] += y[c];
        }
        if (shared_wg) {
            oracle_expert_i8(x, h, shared_inter, shared_wg, shared_sg, shared_wu, shared_su,
                             shared_wd, shared_sd, y, NULL, NULL, NULL);
            for (size_t c = 0; c < h; ++c) o[c] += y[c];
        }
    }
    free(y);
    return ORACLE_OK;
}

/* ---- src/simd/int4.rs:97-142 nibble semantics ----------------------------- */
int8_t oracle_sign_extend_nibble(uint8_t nib) { return (int8_t)((int8_t)(uint8_t)(nib << 4) >> 4); }

void oracle_unpack_byte(uint8_t b, int8_t* lo, int8_t* hi) {
    *lo = oracle_sign_extend_nibble(b & 0x0f);
    *hi = oracle_sign_extend_nibble(b >> 4);
}

int oracle_unpack_to_i8(const uint8_t* packed, size_t n, size_t k, int8_t* out) {
    size_t t;
    if (k % 2 || !mul_ok(n, k / 2, &t) || !mul_ok(n, k, &t)) return ORACLE_E_SHAPE;
    for (size_t j = 0; j < n * (k / 2); ++j) oracle_unpack_byte(packed[j], &out[2 * j], &out[2 * j + 1]);
    return ORACLE_OK;
}

static int s4_shapes_ok(size_t group, size_t m, size_t k, size_t n) {
    size_t t;
    if (k % 2) return 0;
    if (group != 16 && group != 32) return 0;
    if (k % group) return 0;
    if (!mul_ok(m, k, &t) || !mul_ok(n, k / 2, &t) || !mul_ok(n, k / group, &t) || !mul_ok(m, n, &t))
        return 0;
    return 1;
}

/* int4.rs:304-343 s4s8_packed_kernel_scalar: per (m, n), per group in
 * increasing order: acc_i = i32 dot over the group (even k = low nibble),
 * acc_f = acc_f + scale * (f32)acc_i (separate multiply and add); out is
 * overwritten. */
int oracle_igemm_s4s8_packed(const int8_t* a, const uint8_t* b_packed, const float* scales,
                             size_t group, size_t m, size_t k, size_t n, float* out) {
    if (!s4_shapes_ok(group, m, k, n)) return ORACLE_E_SHAPE;
    size_t groups = k / group, kb = k / 2;
    for (size_t mi = 0; mi < m; ++mi)
        for (size_t ni = 0; ni < n; ++ni) {
            float acc_f = 0.0f;
            for (size_t g = 0; g < groups; ++g) {
                int32_t acc_i = 0;
                for (size_t kk = g * group; kk < (g + 1) * group; ++kk) {
                    uint8_t byte = b_packed[ni * kb + kk / 2];
                    int8_t wv = (kk & 1) ? oracle_sign_extend_nibble(byte >> 4)
                                         : oracle_sign_extend_nibble(byte & 0x0f);
                    acc_i += (int32_t)a[mi * k + kk] * (int32_t)wv;
                }
                float prod = scales[ni * groups + g] * (float)acc_i;
                acc_f = acc_f + prod;
            }
            out[mi * n + ni] = acc_f;
        }
    return ORACLE_OK;
}

/* The per-group i32 partials of the contraction above, [m][n][k/group]. */
int oracle_s4s8_group_i32(const int8_t* a, const uint8_t* b_packed, size_t group, size_t m,
                          size_t k, size_t n, int32_t* partials) {
    if (!s4_shapes_ok(group, m, k, n)) return ORACLE_E_SHAPE;
    size_t groups = k / group, kb = k / 2;
    for (size_t mi = 0; mi < m; ++mi)
        for (size_t ni = 0; ni < n; ++ni)
            for (size_t g = 0; g < groups; ++g) {
                int32_t acc_i = 0;
                for (size_t kk = g * group; kk < (g + 1) * group; ++kk) {
                    int8_t lo, hi;
                    oracle_unpack_byte(b_packed[ni * kb + kk / 2], &lo, &hi);
                    acc_i += (int32_t)a[mi * k + kk] * (int32_t)((kk & 1) ? hi : lo);
                }
                partials[(mi * n + ni) * groups + g] = acc_i;
            }
    return ORACLE_OK;
}

/* int4 prefill MoE: this build's composition (the reference has no int4
 * model wiring: no decoder layer loads int4 experts). Activations are quantized per row with the
 * prefill ties-even rule (decoder.rs:1647-1656); each projection is the int4
 * kernel contract (int4.rs:304-343) times the row's activation scale; the
 * grouped structure and ascending-expert scatter `out[t] += w * y` follow
 * moe_block_i8 (decoder.rs:2142-2181): members of expert e in (token, slot)
 * order, one output row each. Expert e: wg/wu packed [e][inter][h/2],
 * sg/su [e][inter][h/group], wd [e][h][inter/2], sd [e][h][inter/group]. */
int oracle_moe_prefill_i4(const float* x, size_t t, size_t h, size_t inter, size_t n_experts,
                          size_t top_k, const uint32_t* idx, const float* gates, size_t group,
                          const uint8_t* wg, const float* sg, const uint8_t* wu, const float* su,
                          const uint8_t* wd, const float* sd, float* out, int8_t* xq,
                          float* x_scales) {
    if (!s4_shapes_ok(group, 1, h, inter) || !s4_shapes_ok(group, 1, inter, h)) return ORACLE_E_SHAPE;
    for (size_t r = 0; r < t * top_k; ++r)
        if (idx[r] >= n_experts) return ORACLE_E_SHAPE;
    for (size_t r = 0; r < t; ++r) x_scales[r] = oracle_quantize_row_i8_te(x + r * h, h, xq + r * h);
    memset(out, 0, t * h * sizeof(float));
    float* g = (float*)malloc(inter * sizeof(float));
    float* u = (float*)malloc(inter * sizeof(float));
    float* act = (float*)malloc(inter * sizeof(float));
    int8_t* aq = (int8_t*)malloc(inter);
    float* y = (float*)malloc(h * sizeof(float));
    size_t gh = h / group, gi = inter / group;
    for (size_t e = 0; e < n_experts; ++e) {
        for (size_t tok = 0; tok < t; ++tok) {
            size_t j;
            for (j = 0; j < top_k; ++j)
                if (idx[tok * top_k + j] == e) break;
            if (j == top_k) continue;
            const int8_t* xr = xq + tok * h;
            oracle_igemm_s4s8_packed(xr, wg + e * inter * (h / 2), sg + e * inter * gh, group, 1,
                                     h, inter, g);
            oracle_igemm_s4s8_packed(xr, wu + e * inter * (h / 2), su + e * inter * gh, group, 1,
                                     h, inter, u);
            for (size_t i = 0; i < inter; ++i) {
                float gv = g[i] * x_scales[tok];
                float uv = u[i] * x_scales[tok];
                act[i] = oracle_silu(gv) * uv;
            }
            float as2 = oracle_quantize_row_i8_te(act, inter, aq);
            oracle_igemm_s4s8_packed(aq, wd + e * h * (inter / 2), sd + e * h * gi, group, 1,
                                     inter, h, y);
            /* every slot of this token routed to e is a member (decoder.rs:2156-2160
             * pushes (t, w) per slot), added in slot order */
            float* o = out + tok * h;
            for (; j < top_k; ++j) {
                if (idx[tok * top_k + j] != e) continue;
                const float wj = gates[tok * top_k + j];
                for (size_t c = 0; c < h; ++c) {
                    float yv = y[c] * as2;
                    float p = wj * yv;
                    o[c] = o[c] + p;
                }
            }
        }
    }
    free(g);
    free(u);
    free(act);
    free(aq);
    free(y);
    return ORACLE_OK;
}

/* ---- decode-layer ops: nn::rms_norm and RoPE ------------------------------- */
void oracle_rms_norm(const float* x, size_t n, const float* w, float eps, float* y) {
    double ss = 0.0;
    for (size_t i = 0; i < n; ++i) ss += (double)x[i] * (double)x[i];
    const float rstd = (float)(1.0 / sqrt(ss / (double)n + (double)eps));
    for (size_t i = 0; i < n; ++i) {
        float v = x[i] * rstd;
        y[i] = w ? v * w[i] : v;
    }
}

/* decoder.rs:170-227 RopeTable::build (one position), :229-268 apply_rope. */
int oracle_rope(float* x, size_t n_heads, size_t head_dim, size_t pos, float theta) {
    if (head_dim == 0 || head_dim % 2) return ORACLE_E_SHAPE;
    const size_t half = head_dim / 2;
    for (size_t i = 0; i < half; ++i) {
        const double exponent = (double)(2 * i) / (double)head_dim;
        const float inv_freq = (float)(1.0 / pow((double)theta, exponent));
        const float angle = (float)pos * inv_freq;
        const float s = sinf(angle), c = cosf(angle);
        for (size_t h = 0; h < n_heads; ++h) {
            float* r = x + h * head_dim;
            const float a = r[i], b = r[half + i];
            r[i] = a * c - b * s;
            r[half + i] = b * c + a * s;
        }
    }
    return ORACLE_OK;
}

/* ---- nn::linear_int8_dynamic (nn.rs:151-173) --------------------------------
 * ft-kernel-cpu's linear_int8_dynamic_f32 is not in the reference tree; its
 * activation rule is the documented one (docs/focrq-format.md:296-320, pinned
 * by nn.rs:601-628 ties-even); the dequant is the decoder's order
 * ((f32)acc * scale_a) * w_scale (decoder.rs:1636), then + bias. */
float oracle_quantize_row_dynamic(const float* x, size_t k, int8_t* q) {
    float amax = 0.0f;
    for (size_t i = 0; i < k; ++i) amax = fmaxf(amax, fabsf(x[i]));
    float a_scale = amax > 0.0f ? amax / 127.0f : 1.0f;
    for (size_t i = 0; i < k; ++i) {
        float v = x[i] / a_scale;
        if (v != v) {
            q[i] = 0;
            continue;
        }
        v = fminf(fmaxf(v, -127.0f), 127.0f);
        q[i] = (int8_t)(int)rintf(v);
    }
    return a_scale;
}

int oracle_linear_i8_dynamic(const float* x, size_t m, size_t k, const int8_t* w, const float* w_scales,
                             size_t n, const float* bias, float* y, int8_t* xq, float* x_scales) {
    size_t t;
    if (!mul_ok(m, k, &t) || !mul_ok(n, k, &t) || !mul_ok(m, n, &t)) return ORACLE_E_SHAPE;
    int32_t* acc = (int32_t*)calloc((m * n) > 0 ? (m * n) : 1, sizeof(int32_t));
    if (!acc) return ORACLE_E_SHAPE;
    for (size_t r = 0; r < m; ++r) x_scales[r] = oracle_quantize_row_dynamic(x + r * k, k, xq + r * k);
    oracle_igemm_s8s8(xq, w, m, k, n, acc);
    for (size_t r = 0; r < m; ++r)
        for (size_t o = 0; o < n; ++o) {
            float v = (float)acc[r * n + o] * x_scales[r];
            v = v * w_scales[o];
            if (bias) v = v + bias[o];
            y[r * n + o] = v;
        }
    free(acc);
    return ORACLE_OK;
}

/* expert_mlp_i8 (decoder.rs:2120-2135) over rows x[0..rows) of width h:
 * y [rows][h]. */
static int expert_mlp_i8_rows(const float* x, size_t rows, size_t h, size_t inter, const int8_t* wg,
                              const float* sg, const int8_t* wu, const float* su, const int8_t* wd,
                              const float* sd, float* y) {
    float* g = (float*)malloc(rows * inter * sizeof(float));
    float* u = (float*)malloc(rows * inter * sizeof(float));
    int8_t* xq = (int8_t*)malloc(rows * (h > inter ? h : inter));
    float* xs = (float*)malloc(rows * sizeof(float));
    int st = ORACLE_E_SHAPE;
    if (g && u && xq && xs) {
        st = oracle_linear_i8_dynamic(x, rows, h, wg, sg, inter, NULL, g, xq, xs);
        if (st == ORACLE_OK) st = oracle_linear_i8_dynamic(x, rows, h, wu, su, inter, NULL, u, xq, xs);
        if (st == ORACLE_OK) {
            for (size_t i = 0; i < rows * inter; ++i) g[i] = oracle_silu(g[i]) * u[i];
            st = oracle_linear_i8_dynamic(g, rows, inter, wd, sd, h, NULL, y, xq, xs);
        }
    }
    free(g);
    free(u);
    free(xq);
    free(xs);
    return st;
}

int oracle_moe_prefill_i8(const float* x, size_t t, size_t h, size_t inter, size_t n_experts,
                          size_t top_k, const uint32_t* idx, const float* gates, const int8_t* wg,
                          const float* sg, const int8_t* wu, const float* su, const int8_t* wd,
                          const float* sd, const int8_t* shared_wg, const float* shared_sg,
                          const int8_t* shared_wu, const float* shared_su, const int8_t* shared_wd,
                          const float* shared_sd, size_t shared_inter, float* out) {
    for (size_t r = 0; r < t * top_k; ++r)
        if (idx[r] >= n_experts) return ORACLE_E_SHAPE;
    memset(out, 0, t * h * sizeof(float));
    /* members of expert e in (token, slot) order (decoder.rs:2152-2157) */
    size_t* mem_t = (size_t*)malloc((t * top_k + 1) * sizeof(size_t));
    float* mem_w = (float*)malloc((t * top_k + 1) * sizeof(float));
    float* sub = (float*)malloc((t * top_k + 1) * h * sizeof(float));
    float* y = (float*)malloc((t * top_k + 1) * h * sizeof(float));
    int st = (mem_t && mem_w && sub && y) ? ORACLE_OK : ORACLE_E_SHAPE;
    for (size_t e = 0; e < n_experts && st == ORACLE_OK; ++e) {
        size_t m = 0;
        for (size_t tok = 0; tok < t; ++tok)
            for (size_t j = 0; j < top_k; ++j)
                if (idx[tok * top_k + j] == e) {
                    mem_t[m] = tok;
                    mem_w[m] = gates[tok * top_k + j];
                    memcpy(sub + m * h, x + tok * h, h * sizeof(float));
                    ++m;
                }
        if (m == 0) continue;
        st = expert_mlp_i8_rows(sub, m, h, inter, wg + e * inter * h, sg + e * inter, wu + e * inter * h,
                                su + e * inter, wd + e * h * inter, sd + e * h, y);
        for (size_t r = 0; r < m && st == ORACLE_OK; ++r) {
            float* o = out + mem_t[r] * h;
            for (size_t c = 0; c < h; ++c) {
                float p = mem_w[r] * y[r * h + c];
                o[c] = o[c] + p;
            }
        }
    }
    if (st == ORACLE_OK && shared_wg) {
        float* sy = (float*)malloc(t * h * sizeof(float));
        st = sy ? expert_mlp_i8_rows(x, t, h, shared_inter, shared_wg, shared_sg, shared_wu, shared_su,
                                     shared_wd, shared_sd, sy)
                : ORACLE_E_SHAPE;
        for (size_t i = 0; i < t * h && st == ORACLE_OK; ++i) out[i] = out[i] + sy[i];
        free(sy);
    }
    free(mem_t);
    free(mem_w);
    free(sub);
    free(y);
    return st;
}

/* ---- src/quant/int8.rs:110-163 quantize_int8_f32 --------------------------
 * scale = max|row|/127 (all-zero row: scale 1, q 0); q =
 * clamp(round_ties_even(w / scale), -127, 127) with true division. */
int oracle_quantize_int8_f32(const float* w, size_t n, size_t k, int8_t* q, float* scales) {
    size_t t;
    if (!mul_ok(n, k, &t)) return ORACLE_E_SHAPE;
    for (size_t o = 0; o < n; ++o) {
        const float* row = w + o * k;
        float mx = 0.0f;
        for (size_t i = 0; i < k; ++i) mx = fmaxf(mx, fabsf(row[i]));
        if (mx == 0.0f) {
            scales[o] = 1.0f;
            memset(q + o * k, 0, k);
            continue;
        }
        float s = mx / 127.0f;
        scales[o] = s;
        for (size_t i = 0; i < k; ++i) q[o * k + i] = clamp_cast_i8(rintf(row[i] / s), -127.0f, 127.0f);
    }
    return ORACLE_OK;
}

/* src/quant/int4.rs:142-205 pack_int4_f32: per-group scale = max|g|/7 (all-
 * zero group: 1.0), q = clamp(round_ties_even(w/scale), -8, 7), packed low
 * nibble = even column, high nibble = odd column. */
int oracle_pack_int4_f32(const float* w, size_t n, size_t k, size_t group, uint8_t* packed,
                         float* scales) {
    if (!s4_shapes_ok(group, 1, k, n)) return ORACLE_E_SHAPE;
    size_t groups = k / group;
    int8_t* rq = (int8_t*)malloc(k);
    for (size_t o = 0; o < n; ++o) {
        const float* row = w + o * k;
        for (size_t g = 0; g < groups; ++g) {
            float mx = 0.0f;
            for (size_t i = 0; i < group; ++i) mx = fmaxf(mx, fabsf(row[g * group + i]));
            float s = mx == 0.0f ? 1.0f : mx / 7.0f;
            scales[o * groups + g] = s;
            for (size_t i = 0; i < group; ++i)
                rq[g * group + i] = clamp_cast_i8(rintf(row[g * group + i] / s), -8.0f, 7.0f);
        }
        for (size_t j = 0; j < k / 2; ++j)
            packed[o * (k / 2) + j] = (uint8_t)(((uint8_t)rq[2 * j] & 0x0f) | (((uint8_t)rq[2 * j + 1] & 0x0f) << 4));
    }
    free(rq);
    return ORACLE_OK;
}

/* ---- src/native_engine/rswa.rs:451-513 write_decode_step -------------------
 * Ring regions are head-major [NUM_HEADS][RING_WINDOW][HEAD_DIM]. Warm-up
 * (ring_len < W): append at ring_len, ring_len += 1, ring_pos = ring_len % W.
 * Steady state: overwrite ring_pos, ring_pos = (ring_pos + 1) % W. */
int oracle_ring_write(float* ring_k, float* ring_v, uint32_t* ring_len, uint32_t* ring_pos,
                      const float* k_step, const float* v_step, uint32_t* slot) {
    const size_t H = ORACLE_NUM_HEADS, D = ORACLE_HEAD_DIM, W = ORACLE_RING_WINDOW;
    uint32_t s;
    if (*ring_len > W || *ring_pos >= W) return ORACLE_E_SHAPE;
    if (*ring_len < W) {
        s = *ring_len;
        *ring_len += 1;
        *ring_pos = *ring_len % W;
    } else {
        s = *ring_pos;
        *ring_pos = (*ring_pos + 1) % W;
    }
    for (size_t hh = 0; hh < H; ++hh) {
        memcpy(ring_k + (hh * W + s) * D, k_step + hh * D, D * sizeof(float));
        memcpy(ring_v + (hh * W + s) * D, v_step + hh * D, D * sizeof(float));
    }
    *slot = s;
    return ORACLE_OK;
}

/* rswa.rs:52-55 scale() = 1 / sqrt(128) in f32 */
static float attn_scale(void) { return 1.0f / sqrtf((float)ORACLE_HEAD_DIM); }

/* rswa.rs:1163-1182 fold: one online-softmax step. */
static void fold(float* run_max, float* run_den, float* acc, float score, const float* v) {
    const size_t D = ORACLE_HEAD_DIM;
    if (score > *run_max) {
        float correction = isfinite(*run_max) ? expf(*run_max - score) : 0.0f;
        *run_den *= correction;
        for (size_t i = 0; i < D; ++i) acc[i] *= correction;
        *run_max = score;
    }
    float wv = expf(score - *run_max);
    *run_den += wv;
    for (size_t i = 0; i < D; ++i) acc[i] += wv * v[i];
}

/* rswa.rs:894-939 decode_attention_scalar: per head, fold over
 * ref[0..prefill_len] then ring[0..ring_len] in physical slot order; score =
 * dot(q, k) * scale (dot rswa.rs:612-618, increasing d); out = acc * (1/den).
 * No causal mask. ref regions are [NUM_HEADS][ref_cap][HEAD_DIM]. */
int oracle_decode_attention(const float* ref_k, const float* ref_v, size_t ref_cap,
                            size_t prefill_len, const float* ring_k, const float* ring_v,
                            size_t ring_len, const float* q, float* out) {
    const size_t H = ORACLE_NUM_HEADS, D = ORACLE_HEAD_DIM, W = ORACLE_RING_WINDOW;
    if (prefill_len > ref_cap || ring_len > W) return ORACLE_E_SHAPE;
    if (prefill_len + ring_len == 0) return ORACLE_E_SHAPE;
    const float s = attn_scale();
    float acc[ORACLE_HEAD_DIM];
    for (size_t hh = 0; hh < H; ++hh) {
        const float* qh = q + hh * D;
        float run_max = -INFINITY, run_den = 0.0f;
        for (size_t i = 0; i < D; ++i) acc[i] = 0.0f;
        for (size_t r = 0; r < prefill_len; ++r) {
            const float* kr = ref_k + (hh * ref_cap + r) * D;
            float d = 0.0f;
            for (size_t i = 0; i < D; ++i) d += qh[i] * kr[i];
            fold(&run_max, &run_den, acc, d * s, ref_v + (hh * ref_cap + r) * D);
        }
        for (size_t r = 0; r < ring_len; ++r) {
            const float* kr = ring_k + (hh * W + r) * D;
            float d = 0.0f;
            for (size_t i = 0; i < D; ++i) d += qh[i] * kr[i];
            fold(&run_max, &run_den, acc, d * s, ring_v + (hh * W + r) * D);
        }
        float inv = run_den > 0.0f ? 1.0f / run_den : 0.0f;
        for (size_t i = 0; i < D; ++i) out[hh * D + i] = acc[i] * inv;
    }
    return ORACLE_OK;
}

/* ---- decoder.rs:1282-1340 chunk_prefill_attention (and :568-640 prefill_attention)
 * The reference front-pads the chunk's queries to the prefix length and runs
 * nn::sdpa (ft_kernel_cpu::sdpa_forward_f32, un-vendored) with the top-left
 * causal mask, so the kept row t (= c0 + i) attends keys [0, t]; the padded
 * rows are discarded. The kept row is restated directly: per head, the score
 * q.k over head_dim times scale = 1/sqrt(head_dim) (rswa.rs:52-55 form), a
 * max-subtracted softmax over [0, t], P.V over the keys.
 *
 * ft-kernel-cpu's f32 summation order is unknowable here, and any f32 order
 * lands about 1e-4 (relative to 1% of a row's largest output) from the exact
 * result at 1024 keys — the 128-term f32 score dots dominate. So the oracle
 * evaluates this math in float64 from the f32 inputs and rounds once to f32:
 * the attention every f32 implementation, the reference's included,
 * approximates (parity with the reference's exact bits unpinned). The f32
 * restatement in the order the reference's comments give
 * (decoder.rs:1274-1279: ascending dims, ascending keys) is kept beside it
 * as oracle_chunk_prefill_attention_f32, to measure that spread. Either way a
 * row is a pure function of (q_t, k[0..t], v[0..t]), so a chunked schedule
 * equals the monolithic one bit for bit. */
static int attention_shape_ok(size_t cs, size_t c1, size_t num_heads, size_t head_dim, size_t c0) {
    return num_heads != 0 && head_dim != 0 && c0 <= c1 && c0 + cs == c1;
}

int oracle_chunk_prefill_attention(const float* q_chunk, size_t cs, const float* k_prefix,
                                   const float* v_prefix, size_t c1, size_t num_heads,
                                   size_t head_dim, size_t c0, float* out) {
    if (!attention_shape_ok(cs, c1, num_heads, head_dim, c0)) return ORACLE_E_SHAPE;
    const size_t dim = num_heads * head_dim;
    const double scale = 1.0 / sqrt((double)head_dim);
    double* s = (double*)malloc((c1 ? c1 : 1) * sizeof(double));
    double* o = (double*)malloc(head_dim * sizeof(double));
    if (!s || !o) {
        free(s);
        free(o);
        return ORACLE_E_SHAPE;
    }
    for (size_t i = 0; i < cs; ++i) {
        const size_t t = c0 + i;
        for (size_t h = 0; h < num_heads; ++h) {
            const float* q = q_chunk + i * dim + h * head_dim;
            double mx = -INFINITY;
            for (size_t j = 0; j <= t; ++j) {
                const float* k = k_prefix + j * dim + h * head_dim;
                double acc = 0.0;
                for (size_t d = 0; d < head_dim; ++d) acc += (double)q[d] * (double)k[d];
                s[j] = acc * scale;
                if (s[j] > mx) mx = s[j];
            }
            double sum = 0.0;
            for (size_t j = 0; j <= t; ++j) {
                s[j] = exp(s[j] - mx);
                sum += s[j];
            }
            for (size_t d = 0; d < head_dim; ++d) o[d] = 0.0;
            for (size_t j = 0; j <= t; ++j) {
                const double p = s[j] / sum;
                const float* v = v_prefix + j * dim + h * head_dim;
                for (size_t d = 0; d < head_dim; ++d) o[d] += p * (double)v[d];
            }
            float* orow = out + i * dim + h * head_dim;
            for (size_t d = 0; d < head_dim; ++d) orow[d] = (float)o[d];
        }
    }
    free(s);
    free(o);
    return ORACLE_OK;
}

int oracle_chunk_prefill_attention_f32(const float* q_chunk, size_t cs, const float* k_prefix,
                                       const float* v_prefix, size_t c1, size_t num_heads,
                                       size_t head_dim, size_t c0, float* out) {
    if (!attention_shape_ok(cs, c1, num_heads, head_dim, c0)) return ORACLE_E_SHAPE;
    const size_t dim = num_heads * head_dim;
    const float scale = 1.0f / sqrtf((float)head_dim);
    float* s = (float*)malloc((c1 ? c1 : 1) * sizeof(float));
    if (!s) return ORACLE_E_SHAPE;
    for (size_t i = 0; i < cs; ++i) {
        const size_t t = c0 + i;
        for (size_t h = 0; h < num_heads; ++h) {
            const float* q = q_chunk + i * dim + h * head_dim;
            float mx = -INFINITY;
            for (size_t j = 0; j <= t; ++j) {
                const float* k = k_prefix + j * dim + h * head_dim;
                float acc = 0.0f;
                for (size_t d = 0; d < head_dim; ++d) acc += q[d] * k[d];
                s[j] = acc * scale;
                if (s[j] > mx) mx = s[j];
            }
            float sum = 0.0f;
            for (size_t j = 0; j <= t; ++j) {
                s[j] = expf(s[j] - mx);
                sum += s[j];
            }
            float* o = out + i * dim + h * head_dim;
            for (size_t d = 0; d < head_dim; ++d) o[d] = 0.0f;
            for (size_t j = 0; j <= t; ++j) {
                const float p = s[j] / sum;
                const float* v = v_prefix + j * dim + h * head_dim;
                for (size_t d = 0; d < head_dim; ++d) o[d] += p * v[d];
            }
        }
    }
    free(s);
    return ORACLE_OK;
}

int oracle_prefill_attention(const float* q, const float* k, const float* v, size_t seq,
                             size_t num_heads, size_t head_dim, float* out) {
    return oracle_chunk_prefill_attention(q, seq, k, v, seq, num_heads, head_dim, 0, out);
}
