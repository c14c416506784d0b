/*
 * cpu_int4.c — the reference's two x86 int4 GEMM paths and an int4 MoE
 * block over them, restated in C for the CPU baseline (TEST/BENCH
 * INFRASTRUCTURE ONLY: never linked into the product library).
 *
 * The reference has no x86 int4 multiply-accumulate kernel (int4.rs:454-460),
 * so on x86 its int4 GEMMs run one of:
 *   - s4s8_packed_kernel_scalar (int4.rs:304-343): each nibble read out of the
 *     packed byte inside the group loop;
 *   - igemm_s4s8 (int4.rs:245-278): the whole B unpacked to i8 once per call
 *     (accel::unpack_nibbles, AVX2 when the host has it, int4.rs:560-650),
 *     then igemm_s4s8_unpacked's per-group loop (int4.rs:280-302).
 * Both are plain loops that rustc's release profile (opt-level 3, x86-64
 * baseline target: Cargo.toml [profile.release], no target-cpu) hands to the
 * LLVM vectorizer; this file is therefore built with clang -O3 for the same
 * baseline ISA (oracle/Makefile). The AVX2 unpack carries its own target
 * attribute, as the reference's #[target_feature(enable = "avx2")] does.
 *
 * Results are bit-identical to the oracle's (the per-group i32 dot is exact;
 * the f32 dequant-and-sum runs in increasing group order).
 */
#include <immintrin.h>
#include <stdlib.h>
#include <string.h>

#include "cpu_tier.h"
#include "focr_oracle.h"

/* int4.rs:304-343 */
static void s4s8_packed(const int8_t* a, const uint8_t* bp, const float* scales, size_t group, size_t m, size_t k,
                        size_t n, float* out) {
    const size_t groups = k / group, kb = k / 2;
    for (size_t mi = 0; mi < m; ++mi) {
        const int8_t* ar = a + mi * k;
        for (size_t ni = 0; ni < n; ++ni) {
            const uint8_t* br = bp + ni * kb;
            const float* sr = scales + ni * groups;
            float acc_f = 0.0f;
            for (size_t g = 0; g < groups; ++g) {
                int32_t acc_i = 0;
                for (size_t kk = g * group; kk < (g + 1) * group; ++kk) {
                    uint8_t byte = br[kk / 2];
                    uint8_t nib = (kk & 1) ? (uint8_t)(byte >> 4) : (uint8_t)(byte & 0x0f);
                    int32_t w = (int32_t)(int8_t)(uint8_t)(nib << 4) >> 4;
                    acc_i += (int32_t)ar[kk] * w;
                }
                acc_f += sr[g] * (float)acc_i;
            }
            out[mi * n + ni] = acc_f;
        }
    }
}

/* int4.rs:507-515: out[2j] = lo(src[j]), out[2j+1] = hi(src[j]), sign-extended */
static void unpack_scalar(const uint8_t* src, size_t len, int8_t* out) {
    for (size_t j = 0; j < len; ++j) {
        out[2 * j] = (int8_t)((int8_t)(uint8_t)(src[j] << 4) >> 4);
        out[2 * j + 1] = (int8_t)((int8_t)src[j] >> 4);
    }
}

/* The AVX2 nibble unpack of int4.rs:600-650 (32 packed bytes -> 64 i8 per
 * step, then the scalar tail). The 4-bit sign extension here is a pshufb
 * table lookup of the nibble's value in [-8, 7]; the lo/hi interleave is the
 * byte unpack plus the 128-bit lane fix-up the layout needs. */
__attribute__((target("avx2"))) static void unpack_avx2(const uint8_t* src, size_t len, int8_t* out) {
    const __m256i lut = _mm256_setr_epi8(0, 1, 2, 3, 4, 5, 6, 7, -8, -7, -6, -5, -4, -3, -2, -1, 0, 1, 2, 3, 4, 5, 6,
                                         7, -8, -7, -6, -5, -4, -3, -2, -1);
    const __m256i m4 = _mm256_set1_epi8(0x0f);
    size_t blocks = len / 32;
    for (size_t b = 0; b < blocks; ++b) {
        __m256i v = _mm256_loadu_si256((const __m256i*)(src + 32 * b));
        __m256i lo = _mm256_shuffle_epi8(lut, _mm256_and_si256(v, m4));
        __m256i hi = _mm256_shuffle_epi8(lut, _mm256_and_si256(_mm256_srli_epi16(v, 4), m4));
        __m256i il = _mm256_unpacklo_epi8(lo, hi);
        __m256i ih = _mm256_unpackhi_epi8(lo, hi);
        _mm256_storeu_si256((__m256i*)(out + 64 * b), _mm256_permute2x128_si256(il, ih, 0x20));
        _mm256_storeu_si256((__m256i*)(out + 64 * b + 32), _mm256_permute2x128_si256(il, ih, 0x31));
    }
    unpack_scalar(src + 32 * blocks, len - 32 * blocks, out + 64 * blocks);
}

static void unpack_nibbles(const uint8_t* src, size_t len, int8_t* out) {
    __builtin_cpu_init();
    if (__builtin_cpu_supports("avx2"))
        unpack_avx2(src, len, out);
    else
        unpack_scalar(src, len, out);
}

/* int4.rs:280-302 igemm_s4s8_unpacked */
static void s4s8_unpacked(const int8_t* a, const int8_t* b, const float* scales, size_t group, size_t m, size_t k,
                          size_t n, float* out) {
    const size_t groups = k / group;
    for (size_t mi = 0; mi < m; ++mi) {
        const int8_t* ar = a + mi * k;
        for (size_t ni = 0; ni < n; ++ni) {
            const int8_t* br = b + ni * k;
            const float* sr = scales + ni * groups;
            float acc_f = 0.0f;
            for (size_t g = 0; g < groups; ++g) {
                int32_t acc_i = 0;
                for (size_t kk = g * group; kk < (g + 1) * group; ++kk) acc_i += (int32_t)ar[kk] * (int32_t)br[kk];
                acc_f += sr[g] * (float)acc_i;
            }
            out[mi * n + ni] = acc_f;
        }
    }
}

void cpu_igemm_s4s8(int kind, const int8_t* a, const uint8_t* b_packed, const float* scales, size_t group, size_t m,
                    size_t k, size_t n, float* out) {
    if (kind == CPU_I4_PACKED) {
        s4s8_packed(a, b_packed, scales, group, m, k, n, out);
        return;
    }
    int8_t* b = (int8_t*)malloc(n * k);
    unpack_nibbles(b_packed, n * (k / 2), b);
    s4s8_unpacked(a, b, scales, group, m, k, n, out);
    free(b);
}

int cpu_moe_prefill_i4(int kind, const float* x, size_t t, size_t h, size_t inter, size_t n_experts, size_t top_k,
                       const uint32_t* idx, const float* gates, size_t group, const uint8_t* wg, const float* sg,
                       const uint8_t* wu, const float* su, const uint8_t* wd, const float* sd, float* out) {
    if (group != 16 && group != 32) return ORACLE_E_SHAPE;
    if (h % group || inter % group) return ORACLE_E_SHAPE;
    for (size_t r = 0; r < t * top_k; ++r)
        if (idx[r] >= n_experts) return ORACLE_E_SHAPE;
    const size_t gh = h / group, gi = inter / group;
    int8_t* xq = (int8_t*)malloc(t * h);
    float* xs = (float*)malloc(t * sizeof(float));
    int8_t* sub = (int8_t*)malloc(t * h);
    size_t* tok_of = (size_t*)malloc(t * sizeof(size_t));
    size_t* slot_of = (size_t*)malloc(t * sizeof(size_t));
    float* g = (float*)malloc(t * inter * sizeof(float));
    float* u = (float*)malloc(t * inter * sizeof(float));
    float* act = (float*)malloc(inter * sizeof(float));
    int8_t* aq = (int8_t*)malloc(t * inter);
    float* as2 = (float*)malloc(t * sizeof(float));
    float* y = (float*)malloc(t * h * sizeof(float));
    for (size_t r = 0; r < t; ++r) xs[r] = oracle_quantize_row_i8_te(x + r * h, h, xq + r * h);
    memset(out, 0, t * h * sizeof(float));
    for (size_t e = 0; e < n_experts; ++e) {
        size_t me = 0;
        for (size_t tok = 0; tok < t; ++tok)
            for (size_t j = 0; j < top_k; ++j)
                if (idx[tok * top_k + j] == e) {
                    tok_of[me] = tok;
                    slot_of[me] = j;
                    memcpy(sub + me * h, xq + tok * h, h);
                    ++me;
                    break;
                }
        if (!me) continue;
        cpu_igemm_s4s8(kind, sub, wg + e * inter * (h / 2), sg + e * inter * gh, group, me, h, inter, g);
        cpu_igemm_s4s8(kind, sub, wu + e * inter * (h / 2), su + e * inter * gh, group, me, h, inter, u);
        for (size_t r = 0; r < me; ++r) {
            const float s = xs[tok_of[r]];
            for (size_t i = 0; i < inter; ++i) {
                float gv = g[r * inter + i] * s;
                float uv = u[r * inter + i] * s;
                act[i] = oracle_silu(gv) * uv;
            }
            as2[r] = oracle_quantize_row_i8_te(act, inter, aq + r * inter);
        }
        cpu_igemm_s4s8(kind, aq, wd + e * h * (inter / 2), sd + e * h * gi, group, me, inter, h, y);
        /* every slot of the token routed to e adds the member's output, in
         * slot order (decoder.rs:2156-2160 pushes one member per slot) */
        for (size_t r = 0; r < me; ++r) {
            float* o = out + tok_of[r] * h;
            for (size_t j = slot_of[r]; j < top_k; ++j) {
                if (idx[tok_of[r] * top_k + j] != e) continue;
                const float wj = gates[tok_of[r] * top_k + j];
                for (size_t c = 0; c < h; ++c) {
                    float yv = y[r * h + c] * as2[r];
                    float p = wj * yv;
                    o[c] = o[c] + p;
                }
            }
        }
    }
    free(xq);
    free(xs);
    free(sub);
    free(tok_of);
    free(slot_of);
    free(g);
    free(u);
    free(act);
    free(aq);
    free(as2);
    free(y);
    return ORACLE_OK;
}
