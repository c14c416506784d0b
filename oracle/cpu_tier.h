/*
 * cpu_tier.h — the reference's CPU int8 tier, restated in C for the CPU
 * baseline bench.py reports beside the GPU numbers (TEST/BENCH
 * INFRASTRUCTURE ONLY: never linked into the product library).
 *
 * Kernels follow src/simd/x86.rs (2x2 register blocking; AVX-512-VNNI and
 * AVX-VNNI via vpdpbusd with the +128 S8S8 correction; AVX2 via vpmaddwd;
 * scalar K tail), selected in the reference's order
 * avx512vnni > avxvnni > avx2 > scalar (src/simd/dispatch.rs:179-200).
 * Threading follows the reference: GEMV output rows in 64-row blocks fanned
 * over all host threads (decoder.rs:1582, :1621-1640); MoE decode runs the
 * top-k experts of a token as concurrent serial tasks (decoder.rs:2231-2252)
 * and the T tokens one after another (decoder.rs:2924-2930).
 */
#ifndef FOCR_CPU_TIER_H
#define FOCR_CPU_TIER_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { CPU_TIER_SCALAR = 0, CPU_TIER_AVX2 = 1, CPU_TIER_AVXVNNI = 2, CPU_TIER_AVX512VNNI = 3 };

/* Best tier available on this host, in the reference's order. */
int cpu_detect_tier(void);
/* 1 if this host supports the tier's instructions. */
int cpu_tier_available(int tier);
const char* cpu_tier_tag(int tier);          /* "avx512vnni", ... */
const char* cpu_tier_feature(int tier);      /* "x86_64+avx512vnni", ... */
/* Thread pool size (defaults to all logical CPUs; 0 keeps the default). */
int cpu_set_threads(int n);
int cpu_threads(void);

/* out[M,N] += A . B^T on the given tier (single thread). */
void cpu_igemm_s8s8(int tier, const int8_t* a, const int8_t* b, size_t m, size_t k, size_t n,
                    int32_t* out);

/* gemv_i8_batched on the tier with 64-row blocks over the pool. */
void cpu_gemv_i8(int tier, const float* x, size_t m, const int8_t* w, const float* scales,
                 size_t n, size_t k, float* y);
/* LM head: gemv + first-max argmax per row. */
void cpu_lm_head_i8(int tier, const float* x, size_t m, const int8_t* w, const float* scales,
                    size_t n, size_t k, float* logits, uint32_t* argmax);

/* MoE decode step over t tokens (same arguments as oracle_moe_decode, routed
 * experts only). Returns 0 or ORACLE_E_ROUTE. */
int cpu_moe_decode(int tier, const float* hidden, size_t t, size_t h, size_t inter,
                   size_t n_experts, size_t top_k, const float* router, const int8_t* wg,
                   const float* sg, const int8_t* wu, const float* su, const int8_t* wd,
                   const float* sd, int norm_topk, float routed_scale, float* out, uint32_t* idx,
                   float* gates);

#ifdef __cplusplus
}
#endif
#endif
