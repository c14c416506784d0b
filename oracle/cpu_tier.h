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

/* `batch` independent products (instance i: a + i*m*k, b + i*n*k, out + i*m*n,
 * out += A.B^T), one task per instance over the pool. */
void cpu_igemm_s8s8_batched(int tier, const int8_t* a, const int8_t* b, size_t batch, size_t m, size_t k,
                            size_t n, int32_t* out);

/* nn::linear_int8_dynamic (nn.rs:151-173): the dynamic activation rule per
 * row, i32 products in 64-output-row blocks over the pool, ((f32)acc * a_s) *
 * w_s. y [m][n]. */
void cpu_linear_i8_dynamic(int tier, const float* x, size_t m, size_t k, const int8_t* w, const float* ws,
                           size_t n, float* y);

/* decode_mlp_i8 with the shared expert (swg NULL: none): the routed experts
 * and the shared one as concurrent serial tasks per token. */
int cpu_moe_decode_shared(int tier, const float* hidden, size_t t, size_t h, size_t inter, size_t n_experts,
                          size_t top_k, const float* router, const int8_t* wg, const float* sg, const int8_t* wu,
                          const float* su, const int8_t* wd, const float* sd, int norm_topk, float routed_scale,
                          const int8_t* swg, const float* ssg, const int8_t* swu, const float* ssu,
                          const int8_t* swd, const float* ssd, size_t shared_inter, float* out, uint32_t* idx,
                          float* gates);

/* One decoder layer of batched_decode_step_i8_streams (decoder.rs:2812-2933)
 * for b streams (hidden 1280, 10 heads x 128): x [b][1280] in place; stream
 * s's ring regions and cursors are advanced by its ring write. */
int cpu_decoder_layer_step(int tier, float* x, size_t b, const uint32_t* positions, float* const* ref_k,
                           float* const* ref_v, size_t ref_cap, const uint32_t* prefill_len, float* const* ring_k,
                           float* const* ring_v, uint32_t* ring_len, uint32_t* ring_pos, const float* input_ln,
                           const float* post_ln, float eps, float theta, const int8_t* wqkv, const float* sqkv,
                           const int8_t* wo, const float* so, const float* router, size_t n_experts, size_t top_k,
                           size_t inter, const int8_t* wg, const float* sg, const int8_t* wu, const float* su,
                           const int8_t* wd, const float* sd, const int8_t* swg, const float* ssg,
                           const int8_t* swu, const float* ssu, const int8_t* swd, const float* ssd,
                           size_t shared_inter);

/* ---- int4 (cpu_int4.c, built -O3 with LLVM for the x86-64 baseline ISA, as
 * rustc's release profile builds the reference) ----------------------------
 * The reference's two x86 int4 paths (int4.rs:454-460: no x86 MAC kernel):
 * kind CPU_I4_PACKED = s4s8_packed_kernel_scalar (int4.rs:304-343),
 * kind CPU_I4_UNPACK = igemm_s4s8 (int4.rs:245-278: the AVX2 nibble unpack of
 * int4.rs:560-650 once per call, then igemm_s4s8_unpacked). out [m][n] is
 * overwritten. */
enum { CPU_I4_PACKED = 0, CPU_I4_UNPACK = 1 };
void cpu_igemm_s4s8(int kind, const int8_t* a, const uint8_t* b_packed, const float* scales, size_t group,
                    size_t m, size_t k, size_t n, float* out);
/* moe_block over int4 experts with given routing (the structure of
 * decoder.rs:2142-2181): each routed expert's members gathered in token
 * order, its gate/up/down products as one m = M_e call each, SwiGLU and the
 * ties-even act quantize per member, out[t] += w * y in ascending expert
 * order; one thread. Same arguments as oracle_moe_prefill_i4. */
int cpu_moe_prefill_i4(int kind, const float* x, size_t t, size_t h, size_t inter, size_t n_experts,
                       size_t top_k, const uint32_t* idx, const float* gates, size_t group, const uint8_t* wg,
                       const float* sg, const uint8_t* wu, const float* su, const uint8_t* wd, const float* sd,
                       float* out);

#ifdef __cplusplus
}
#endif
#endif
