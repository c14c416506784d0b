/*
 * focr_oracle.h — CPU oracle for the quantized decoder hot path.
 *
 * TEST INFRASTRUCTURE ONLY. This is a plain-C restatement of the reference's
 * scalar semantics (Dicklesworthstone/franken_ocr v0.3.0, Rust). It is the
 * checker the parity tests compare the HIP path against, and the CPU baseline
 * that bench.py times beside the GPU. Nothing in the product library links,
 * loads or calls it: only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may.
 *
 * Every function cites the reference file:line it restates. Floating-point
 * code is compiled with -ffp-contract=off so each IEEE operation rounds on its
 * own, as Rust does (Rust never contracts a*b+c into an FMA).
 *
 * Pinning (what checks each function beyond restating its formula; see
 * tests/test_oracle.py):
 *   igemm_s8s8/u8s8   — hand values (scalar.rs:176-220), K=6848 extremes
 *                       (scalar.rs:227-262), i64 brute force.
 *   selftest fills    — xs32 stream regenerated independently in numpy.
 *   quantize_row_i8*  — quantizer known answers (quant/int8.rs:300-366,
 *                       nn.rs:600-628) + half-away vs ties-even split cases.
 *   argmax_row        — sampler.rs:618-640 (ties, NaN, -inf, all-NaN -> 0).
 *   ngram_bans/sample — sampler.rs:717-925 known answers (n-gram sizes 1/2/35,
 *                       window 0/2/16/128/1024 boundaries, whitelist,
 *                       out-of-range ids, all-banned row) + a brute-force
 *                       re-derivation from the n-gram definition.
 *   route             — moe.rs:777-1028 known answers; the f64 logit/softmax
 *                       rule is this build's documented definition
 *                       (router numerics in the reference live in the
 *                       un-vendored ft-kernel-cpu: parity unpinned there).
 *   expert/moe decode — hand SwiGLU value (moe.rs:892-915); i32 accumulators
 *                       vs brute force; the f32 combine order vs a float64
 *                       recomputation within tolerance.
 *   int4              — sign-extension table, unpack fixtures, adversarial
 *                       32,512 cell, single-group == int8 per-channel
 *                       (int4.rs:660-925), independent spec oracle.
 *   ring / attention  — rswa.rs:1475-1613 (single key, equal scores, online
 *                       == naive softmax, warm-up/steady-state slots) plus a
 *                       float64 softmax recomputation.
 */
#ifndef FOCR_ORACLE_H
#define FOCR_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* status codes (match the product library's, so tests compare them) */
#define ORACLE_OK 0
#define ORACLE_E_SHAPE (-1)
#define ORACLE_E_ROUTE (-7)

/* ---- src/simd/scalar.rs ------------------------------------------------ */
int oracle_igemm_s8s8(const int8_t* a, const int8_t* b, size_t m, size_t k, size_t n,
                      int32_t* out);
int oracle_igemm_u8s8(const uint8_t* a, const int8_t* b, size_t m, size_t k, size_t n,
                      int32_t* out);

/* ---- src/simd/dispatch.rs self-test battery ----------------------------- */
uint32_t oracle_xs32(uint32_t* state);
size_t oracle_selftest_n_shapes(void);
int oracle_selftest_shape(size_t i, const char** label, size_t* m, size_t* k, size_t* n,
                          uint32_t* seed);
int oracle_selftest_fill_s8(size_t i, int8_t* a, int8_t* b);
int oracle_selftest_fill_u8(size_t i, uint8_t* a, int8_t* b);

/* ---- src/native_engine/decoder.rs quantizers / GEMV --------------------- */
float oracle_quantize_row_i8(const float* x, size_t k, int8_t* q);
float oracle_quantize_row_i8_te(const float* x, size_t k, int8_t* q);
void oracle_gemv_i8_batched(const float* x, size_t m, const int8_t* w, const float* scales,
                            size_t n, size_t k, int8_t* xq, float* a_scales, int32_t* acc,
                            float* y);
void oracle_dequant_i8(const int32_t* acc, size_t m, size_t n, const float* a_scales,
                       const float* w_scales, float* y);

/* ---- src/native_engine/sampler.rs --------------------------------------- */
int oracle_argmax_row(const float* logits, size_t n, uint32_t* idx);

/* sampler.rs:191-235 ban set (scan order, repeats kept) and :346-395 greedy
 * sample of one row under it (masked nullable). */
size_t oracle_ngram_bans(const uint32_t* seq, size_t len, size_t ngram, size_t window, const uint32_t* white,
                         size_t n_white, size_t vocab, uint32_t* bans);
int oracle_sample(const float* row, size_t n, const uint32_t* seq, size_t len, size_t ngram, size_t window,
                  const uint32_t* white, size_t n_white, float* masked, uint32_t* token);
/* LM head: per-row quantize + GEMV + dequant + argmax (decoder.rs:2275-2296,
 * 2943-2965 with sampler.rs:168-186). */
int oracle_lm_head_i8(const float* x, size_t m, const int8_t* w, const float* scales, size_t n,
                      size_t k, float* logits, uint32_t* argmax);

/* ---- src/native_engine/moe.rs ------------------------------------------- */
int oracle_route(const float* hidden, size_t t, size_t h, const float* gate, size_t n_experts,
                 size_t top_k, int norm_topk, float routed_scale, uint32_t* idx, float* w,
                 float* probs);
float oracle_silu(float x);
void oracle_expert_i8(const float* x, size_t h, size_t inter, const int8_t* wg, const float* sg,
                      const int8_t* wu, const float* su, const int8_t* wd, const float* sd,
                      float* y, float* act, int8_t* aq, float* a_scale2);
int oracle_moe_decode(const float* hidden, size_t t, size_t h, size_t inter, size_t n_experts,
                      size_t top_k, const float* router, const int8_t* wg, const float* sg,
                      const int8_t* wu, const float* su, const int8_t* wd, const float* sd,
                      int norm_topk, float routed_scale, const int8_t* shared_wg,
                      const float* shared_sg, const int8_t* shared_wu, const float* shared_su,
                      const int8_t* shared_wd, const float* shared_sd, size_t shared_inter,
                      float* out, uint32_t* idx, float* gates);

/* ---- prefill int8 linear: nn::linear_int8_dynamic (nn.rs:151-173) ---------
 * The dynamic activation rule of docs/focrq-format.md:296-320: scale_a =
 * max|x|/127 (1.0 for an all-zero row), q = round_ties_even(clamp(x / scale_a,
 * -127, 127)) with TRUE division (not a reciprocal multiply). */
float oracle_quantize_row_dynamic(const float* x, size_t k, int8_t* q);
/* y[r][o] = ((f32)acc * scale_a[r]) * w_scale[o] (+ bias[o]); bias may be NULL.
 * xq [m][k] / x_scales [m] receive the quantized rows. */
int oracle_linear_i8_dynamic(const float* x, size_t m, size_t k, const int8_t* w, const float* w_scales,
                             size_t n, const float* bias, float* y, int8_t* xq, float* x_scales);
/* moe_block_i8 (decoder.rs:2142-2181) over given routing: each routed
 * expert's expert_mlp_i8 (decoder.rs:2120-2135: linear_int8_dynamic gate, silu,
 * linear_int8_dynamic up, product, linear_int8_dynamic down) on its member
 * tokens, scattered out[t] += w * y in ascending expert order (slot order
 * inside an expert); with shared_wg != NULL the shared expert's
 * expert_mlp_i8 over every token is added last at weight 1.0. */
int oracle_moe_prefill_i8(const float* x, size_t t, size_t h, size_t inter, size_t n_experts,
                          size_t top_k, const uint32_t* idx, const float* gates, const int8_t* wg,
                          const float* sg, const int8_t* wu, const float* su, const int8_t* wd,
                          const float* sd, const int8_t* shared_wg, const float* shared_sg,
                          const int8_t* shared_wu, const float* shared_su, const int8_t* shared_wd,
                          const float* shared_sd, size_t shared_inter, float* out);

/* ---- the decode layer's other ops (decoder.rs:2542-2627) ------------------
 * nn::rms_norm (nn.rs:240-253) calls ft-kernel-cpu's rms_norm_forward_f32,
 * which is not in the reference tree; this build fixes y = (x * rstd) * w
 * with the sum of squares in f64 (increasing index) and rstd = (float)(1 /
 * sqrt(ss / n + eps)) in f64 (w NULL: no weight). Pinned by the reference's
 * hand values at 1e-6 (nn.rs:438-458); the exact f32 bits are unpinned. */
void oracle_rms_norm(const float* x, size_t n, const float* w, float eps, float* y);
/* RopeTable::build + apply_rope (decoder.rs:150-268) on one row of n_heads
 * blocks of head_dim at absolute position pos: inv_freq[i] = (f32)(1 /
 * theta^(2i/head_dim)) in f64, angle = (f32)pos * inv_freq[i], NEOX
 * rotate_half over the two halves of each head. */
int oracle_rope(float* x, size_t n_heads, size_t head_dim, size_t pos, float theta);

/* ---- src/simd/int4.rs ---------------------------------------------------- */
int8_t oracle_sign_extend_nibble(uint8_t nib);
void oracle_unpack_byte(uint8_t b, int8_t* lo, int8_t* hi);
int oracle_unpack_to_i8(const uint8_t* packed, size_t n, size_t k, int8_t* out);
int oracle_igemm_s4s8_packed(const int8_t* a, const uint8_t* b_packed, const float* scales,
                             size_t group, size_t m, size_t k, size_t n, float* out);
int oracle_s4s8_group_i32(const int8_t* a, const uint8_t* b_packed, size_t group, size_t m,
                          size_t k, size_t n, int32_t* partials);

/* int4 prefill MoE (this build's composition of the int4 kernel contract with
 * moe_block_i8's grouped structure, decoder.rs:2142-2181). */
int oracle_moe_prefill_i4(const float* x, size_t t, size_t h, size_t inter, size_t n_experts,
                          size_t top_k, const uint32_t* idx, const float* gates, size_t group,
                          const uint8_t* wg, const float* sg, const uint8_t* wu, const float* su,
                          const uint8_t* wd, const float* sd, float* out, int8_t* xq,
                          float* x_scales);

/* ---- src/quant ----------------------------------------------------------- */
int oracle_quantize_int8_f32(const float* w, size_t n, size_t k, int8_t* q, float* scales);
int oracle_pack_int4_f32(const float* w, size_t n, size_t k, size_t group, uint8_t* packed,
                         float* scales);

/* ---- src/native_engine/rswa.rs ------------------------------------------- */
#define ORACLE_NUM_HEADS 10
#define ORACLE_HEAD_DIM 128
#define ORACLE_RING_WINDOW 128
int oracle_ring_write(float* ring_k, float* ring_v, uint32_t* ring_len, uint32_t* ring_pos,
                      const float* k_step, const float* v_step, uint32_t* slot);
int oracle_decode_attention(const float* ref_k, const float* ref_v, size_t ref_cap,
                            size_t prefill_len, const float* ring_k, const float* ring_v,
                            size_t ring_len, const float* q, float* out);

/* ---- decoder.rs:568-640 prefill_attention / :1282-1340 chunk_prefill_attention
 * Causal multi-head attention over token-major f32 [rows, num_heads*head_dim]
 * matrices (head h in columns h*head_dim ..). Query row i of a chunk sits at
 * global position t = c0 + i and attends keys [0, t]; scale = 1/sqrt(head_dim).
 * chunk: q_chunk [cs, dim], k_prefix / v_prefix [c1, dim], c0 + cs == c1
 * (ORACLE_E_SHAPE otherwise). prefill_attention is the chunk with c0 = 0.
 * Evaluated in float64 and rounded once; the _f32 variant is the f32
 * restatement in the reference's described order (ascending dims and keys). */
int oracle_chunk_prefill_attention(const float* q_chunk, size_t cs, const float* k_prefix,
                                   const float* v_prefix, size_t c1, size_t num_heads,
                                   size_t head_dim, size_t c0, float* out);
int oracle_chunk_prefill_attention_f32(const float* q_chunk, size_t cs, const float* k_prefix,
                                       const float* v_prefix, size_t c1, size_t num_heads,
                                       size_t head_dim, size_t c0, float* out);
int oracle_prefill_attention(const float* q, const float* k, const float* v, size_t seq,
                             size_t num_heads, size_t head_dim, float* out);

#ifdef __cplusplus
}
#endif
#endif
