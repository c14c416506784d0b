/*
 * focr_hip.h — C ABI of the MI355X (gfx950) tier for franken_ocr's quantized
 * decoder hot path.
 *
 * Two layers, both plain C (pointers + sizes, no framework types):
 *
 *  1. Drop-in kernel tier. Same contract as the reference's dispatched
 *     `simd` entry points (host slices in, host slices out, synchronous,
 *     `+=` for int8 / overwrite for int4). A Rust `IsaTier::Gfx950` arm calls
 *     these exactly where it calls `x86::igemm_s8s8` today.
 *
 *  2. Device-resident engine ops. Weights are uploaded once into HBM
 *     (the analogue of `DecoderWeightCacheI8::build`, decoder.rs:2018-2116)
 *     and every per-token op works on device pointers, stream-ordered on the
 *     context's HIP stream. These replace the engine functions one level up
 *     (gemv_i8, lm_head_cached_i8 + argmax, decode_mlp_i8, RingCache +
 *     decode_attention), because per-call host slices would copy the 165 MB
 *     LM-head panel over PCIe on every token.
 *
 * Every function returns an int32_t status (FOCR_HIP_OK == 0). On failure the
 * calling thread's focr_hip_last_error() holds the message; for contract
 * violations the text is the one the reference panics with
 * (e.g. "igemm_s8s8: a.len 2 != m*k 1"), so a Rust binding can re-raise it
 * as the same panic. Entry points taking a context are thread-safe (one
 * mutex per context serialises use of its stream).
 *
 * Citations are to Dicklesworthstone/franken_ocr v0.3.0.
 */
#ifndef FOCR_HIP_H
#define FOCR_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ------------------------------------------------------ */
#define FOCR_HIP_OK 0
#define FOCR_HIP_E_SHAPE (-1)      /* shape/length contract violation (a Rust panic) */
#define FOCR_HIP_E_HIP (-2)        /* HIP runtime error */
#define FOCR_HIP_E_OOM (-3)        /* device allocation failed */
#define FOCR_HIP_E_NO_DEVICE (-4)  /* no usable gfx950 device */
#define FOCR_HIP_E_BAD_HANDLE (-5) /* null / foreign handle */
#define FOCR_HIP_E_ARG (-6)        /* invalid argument (null pointer, bad flag) */
#define FOCR_HIP_E_ROUTE (-7)      /* moe.rs:261-265 "no finite router score" */
#define FOCR_HIP_E_STATE (-8)      /* rswa.rs:452-455/869-887 state errors */
#define FOCR_HIP_E_FORMAT (-9)     /* FocrError::FormatMismatch of the weight container */
#define FOCR_HIP_E_NOT_FOUND (-10) /* FocrError::ModelNotFound: weights file unreadable */
#define FOCR_HIP_E_NOT_IMPLEMENTED (-11) /* FocrError::NotImplemented (temperature > 0) */

/* Stored dtypes of the weight container (weights.rs:148-170 DType). */
#define FOCR_HIP_DT_F32 0
#define FOCR_HIP_DT_F16 1
#define FOCR_HIP_DT_BF16 2
#define FOCR_HIP_DT_QINT8_PER_CHAN 3
#define FOCR_HIP_DT_QINT4_PER_GROUP 4

typedef struct focr_hip_ctx focr_hip_ctx;
typedef struct focr_hip_qint8 focr_hip_qint8;
typedef struct focr_hip_moe_layer focr_hip_moe_layer;
typedef struct focr_hip_moe_layer_i4 focr_hip_moe_layer_i4;
typedef struct focr_hip_decoder_layer focr_hip_decoder_layer;
typedef struct focr_hip_decoder focr_hip_decoder;
typedef struct focr_hip_rswa focr_hip_rswa;
typedef struct focr_hip_focrq focr_hip_focrq;
typedef struct focr_hip_focrq_writer focr_hip_focrq_writer;

/* Message of the last failed call on this thread ("" if none). */
const char* focr_hip_last_error(void);
/* Library version string. */
const char* focr_hip_version(void);

/* ---- context ----------------------------------------------------------- */
/* Number of visible HIP devices (0 when none). */
int32_t focr_hip_device_count(int32_t* count);
/* Create a context on `device`: one default-priority HIP stream plus the
 * scratch buffers the engine ops reuse. Fails with E_NO_DEVICE when the
 * device is absent or is not gfx950 (the library ships gfx950 code only). */
int32_t focr_hip_ctx_create(int32_t device, focr_hip_ctx** out);
int32_t focr_hip_ctx_destroy(focr_hip_ctx* ctx);
/* Block until all work queued on the context's stream has finished. */
int32_t focr_hip_ctx_synchronize(focr_hip_ctx* ctx);
/* hipDeviceSynchronize on the context's device (whole-device barrier). */
int32_t focr_hip_device_synchronize(focr_hip_ctx* ctx);
/* The context's hipStream_t, for callers that order their own work on it. */
int32_t focr_hip_ctx_stream(focr_hip_ctx* ctx, void** stream);
/* No counterpart in the reference (a diagnostic): the bytes the context's
 * grow-only scratch slots hold now; an entry point that allocates nothing
 * leaves it unchanged. */
int32_t focr_hip_ctx_scratch_bytes(focr_hip_ctx* ctx, size_t* bytes);
/* No counterpart in the reference (a test hook): the bound, in 10 ns ticks
 * (default 1000 = 10 us), of the MoE route's wait for the other blocks of a
 * token; a part not seen within it is computed by the waiting block itself,
 * with the same result. 0 takes that path for every part. */
int32_t focr_hip_ctx_set_route_wait(focr_hip_ctx* ctx, uint32_t ticks);
/* Device name / gcnArchName / CU count of the context's device. */
int32_t focr_hip_ctx_device_info(focr_hip_ctx* ctx, char* arch, size_t arch_cap,
                                 int32_t* cu_count);

/* ---- tier reflection (dispatch.rs:48-138 IsaTier::tag/feature_string) --- */
/* tag "gfx950", feature "gfx950+mfma-i8" — the strings `robot backends`
 * reports for the GPU tier beside "avx512vnni"/"x86_64+avx512vnni". */
int32_t focr_hip_tier(char* tag, size_t tag_cap, char* feature, size_t feature_cap);

/* ---- device buffers (plumbing for callers without a device allocator) ---- */
int32_t focr_hip_dmalloc(focr_hip_ctx* ctx, size_t bytes, void** out);
int32_t focr_hip_dfree(focr_hip_ctx* ctx, void* ptr);
/* Synchronous copies (they also wait for the context's stream). */
int32_t focr_hip_h2d(focr_hip_ctx* ctx, void* dst, const void* src, size_t bytes);
int32_t focr_hip_d2h(focr_hip_ctx* ctx, void* dst, const void* src, size_t bytes);
/* Stream-ordered device-to-device copy. */
int32_t focr_hip_d2d(focr_hip_ctx* ctx, void* dst, const void* src, size_t bytes);

/* =========================================================================
 * Layer 1 — drop-in kernel tier (host pointers, synchronous)
 * ========================================================================= */

/* simd::igemm_s8s8 (simd/mod.rs:30-46, scalar.rs:78-116, dispatch.rs:246-262):
 * out[M,N] += A[M,K] (i8, row-major) . B[N,K]^T (i8, output-channel-major),
 * i32 accumulation. Length checks and messages as scalar.rs:79-102. */
int32_t focr_hip_igemm_s8s8(focr_hip_ctx* ctx, const int8_t* a, size_t a_len, const int8_t* b,
                            size_t b_len, size_t m, size_t k, size_t n, int32_t* out,
                            size_t out_len);
/* simd::igemm_u8s8 (scalar.rs:129-166, dispatch.rs:276-289): A is u8. */
int32_t focr_hip_igemm_u8s8(focr_hip_ctx* ctx, const uint8_t* a, size_t a_len, const int8_t* b,
                            size_t b_len, size_t m, size_t k, size_t n, int32_t* out,
                            size_t out_len);
/* simd::int4::igemm_s4s8_packed (int4.rs:437-461; contract :304-343, checks
 * :350-402): out[M,N] = sum_g scale[n,g] * (i32 dot over group g), summed in
 * f32 in increasing g; out is overwritten. group in {16, 32}. */
int32_t focr_hip_igemm_s4s8_packed(focr_hip_ctx* ctx, const int8_t* a, size_t a_len,
                                   const uint8_t* b_packed, size_t b_len, const float* scales,
                                   size_t scales_len, size_t group, size_t m, size_t k, size_t n,
                                   float* out, size_t out_len);
/* simd::int4::igemm_s4s8 (int4.rs:170-229): the same function under the
 * unpack-then-int8 entry's name and messages (its result is identical). */
int32_t focr_hip_igemm_s4s8(focr_hip_ctx* ctx, const int8_t* a, size_t a_len,
                            const uint8_t* b_packed, size_t b_len, const float* scales,
                            size_t scales_len, size_t group, size_t m, size_t k, size_t n,
                            float* out, size_t out_len);
/* simd::int4::unpack_to_i8 (int4.rs:125-142): [n, k/2] packed -> [n, k] i8. */
int32_t focr_hip_unpack_to_i8(focr_hip_ctx* ctx, const uint8_t* b_packed, size_t b_len, size_t n,
                              size_t k, int8_t* out, size_t out_len);
/* Test entry with no single reference counterpart: the per-group i32
 * partial sums inside s4s8_packed_kernel_scalar (int4.rs:322-337), written
 * as partials[m][n][k/group], so int4 "i32 accumulators" can be checked. */
int32_t focr_hip_debug_s4s8_group_i32(focr_hip_ctx* ctx, const int8_t* a, size_t a_len,
                                      const uint8_t* b_packed, size_t b_len, size_t group,
                                      size_t m, size_t k, size_t n, int32_t* partials,
                                      size_t partials_len);

/* The runtime self-test behind `focr robot selftest` (dispatch.rs:376-429,
 * cli.rs:1955-2002): the 12-shape x {s8s8, u8s8} battery run through the
 * gfx950 tier and compared lane by lane with an in-process scalar check.
 * Writes a JSON report {"selected","available","all_ok","cases":[...]} into
 * json (NUL-terminated, truncated to cap) and sets *all_ok. */
int32_t focr_hip_selftest(focr_hip_ctx* ctx, char* json, size_t cap, int32_t* all_ok);

/* Device-pointer forms of the tier (stream-ordered, no host copies). */
int32_t focr_hip_igemm_s8s8_dev(focr_hip_ctx* ctx, const int8_t* a, const int8_t* b, size_t m,
                                size_t k, size_t n, int32_t* out);
int32_t focr_hip_igemm_u8s8_dev(focr_hip_ctx* ctx, const uint8_t* a, const int8_t* b, size_t m,
                                size_t k, size_t n, int32_t* out);
/* `batch` independent s8s8 products in one launch (device pointers): for
 * instance i, out[i] (m x n, i32) += a[i] (m x k) . b[i] (n x k)^T, with
 * a = [batch][m][k], b = [batch][n][k], out = [batch][m][n]. The per-instance
 * contract is simd::igemm_s8s8 (scalar.rs:78-116); the reference makes these
 * calls one expert at a time (decoder.rs:1634, :1920, :2358), this entry
 * takes all of them at once (e.g. 64 experts' gate projections). k must be a
 * positive multiple of 16 (<= 65536), a and b 16-byte aligned, batch <= 65535. */
int32_t focr_hip_igemm_s8s8_batched_dev(focr_hip_ctx* ctx, const int8_t* a, const int8_t* b,
                                        size_t batch, size_t m, size_t k, size_t n, int32_t* out);
int32_t focr_hip_igemm_s4s8_packed_dev(focr_hip_ctx* ctx, const int8_t* a,
                                       const uint8_t* b_packed, const float* scales, size_t group,
                                       size_t m, size_t k, size_t n, float* out);

/* =========================================================================
 * Layer 2 — device-resident engine ops (device pointers, stream-ordered)
 * ========================================================================= */

/* QInt8 weight handle (tensor.rs:149-179): w [n,k] i8 output-channel-major,
 * one f32 scale per output channel. _upload copies host arrays into HBM once;
 * _from_device wraps caller-owned device arrays (not freed by the handle). */
int32_t focr_hip_qint8_upload(focr_hip_ctx* ctx, const int8_t* w, const float* scales, size_t n,
                              size_t k, focr_hip_qint8** out);
int32_t focr_hip_qint8_from_device(focr_hip_ctx* ctx, const int8_t* w, const float* scales,
                                   size_t n, size_t k, focr_hip_qint8** out);
int32_t focr_hip_qint8_free(focr_hip_qint8* w);

/* One scale per row, x [m,k] f32 -> xq [m,k] i8, a_scales [m], by rule:
 * 0 = decoder.rs:1588-1597 quantize_row_i8 (round half away, reciprocal
 * multiply), 1 = :1647-1656 quantize_row_i8_te (ties to even, reciprocal
 * multiply), 2 = the dynamic activation rule of nn::linear_int8_dynamic
 * (docs/focrq-format.md:296-320: ties to even, true division). */
int32_t focr_hip_quantize_rows_i8(focr_hip_ctx* ctx, const float* x, size_t m, size_t k,
                                  int8_t* xq, float* a_scales, int32_t rule);

/* decoder.rs:1607 gemv_i8 (m = 1) and :2703-2747 gemv_i8_batched (m rows):
 * each row quantized with quantize_row_i8, y[m,n] = ((f32)acc * a_scale[m])
 * * scale[n]. m <= 32 per call. */
int32_t focr_hip_gemv_i8(focr_hip_ctx* ctx, const focr_hip_qint8* w, const float* x, size_t m,
                         float* y);
/* decoder.rs:1621-1640 gemv_i8_prequant: from already-quantized rows. acc
 * (nullable) receives the raw i32 accumulators [m,n]. */
int32_t focr_hip_gemv_i8_prequant(focr_hip_ctx* ctx, const focr_hip_qint8* w, const int8_t* xq,
                                  const float* a_scales, size_t m, float* y, int32_t* acc);

/* decoder.rs:2275-2296 lm_head_cached_i8 / :2943-2965 batched_lm_head_i8
 * (input = the already final-normed rows) followed by sampler.rs:168-186
 * argmax_row per row. logits [m,n] (nullable: skip writing them); argmax [m]
 * u32: first index of the maximum, NaN skipped, all-NaN row -> 0. */
int32_t focr_hip_lm_head_i8(focr_hip_ctx* ctx, const focr_hip_qint8* w, const float* x,
                            size_t m, float* logits, uint32_t* argmax);
/* Greedy decode with the sliding-window no-repeat-ngram ban folded into the
 * LM-head epilogue: decoder.rs:2319-2357 gemv_i8_ngram_masked /
 * :2381-2400 lm_head_cached_i8_ngram_masked (input = the already final-normed
 * rows) with the ban set of sampler.rs:191-235 / :269-278, then
 * sampler.rs:426-460 decode_step_premasked, for m streams at once (the
 * batched spine's per-stream ban, sampler.rs:491-545). Per row r:
 * history[r][0..history_len[r]) is stream r's generated sequence (device,
 * [m][history_cap] u32; history_len device [m]); bans use ngram_size /
 * window (0 = the whole history) / whitelist (device, nullable); logits
 * (nullable) receive the masked row; tokens [m] the argmax; is_eos
 * (nullable, u8 [m]) token == eos_token_id. With append = 1 the token is
 * written at history[r][history_len[r]] and history_len[r] is incremented
 * on the device. temperature > 0 -> E_NOT_IMPLEMENTED (sampler.rs:362-367).
 * check = 1 synchronises and reports a history_len over history_cap (or a
 * full history on append) as E_SHAPE. m <= 32. */
int32_t focr_hip_lm_head_sample_i8(focr_hip_ctx* ctx, const focr_hip_qint8* w, const float* x,
                                   size_t m, uint32_t* history, size_t history_cap,
                                   uint32_t* history_len, size_t ngram_size, size_t window,
                                   const uint32_t* whitelist, size_t n_whitelist, float temperature,
                                   uint32_t eos_token_id, int32_t append, float* logits,
                                   uint32_t* tokens, uint8_t* is_eos, int32_t check);
/* sampler.rs:491-545 batched_sample / batched_decode_step (and :346-395
 * sample per row) over given device logits [m, n] (read only): the same ban,
 * argmax, EOS flag and optional append as focr_hip_lm_head_sample_i8. */
int32_t focr_hip_sample_rows(focr_hip_ctx* ctx, const float* logits, size_t m, size_t n,
                             uint32_t* history, size_t history_cap, uint32_t* history_len,
                             size_t ngram_size, size_t window, const uint32_t* whitelist,
                             size_t n_whitelist, float temperature, uint32_t eos_token_id,
                             int32_t append, uint32_t* tokens, uint8_t* is_eos, int32_t check);
/* sampler.rs:168-186 argmax_row over m rows of n f32 logits. */
int32_t focr_hip_argmax_rows(focr_hip_ctx* ctx, const float* logits, size_t m, size_t n,
                             uint32_t* argmax);

/* ---- MoE layer (decoder.rs:1971-1982 CachedMlpI8::Moe) ------------------
 * router f32 [E, hidden]; gate/up i8 [E][inter][hidden] with scales
 * [E][inter]; down i8 [E][hidden][inter] with scales [E][hidden]. With
 * from_device = 0 the arrays are host memory and are uploaded once; with 1
 * they are caller-owned device arrays that the layer borrows. */
int32_t focr_hip_moe_layer_create(focr_hip_ctx* ctx, size_t hidden, size_t inter,
                                  size_t n_experts, size_t top_k, const float* router,
                                  const int8_t* wg, const float* sg, const int8_t* wu,
                                  const float* su, const int8_t* wd, const float* sd,
                                  int32_t from_device, focr_hip_moe_layer** out);
/* The fused shared expert (moe.rs:64-66; decoder.rs:2251, :2259-2261). */
int32_t focr_hip_moe_layer_set_shared(focr_hip_moe_layer* layer, size_t shared_inter,
                                      const int8_t* wg, const float* sg, const int8_t* wu,
                                      const float* su, const int8_t* wd, const float* sd,
                                      int32_t from_device);
int32_t focr_hip_moe_layer_free(focr_hip_moe_layer* layer);

/* decoder.rs:2199-2268 decode_mlp_i8 over t rows (the batched spine calls it
 * per stream, decoder.rs:2924-2930): route (moe.rs:181-266; router logits
 * and softmax in f64, rounded to f32), per (token, slot) the int8 SwiGLU
 * expert (decoder.rs:1744-1755), y *= gate, combine in slot order, plus the
 * shared expert when with_shared. hidden/out [t, hidden] f32; idx/gates
 * [t, top_k] (both nullable). Device pointers. t <= 16384 (more than 64 rows run
 * as consecutive chunks of 64: the same rows). Returns E_ROUTE when
 * a token has no finite router score (moe.rs:261-265) — detected on the
 * device and reported by a synchronising check only when check_route = 1. */
int32_t focr_hip_moe_decode(focr_hip_ctx* ctx, const focr_hip_moe_layer* layer,
                            const float* hidden, size_t t, int32_t norm_topk, float routed_scale,
                            int32_t with_shared, float* out, uint32_t* idx, float* gates,
                            int32_t check_route);
/* No counterpart in the reference. For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): focr_hip_moe_decode with the same arguments, kernels
 * and results, but every intermediate (quantized rows, routing, selection
 * matrices, act rows, expert outputs) lives in one statically allocated
 * device array per GPU of focr_hip_static_scratch_bytes() bytes (8 MiB, held
 * until the process ends), and the call makes no hipMalloc / hipFree or
 * other allocating call. A call needing more scratch than that returns
 * E_SHAPE (at hidden 1280, inter 896, top-6 every t <= 64 fits, with a
 * shared expert up to 1792 wide). Nothing in the array must start at zero;
 * it keeps the last call's contents. Every call on one GPU shares its
 * array, so the calls on one GPU are ordered: each call's stream waits for
 * the previous call's completion event (one event per GPU, created with the
 * array's address at context creation) and records its own, so calls from
 * several contexts or threads run one after another in the order they were
 * issued. A call issued while its stream is being captured into a graph is
 * not ordered that way: overlapping captured calls on one GPU race unless
 * the graphs order them. check_route = 1 synchronises (not capturable); 0
 * leaves the device flag unread. */
int32_t focr_hip_moe_decode_noalloc(focr_hip_ctx* ctx, const focr_hip_moe_layer* layer,
                                    const float* hidden, size_t t, int32_t norm_topk,
                                    float routed_scale, int32_t with_shared, float* out,
                                    uint32_t* idx, float* gates, int32_t check_route);
/* Size in bytes of the per-GPU static scratch of the allocation-free entry
 * points. */
size_t focr_hip_static_scratch_bytes(void);
/* moe.rs:181-266 route alone for t rows, 1 <= t <= 16384 (a decode step or
 * every row of a prefill chunk, moe.rs:181-243): idx/gates [t, top_k]
 * device pointers (required above 64 rows); probs (nullable) receives the
 * f32 softmax [t, E]. Synchronises to report E_ROUTE for the first row with
 * no finite router score. */
int32_t focr_hip_moe_route(focr_hip_ctx* ctx, const focr_hip_moe_layer* layer,
                           const float* hidden, size_t t, int32_t norm_topk, float routed_scale,
                           uint32_t* idx, float* gates, float* probs);

/* ---- int4 MoE layer for chunked prefill ----------------------------------
 * Experts as simd::int4 packed weights (int4.rs:304-343 layout, low nibble =
 * even k): gate/up [E][inter][hidden/2] with group scales
 * [E][inter][hidden/group], down [E][hidden][inter/2] with
 * [E][hidden][inter/group]; group in {16, 32}; hidden, inter multiples of 32
 * up to 4096. from_device as focr_hip_moe_layer_create. */
int32_t focr_hip_moe_layer_i4_create(focr_hip_ctx* ctx, size_t hidden, size_t inter,
                                     size_t n_experts, size_t group, const uint8_t* wg,
                                     const float* sg, const uint8_t* wu, const float* su,
                                     const uint8_t* wd, const float* sd, int32_t from_device,
                                     focr_hip_moe_layer_i4** out);
int32_t focr_hip_moe_layer_i4_free(focr_hip_moe_layer_i4* layer);
/* The grouped MoE block of decoder.rs:2142-2181 (moe_block_i8) over int4
 * experts, for t prefill rows with a given routing: x [t, hidden] f32; idx,
 * gates [t, top_k] (routing from moe::route or any other source). Per row:
 * quantize_row_i8_te (decoder.rs:1647-1656); per member (token, slot) of
 * expert e in (token, slot) order: g, u = int4 GEMMs (int4.rs:304-343 group
 * rule, exact) times the row scale, act = silu(g) * u, requantized with the
 * ties-even rule, y = int4 GEMM times the act scale; out[t] = sum of
 * gate * y over the token's members in ascending expert order. Device
 * pointers; t <= 16384, top_k <= 8. With check_idx = 1 the call synchronises
 * and returns E_SHAPE for an expert index >= n_experts. */
int32_t focr_hip_moe_prefill_i4(focr_hip_ctx* ctx, const focr_hip_moe_layer_i4* layer,
                                const float* x, size_t t, size_t top_k, const uint32_t* idx,
                                const float* gates, float* out, int32_t check_idx);

/* ---- prefill on int8 weights (int8 matrix cores, i32 accumulation) --------- */
/* nn.rs:151-173 linear_int8_dynamic on an uploaded QInt8 [n, k]: each row of
 * x [m, k] f32 quantized by the dynamic rule (rule 2 above), y [m, n] =
 * ((f32)acc * a_scale[row]) * w_scale[col] (+ bias[col]; bias nullable).
 * Device pointers. k must be a multiple of 64 (E_SHAPE otherwise). */
int32_t focr_hip_linear_i8_dynamic(focr_hip_ctx* ctx, const focr_hip_qint8* w, const float* x,
                                   size_t m, const float* bias, float* y);
/* decoder.rs:2142-2181 moe_block_i8 on an uploaded int8 MoE layer (the
 * decode layer's handle, focr_hip_moe_layer_create), for t prefill rows with
 * a given routing idx, gates [t, top_k] (e.g. moe::route_default): per member
 * (token, slot) of expert e, expert_mlp_i8 (decoder.rs:2120-2135) — three
 * linear_int8_dynamic products, act = silu(g) * u — and out[t] = the sum of
 * gate * y over the token's members in ascending expert order, plus (with
 * with_shared) the shared expert's expert_mlp_i8 of every row at weight 1.0.
 * Device pointers; t <= 16384; hidden and inter multiples of 64. With
 * check_idx = 1 the call synchronises and returns E_SHAPE for an expert
 * index >= n_experts. */
int32_t focr_hip_moe_prefill_i8(focr_hip_ctx* ctx, const focr_hip_moe_layer* layer, const float* x,
                                size_t t, const uint32_t* idx, const float* gates,
                                int32_t with_shared, float* out, int32_t check_idx);

/* ---- prefill attention on the f32 matrix cores -----------------------------
 * decoder.rs:1282-1340 chunk_prefill_attention: the cs = c1 - c0 queries
 * q_chunk [cs, num_heads*head_dim] (global positions [c0, c1), RoPE applied)
 * attend over the prefix k_prefix / v_prefix [c1, num_heads*head_dim] under
 * the causal mask — query t sees keys [0, t] — with scale 1/sqrt(head_dim):
 * ctx [cs, num_heads*head_dim] (pre-o_proj). Token-major (head h in columns
 * h*head_dim ..). E_SHAPE with the reference's message when c0 > c1 or
 * c0 + cs != c1 ("chunk_prefill_attention: chunk [c0, c0+cs) of cs rows does
 * not fit prefix c1"); head_dim must be 128 (E_SHAPE otherwise). f32
 * throughout (f32 MFMAs); agrees with the reference's f32 attention to
 * rounding (rel 1e-4). Device pointers. */
int32_t focr_hip_chunk_prefill_attention(focr_hip_ctx* ctx, const float* q_chunk, size_t cs,
                                         const float* k_prefix, const float* v_prefix, size_t c1,
                                         size_t num_heads, size_t head_dim, size_t c0, float* out);
/* decoder.rs:568-640 prefill_attention: the whole sequence, c0 = 0. */
int32_t focr_hip_prefill_attention(focr_hip_ctx* ctx, const float* q, const float* k, const float* v,
                                   size_t seq, size_t num_heads, size_t head_dim, float* out);

/* ---- R-SWA ring KV cache (rswa.rs:121-152 RingCache, :645-824 batched) ---
 * n_streams independent caches of one layer, f32, head-major per stream:
 * ref K/V [NUM_HEADS=10][ref_capacity][HEAD_DIM=128], ring K/V
 * [10][RING_WINDOW=128][128]. Cursor state (prefill_len, ring_len, ring_pos)
 * is kept on the host and follows the reference's rules exactly. */
int32_t focr_hip_rswa_create(focr_hip_ctx* ctx, size_t n_streams, size_t ref_capacity,
                             focr_hip_rswa** out);
int32_t focr_hip_rswa_free(focr_hip_rswa* cache);
/* rswa.rs:389-433 record_prefill: k/v head-major [10][seq][128] (device
 * pointers); resets ring_len = ring_pos = 0. */
int32_t focr_hip_rswa_record_prefill(focr_hip_ctx* ctx, focr_hip_rswa* cache, size_t stream,
                                     const float* k, const float* v, size_t seq);
/* rswa.rs:451-513 write_decode_step for every stream: k_steps/v_steps
 * [n_streams][10*128] device pointers; slots (host, nullable) receives each
 * stream's physical slot. */
int32_t focr_hip_rswa_write_decode_step(focr_hip_ctx* ctx, focr_hip_rswa* cache,
                                        const float* k_steps, const float* v_steps,
                                        uint32_t* slots);
/* rswa.rs:1320-1367 batched_decode_attention (per stream, rswa.rs:894-939
 * semantics; no causal mask; keys ref[0..prefill_len) ++ ring[0..ring_len)):
 * q/out [n_streams][10*128] device pointers. */
int32_t focr_hip_rswa_decode_attention(focr_hip_ctx* ctx, const focr_hip_rswa* cache,
                                       const float* q, float* out);
/* rswa.rs:1184-1200 convenience step: write this token's K/V, then attend. */
int32_t focr_hip_rswa_step(focr_hip_ctx* ctx, focr_hip_rswa* cache, const float* q,
                           const float* k_steps, const float* v_steps, float* out);
/* Chunked prefill of one stream straight into its cache (decoder.rs:
 * 1400-1447 prefill_with_cache_chunked, one layer): the chunk's k / v rows,
 * token-major [cs][10*128] at positions [c0, c0 + cs), are written to the
 * stream's reference block — the reference appends them to its running K/V
 * and seeds the ring from the whole prefix once, which gives the same block
 * — prefill_len becomes c0 + cs and the ring is emptied; then the chunk's
 * queries q_chunk [cs][10*128] attend causally over ref[0 .. c0 + cs)
 * (chunk_prefill_attention) into ctx_out [cs][10*128]. Chunks come in
 * ascending order: c0 is 0 or the stream's current prefill length (E_STATE
 * otherwise); c0 + cs <= ref_capacity (E_STATE). Device pointers. */
int32_t focr_hip_rswa_prefill_chunk(focr_hip_ctx* ctx, focr_hip_rswa* cache, size_t stream,
                                    const float* q_chunk, const float* k_chunk,
                                    const float* v_chunk, size_t cs, size_t c0, float* ctx_out);
/* Cursor reflection / speculative roll-back (rswa.rs:219-283, :524-579). */
int32_t focr_hip_rswa_get_state(const focr_hip_rswa* cache, size_t stream, uint32_t* prefill_len,
                                uint32_t* ring_len, uint32_t* ring_pos);
int32_t focr_hip_rswa_set_state(focr_hip_rswa* cache, size_t stream, uint32_t ring_len,
                                uint32_t ring_pos);
/* Device pointers of one stream's regions (for direct fills/readback). */
int32_t focr_hip_rswa_regions(const focr_hip_rswa* cache, size_t stream, float** ref_k,
                              float** ref_v, float** ring_k, float** ring_v);

/* nn.rs:240-253 rms_norm over rows x [rows, n] f32 -> y (device pointers; w
 * [n] device, nullable): y = (x * rstd) * w, rstd = 1 / sqrt(mean(x^2) + eps)
 * with the sum of squares in f64. n <= 4096. The final norm before the LM
 * head (lm_head_cached_i8, decoder.rs:2275-2296). */
int32_t focr_hip_rms_norm(focr_hip_ctx* ctx, const float* x, size_t rows, size_t n, const float* w,
                          float eps, float* y);

/* ---- one decoder layer's decode step -------------------------------------
 * decoder.rs:2812-2933 batched_decode_step_i8_streams for one layer over every
 * stream of an R-SWA cache (decode_step_with_cache_i8, :2542-2627, per
 * stream): input RMSNorm + quantize_row_i8, the fused qkv GEMV [3 D, hidden],
 * RoPE at each stream's position (RopeTable::build + apply_rope, :150-268),
 * the ring write and decode attention, o_proj [hidden, D], h = x + attn,
 * post-attention RMSNorm, decode_mlp_i8 (:2199-2268: the MoE layer with
 * route_default — norm_topk_prob false, scaling 1.0 — plus its shared expert
 * when one is set, or the dense SwiGLU MLP of layer 0), x = h + mlp.
 * RMSNorm: y = (x * rstd) * w, rstd from the f64 mean of squares + eps.
 * The layer borrows the weight handles (they must outlive it) and copies the
 * two norm weights (host pointers, [hidden]); it also keeps its own device
 * copy of the qkv weights and scales with the q / k rows in RoPE pair order
 * (3 D x hidden bytes), which the qkv GEMV with RoPE in its epilogue reads,
 * and, for the dense MLP, a copy of the gate rows followed by the up rows
 * with their scales (2 x inter x hidden bytes), which the one launch that
 * computes both and silu(gate) * up reads.
 * Exactly one of moe or the three dense handles. D = n_heads * head_dim must
 * be 10 x 128 for the cache. */
int32_t focr_hip_decoder_layer_create(focr_hip_ctx* ctx, size_t hidden, size_t n_heads, size_t head_dim,
                                      const float* input_ln, const float* post_attn_ln,
                                      const focr_hip_qint8* qkv, const focr_hip_qint8* o_proj,
                                      const focr_hip_moe_layer* moe, const focr_hip_qint8* dense_gate,
                                      const focr_hip_qint8* dense_up, const focr_hip_qint8* dense_down,
                                      float rms_eps, float rope_theta, focr_hip_decoder_layer** out);
int32_t focr_hip_decoder_layer_free(focr_hip_decoder_layer* layer);
/* x [n_streams, hidden] f32 device, updated in place; positions [n_streams]
 * host (each stream's absolute position, SPEC-095); route_idx (device,
 * nullable) receives a MoE layer's expert ids [n_streams, top_k]. With
 * check_route = 1 a MoE layer synchronises and returns E_ROUTE for a row with
 * no finite router score. Any number of streams: more than 32 (8 with the
 * 6848-wide dense MLP) run in groups of that many, each the same as alone. */
int32_t focr_hip_decoder_layer_step(focr_hip_ctx* ctx, const focr_hip_decoder_layer* layer,
                                    focr_hip_rswa* cache, const uint32_t* positions, float* x,
                                    uint32_t* route_idx, int32_t check_route);
/* One decoder layer over a prefill chunk of one stream: the per-layer body of
 * prefill_with_cache_i8_chunked (decoder.rs:2428-2520; :2461-2486 for one
 * layer). x [cs, hidden] f32 device holds the chunk's rows (positions c0 ..
 * c0 + cs - 1) and is updated in place: RMSNorm -> q / k / v through
 * linear_int8_dynamic (the dynamic activation rule) -> RoPE at the rows'
 * positions -> K / V into the stream's reference block at [c0, c0 + cs) and
 * the chunk's causal attention over [0, c0 + cs) (focr_hip_rswa_prefill_chunk,
 * which sets the stream's prefill length to c0 + cs, ring empty) -> o_proj ->
 * residual -> RMSNorm -> prefill_mlp_i8 (moe_block_i8: route_default
 * (norm_topk false, scale 1.0) of the chunk's rows, the routed int8 experts
 * and the shared expert on the matrix cores; or the dense expert_mlp_i8) ->
 * residual. Chunks of one stream come in order (c0 = 0, then the previous
 * chunk's end), as rswa_prefill_chunk requires; cs <= 4096. route_idx
 * (device, nullable) receives a MoE layer's expert ids [cs, top_k]; with
 * check_route = 1 a MoE layer synchronises and returns E_ROUTE for a row with
 * no finite router score (the reference's route error). */
int32_t focr_hip_decoder_layer_prefill(focr_hip_ctx* ctx, const focr_hip_decoder_layer* layer,
                                       focr_hip_rswa* cache, size_t stream, float* x, size_t cs,
                                       size_t c0, uint32_t* route_idx, int32_t check_route);

/* ---- the whole batched decode step ----------------------------------------
 * The decode spine of DecoderWeightCacheI8: n_layers layer handles in order
 * (borrowed: they must outlive the decoder), the final RMSNorm weight (host
 * [hidden], copied) and the int8 LM head [vocab, hidden] (borrowed). Every
 * layer has the same hidden size, the MoE layers one top_k. */
int32_t focr_hip_decoder_create(focr_hip_ctx* ctx, size_t n_layers,
                                const focr_hip_decoder_layer* const* layers, const float* final_norm,
                                float rms_eps, const focr_hip_qint8* lm_head, focr_hip_decoder** out);
int32_t focr_hip_decoder_free(focr_hip_decoder* dec);
/* One decode token for every stream, in one call: decoder.rs:2812-2933
 * batched_decode_step_i8 (stream_ids = 0 .. n_streams) through every layer
 * (each as focr_hip_decoder_layer_step), then :2943-2965 batched_lm_head_i8
 * (the final RMSNorm per row, the LM head) and sampler.rs:168-186 argmax_row.
 * caches: n_layers R-SWA caches (layer l's, all with the same n_streams);
 * positions [n_streams] host; x [n_streams, hidden] device: the token
 * embeddings in, the last layer's hidden rows out (what
 * batched_decode_step_i8 returns, before the final norm); logits
 * [n_streams, vocab] device (nullable); tokens [n_streams] u32 device: the
 * argmax per row; route_idx (device, nullable) [n_layers][n_streams][top_k]
 * receives each MoE layer's expert ids (a dense layer's slice untouched).
 * check_route as focr_hip_decoder_layer_step. */
int32_t focr_hip_decoder_step(focr_hip_ctx* ctx, const focr_hip_decoder* dec, focr_hip_rswa* const* caches,
                              const uint32_t* positions, float* x, float* logits, uint32_t* tokens,
                              uint32_t* route_idx, int32_t check_route);
/* The same step with the greedy no-repeat-ngram sampler in the LM-head
 * epilogue instead of the plain argmax: the layers as focr_hip_decoder_step,
 * then the final RMSNorm and focr_hip_lm_head_sample_i8 with these sampler
 * arguments (sampler.rs:426-460 decode_step_premasked per stream,
 * :491-545 batched_decode_step). */
int32_t focr_hip_decoder_step_sample(focr_hip_ctx* ctx, const focr_hip_decoder* dec,
                                     focr_hip_rswa* const* caches, const uint32_t* positions, float* x,
                                     uint32_t* history, size_t history_cap, uint32_t* history_len,
                                     size_t ngram_size, size_t window, const uint32_t* whitelist,
                                     size_t n_whitelist, float temperature, uint32_t eos_token_id,
                                     int32_t append, float* logits, uint32_t* tokens, uint8_t* is_eos,
                                     uint32_t* route_idx, int32_t check_route);
/* The whole prefill of one stream in one call: decoder.rs:2428-2520
 * prefill_with_cache_i8_chunked over the decoder's layers. For each chunk
 * [c0, c1) of prefill_chunk_bounds(seq, chunk), in order, every layer as
 * focr_hip_decoder_layer_prefill (layer l's chunk K / V into caches[l],
 * stream `stream`, starting over at c0 = 0); chunk 0 is the monolithic
 * schedule (the reference's chunk = None); a chunk is at most 4096 rows.
 * x [seq, hidden] device: the input embeddings in, the last layer's hidden
 * rows out (the model.norm-ready hidden the reference returns). With logits
 * [vocab] and / or token [1] (device, nullable) it also takes the first
 * generated token: the final RMSNorm of row seq - 1, the LM head and
 * argmax_row. route_idx (device, nullable) [n_layers][seq][top_k] receives
 * each MoE layer's expert ids (a dense layer's slice untouched); check_route
 * as focr_hip_decoder_layer_prefill (a chunk's row index in the message).
 * seq <= every cache's ref_capacity. */
int32_t focr_hip_decoder_prefill(focr_hip_ctx* ctx, const focr_hip_decoder* dec, focr_hip_rswa* const* caches,
                                 size_t stream, float* x, size_t seq, size_t chunk, float* logits,
                                 uint32_t* token, uint32_t* route_idx, int32_t check_route);

/* ---- weight container: .focrq / safetensors (weights.rs, quant/focrq.rs) --
 * The reader restates weights.rs:443-620 (format detection by magic, the
 * 51-byte .focrq prefix, header JSON, model_id / license / sha checks,
 * validate_directory :949-990) with the reference's FormatMismatch texts
 * (E_FORMAT). A path is memory-mapped read-only; names are byte-sorted. */
int32_t focr_hip_focrq_open(const char* path, focr_hip_focrq** out);          /* weights.rs:416-421 load */
int32_t focr_hip_focrq_from_bytes(const uint8_t* bytes, size_t len,           /* weights.rs:447-453 */
                                  focr_hip_focrq** out);
int32_t focr_hip_focrq_close(focr_hip_focrq* f);
/* is_focrq, arch_target, tensor count, source_sha256 (hex), resolved
 * model_id, license_notice (weights.rs:687-717 getters). Buffers nullable. */
int32_t focr_hip_focrq_info(const focr_hip_focrq* f, int32_t* is_focrq, uint8_t* arch_target,
                            size_t* n_tensors, char* source_sha256, size_t sha_cap, char* model_id,
                            size_t id_cap, char* license, size_t license_cap);
/* The index-th name in sorted order (weights.rs:721-723 names). */
int32_t focr_hip_focrq_name(const focr_hip_focrq* f, size_t index, char* buf, size_t cap);
/* weights.rs:734-736 record(): dtype code (FOCR_HIP_DT_*), shape, ranges. */
int32_t focr_hip_focrq_record(const focr_hip_focrq* f, const char* name, int32_t* dtype,
                              uint64_t* shape, size_t shape_cap, size_t* rank,
                              uint64_t* byte_offset, uint64_t* byte_len, uint64_t* scales_offset,
                              uint64_t* scales_len, uint64_t* group_size, uint8_t* tier);
/* weights.rs:634-670 census: the name set must equal names[0..count). */
int32_t focr_hip_focrq_census(const focr_hip_focrq* f, const char* const* names, size_t count);
/* weights.rs:776-819 mat()/vec(): F32/F16/BF16 widened to f32 on the host
 * (rank 1 reads as [1, len]); out NULL queries rows/cols. */
int32_t focr_hip_focrq_read_f32(const focr_hip_focrq* f, const char* name, float* out, size_t cap,
                                uint64_t* rows, uint64_t* cols);
/* weights.rs:821-862 qint8() / :866-923 qint4(): host copies of the
 * quantized payloads, with the reference's shape checks and messages. */
int32_t focr_hip_focrq_read_qint8(const focr_hip_focrq* f, const char* name, int8_t* w,
                                  size_t w_cap, float* scales, size_t s_cap, uint64_t* n,
                                  uint64_t* k);
int32_t focr_hip_focrq_read_qint4(const focr_hip_focrq* f, const char* name, uint8_t* packed,
                                  size_t p_cap, float* scales, size_t s_cap, uint64_t* n,
                                  uint64_t* k, uint64_t* group_size, uint8_t* tier);

/* Upload once into HBM (DecoderWeightCacheI8::build, decoder.rs:2018-2116).
 * decoder.rs:1777-1786 quant_oc_loaded: a QInt8PerChan record is copied
 * verbatim; an F32/F16/BF16 record is copied raw and quantized per output
 * channel on the device (quant/int8.rs rule). out_channels 0 = the record's
 * rows. */
int32_t focr_hip_focrq_upload_qint8(focr_hip_ctx* ctx, const focr_hip_focrq* f, const char* name,
                                    uint64_t out_channels, focr_hip_qint8** out);
/* weights.rs:776-799 mat() widened on the device into a new device array
 * (*dev, rows*cols f32; release with focr_hip_dfree). */
int32_t focr_hip_focrq_upload_f32(focr_hip_ctx* ctx, const focr_hip_focrq* f, const char* name,
                                  float** dev, uint64_t* rows, uint64_t* cols);
/* decoder.rs:2069-2098: the MoE MLP of model.layers.{layer} — router
 * mlp.gate.weight [n_experts, hidden] (f32), experts mlp.experts.{e}.
 * {gate,up,down}_proj.weight and, with with_shared, mlp.shared_experts.* —
 * as a focr_hip_moe_layer. */
int32_t focr_hip_focrq_moe_layer(focr_hip_ctx* ctx, const focr_hip_focrq* f, size_t layer,
                                 size_t n_experts, size_t top_k, int32_t with_shared,
                                 focr_hip_moe_layer** out);
/* The same experts as QInt4PerGroup records (one group_size for the
 * layer), as the int4 prefill layer. */
int32_t focr_hip_focrq_moe_layer_i4(focr_hip_ctx* ctx, const focr_hip_focrq* f, size_t layer,
                                    size_t n_experts, focr_hip_moe_layer_i4** out);

/* Converter-side weight quantizers on device arrays (src dtype F32/F16/BF16):
 * quant/int8.rs:145-163 quantize_int8_f32 -> q [n,k] + scales [n];
 * quant/int4.rs:142-205 pack_int4_f32 -> packed [n,k/2] + scales
 * [n,k/group] (group 16 or 32; texts of its asserts). Stream-ordered. */
int32_t focr_hip_quantize_weight_i8(focr_hip_ctx* ctx, const void* src, int32_t src_dtype, size_t n,
                                    size_t k, int8_t* q, float* scales);
int32_t focr_hip_pack_weight_i4(focr_hip_ctx* ctx, const void* src, int32_t src_dtype, size_t n,
                                size_t k, size_t group, uint8_t* packed, float* scales);

/* quant/focrq.rs:170-714 FocrqBuilder: tensors emitted sorted by name,
 * canonical header JSON, optional 64-byte payload alignment (align = 1). */
int32_t focr_hip_focrq_writer_new(focr_hip_focrq_writer** out);
int32_t focr_hip_focrq_writer_free(focr_hip_focrq_writer* w);
/* focrq.rs:225-290 with_arch_target / with_source_sha256 (32 bytes,
 * nullable) / with_license_notice (nullable) / with_model_id (nullable) /
 * with_alignment. */
int32_t focr_hip_focrq_writer_set_meta(focr_hip_focrq_writer* w, uint8_t arch_target,
                                       const uint8_t* source_sha256, const char* license_notice,
                                       const char* model_id, int32_t align);
/* focrq.rs:246-270: "provenance" | "model_config" | "packing_manifest". */
int32_t focr_hip_focrq_writer_set_json(focr_hip_focrq_writer* w, const char* field,
                                       const char* json);
int32_t focr_hip_focrq_writer_add_tensor(focr_hip_focrq_writer* w, const char* name, int32_t dtype,
                                         const uint64_t* shape, size_t rank, const void* data,
                                         size_t len); /* focrq.rs:299-313 */
int32_t focr_hip_focrq_writer_add_quantized(focr_hip_focrq_writer* w, const char* name,
                                            int32_t dtype, const uint64_t* shape, size_t rank,
                                            const void* data, size_t len, const float* scales,
                                            size_t n_scales, uint64_t group_size,
                                            uint8_t tier); /* focrq.rs:327-349 */
/* The blob (out NULL: *len only). focrq.rs:479-533 build. */
int32_t focr_hip_focrq_writer_build(const focr_hip_focrq_writer* w, uint8_t* out, size_t cap,
                                    size_t* len);
int32_t focr_hip_focrq_writer_write(const focr_hip_focrq_writer* w, const char* path);

/* ---- profiling (decoder.rs:986-1024 prof counters, GPU-timed) -----------
 * When enabled, every kernel launch carries HIP start/stop events in its
 * dispatch (hipExtLaunchKernelGGL), timing the kernel's own execution;
 * focr_hip_prof_read synchronises and returns, per kernel name, the launch
 * count, total milliseconds and the minimum, median and 90th percentile of
 * the launches (nearest rank, as the reference's bench statistics,
 * benches/support/perf_harness.rs:186-282) as a JSON object. The extra
 * completion signals slow a sequence of launches, so time throughput with it
 * off. */
int32_t focr_hip_prof_enable(focr_hip_ctx* ctx, int32_t on);
int32_t focr_hip_prof_reset(focr_hip_ctx* ctx);
int32_t focr_hip_prof_read(focr_hip_ctx* ctx, char* json, size_t cap);

/* Step marks (no reference counterpart; the GPU form of the per-iteration
 * wall-clock samples of perf_harness.rs:186-263): focr_hip_mark records an
 * event on the context's stream; focr_hip_marks_read synchronises, writes the
 * n - 1 intervals between consecutive marks (ms) into ms[0..cap) and forgets
 * the marks. At most 65536 marks; E_SHAPE when cap is too small. */
int32_t focr_hip_mark(focr_hip_ctx* ctx);
int32_t focr_hip_marks_read(focr_hip_ctx* ctx, float* ms, size_t cap, size_t* n_out);

#ifdef __cplusplus
}
#endif
#endif /* FOCR_HIP_H */
