// focr_internal.hpp — internals shared by the C ABI layer and the gfx950
// kernels: the context, status/error plumbing, scratch buffers, profiling,
// and the host-side launch functions each kernel file exports.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <map>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/focr_hip.h"

namespace focr {

// ---- status / error ------------------------------------------------------
// The calling thread's last error message (focr_hip_last_error).
void set_error(const std::string& msg);
void clear_error();
int32_t fail(int32_t code, const std::string& msg);
// Map a HIP error to FOCR_HIP_E_HIP with "<what>: <hipGetErrorString>".
int32_t hip_fail(hipError_t e, const char* what);

#define FOCR_HIP_TRY(expr, what)                        \
    do {                                                \
        hipError_t e_ = (expr);                         \
        if (e_ != hipSuccess) return focr::hip_fail(e_, what); \
    } while (0)

// ---- scratch buffer slots (grow-only, per context) -----------------------
enum ScratchSlot : int {
    kScrA = 0,  // drop-in tier operand A
    kScrB,      // drop-in tier operand B
    kScrOut,    // drop-in tier output
    kScrAux,    // drop-in tier scales / extra
    kScrXq,     // quantized activation rows
    kScrXs,     // activation scales
    kScrArg,    // argmax partial keys
    kScrLogits, // router logits / probs
    kScrRoute,  // routing indices / gates / permutation tables
    kScrRouteX, // the route's cross-block exchange (zeroed once, never cleared)
    kScrAct,    // MoE SwiGLU activations [pairs][inter]
    kScrY,      // MoE weighted expert outputs [pairs][hidden]
    kScrShared, // shared-expert output [t][hidden]
    kScrRswa,   // attention split-K partials
    kScrI4,     // int4 prefill intermediates
    kScrI4b,
    kScrFlag,   // device status flags
    kScrBan,    // sampler ban bitmaps
    kScrLayer,  // decoder layer step intermediates
    kScrAttn,   // prefill attention key-range partials
    kScrDec,    // decode step: the final-normed rows
    kScrCount
};

// ---- static scratch of the allocation-free entry points ------------------
// One array of this many bytes per GPU, held until the process ends.
constexpr size_t kStaticScratchBytes = size_t(8) << 20;
constexpr unsigned kRouteWaitTicksDefault = 1000;  // 10 us
// profiling: intervals kept per scope name, and step marks per context
constexpr size_t kProfMaxSamples = 1 << 20;
constexpr size_t kMaxMarks = 1 << 16;
// With `device` current, the device address of that GPU's array (resolved
// once per device and cached on success; a failure is returned and not
// cached, so a later call resolves again).
hipError_t static_scratch_init(int device, void** out);
// Orders the calls that share one device's static array: construction makes
// `stream` wait for the previous call's completion event (held under a
// per-device lock until destruction), destruction records this call's.
// Nothing is created or allocated. err() reports a failed wait.
class StaticScratchOrder {
   public:
    StaticScratchOrder(int device, hipStream_t stream);
    ~StaticScratchOrder();
    StaticScratchOrder(const StaticScratchOrder&) = delete;
    StaticScratchOrder& operator=(const StaticScratchOrder&) = delete;
    hipError_t err() const { return err_; }

   private:
    int device_;
    hipStream_t stream_;
    hipEvent_t ev_ = nullptr;  // the device's completion event (null while capturing)
    hipError_t err_ = hipSuccess;
    bool locked_ = false, capturing_ = false;
};

struct ProfPending {
    std::string name;
    hipEvent_t start, stop;
};

}  // namespace focr

struct focr_hip_ctx {
    int device = 0;
    int cu_count = 0;
    std::string arch;
    hipStream_t stream = nullptr;
    std::mutex mu;
    struct Buf {
        void* p = nullptr;
        size_t cap = 0;
    } scratch[focr::kScrCount];
    // this device's static scratch (focr::static_scratch_init), or null with
    // the error that kept it from resolving
    void* static_scratch = nullptr;
    hipError_t static_scratch_err = hipSuccess;
    // bound of the MoE route's cross-block wait (s_memrealtime ticks, 10 ns)
    unsigned route_wait_ticks = focr::kRouteWaitTicksDefault;
    // profiling: per scope name, every drained interval in ms
    bool prof = false;
    std::vector<focr::ProfPending> pending;
    std::map<std::string, std::vector<float>> prof_samples;
    // step marks (focr_hip_mark): events recorded on the stream between steps
    std::vector<hipEvent_t> marks;

    // Grow-only scratch. Returns nullptr (and sets the error) on failure.
    void* scratch_get(int slot, size_t bytes);
    // Make current the device this context lives on.
    hipError_t bind() const { return hipSetDevice(device); }
    hipEvent_t take_event();
};

struct focr_hip_qint8 {
    focr_hip_ctx* ctx = nullptr;
    int8_t* w = nullptr;
    float* scales = nullptr;
    size_t n = 0, k = 0;
    bool owned = false;
    // the weights in the matrix-core fragment order (launch_retile_i8), built
    // the first time the handle is used for prefill; always owned
    mutable int8_t* w_mfma = nullptr;
    // the weights in the large-row GEMM's tiled order (launch_i8_gemm256_retile_b),
    // built the first time the handle multiplies 256 rows or more; always owned
    mutable int8_t* w_tiled = nullptr;
};

struct focr_hip_moe_layer {
    focr_hip_ctx* ctx = nullptr;
    size_t hidden = 0, inter = 0, n_experts = 0, top_k = 0;
    float* router = nullptr;
    int8_t *wg = nullptr, *wu = nullptr, *wd = nullptr;
    float *sg = nullptr, *su = nullptr, *sd = nullptr;
    bool owned = false;
    // shared expert (optional)
    size_t shared_inter = 0;
    int8_t *swg = nullptr, *swu = nullptr, *swd = nullptr;
    float *ssg = nullptr, *ssu = nullptr, *ssd = nullptr;
    bool shared_owned = false;
    // fragment-ordered copies for prefill (launch_retile_i8), built on the
    // first prefill call; always owned
    mutable int8_t *wg_mfma = nullptr, *wu_mfma = nullptr, *wd_mfma = nullptr;
    mutable int8_t *swg_mfma = nullptr, *swu_mfma = nullptr, *swd_mfma = nullptr;
};

// One decoder layer for decode steps (decoder.rs:1971-1982 CachedLayerI8):
// borrowed weight handles, device copies of the two RMSNorm weights and the
// RoPE inverse frequencies.
struct focr_hip_decoder_layer {
    focr_hip_ctx* ctx = nullptr;
    size_t hidden = 0, n_heads = 0, head_dim = 0;
    float eps = 1e-6f;
    float* input_ln = nullptr;   // [hidden]
    float* post_ln = nullptr;    // [hidden]
    float* inv_freq = nullptr;   // [head_dim / 2]
    const focr_hip_qint8* qkv = nullptr;   // [3 * n_heads * head_dim, hidden]
    const focr_hip_qint8* o_proj = nullptr;  // [hidden, n_heads * head_dim]
    const focr_hip_moe_layer* moe = nullptr;  // MoE MLP, or the dense one below
    const focr_hip_qint8 *gate = nullptr, *up = nullptr, *down = nullptr;
    // qkv weights / scales with the q and k rows in RoPE pair order
    // (qkv_rope_row), for the GEMV whose epilogue applies RoPE; owned
    int8_t* qkv_rope_w = nullptr;
    float* qkv_rope_s = nullptr;
    // dense MLP: gate rows then up rows [2 * inter, hidden] and their scales,
    // for the one GEMV launch that computes both; owned
    int8_t* gate_up_w = nullptr;
    float* gate_up_s = nullptr;
};

// decoder.rs DecoderWeightCacheI8 for the decode spine: the layers (borrowed),
// the final RMSNorm weight (owned device copy) and the LM head (borrowed).
struct focr_hip_decoder {
    focr_hip_ctx* ctx = nullptr;
    size_t hidden = 0, top_k = 0;
    float eps = 1e-6f;
    std::vector<const focr_hip_decoder_layer*> layers;
    float* final_norm = nullptr;  // [hidden]
    const focr_hip_qint8* lm_head = nullptr;
};

struct focr_hip_moe_layer_i4 {
    focr_hip_ctx* ctx = nullptr;
    size_t hidden = 0, inter = 0, n_experts = 0, group = 0;
    uint8_t *wg = nullptr, *wu = nullptr, *wd = nullptr;
    float *sg = nullptr, *su = nullptr, *sd = nullptr;
    bool owned = false;
};

struct focr_hip_rswa {
    focr_hip_ctx* ctx = nullptr;
    size_t n_streams = 0, ref_capacity = 0;
    float* base = nullptr;  // one allocation for all regions
    // host cursors (rswa.rs:132-146)
    std::vector<int64_t> prefill_len;  // -1 = never recorded
    std::vector<uint32_t> ring_len, ring_pos;
    size_t stream_floats() const;
    float* ref_k(size_t s) const;
    float* ref_v(size_t s) const;
    float* ring_k(size_t s) const;
    float* ring_v(size_t s) const;
};

namespace focr {

// Profiling: while a ProfScope is open (and ctx->prof is on), the kernels
// launched through FOCR_LAUNCH carry the scope's start/stop events in their
// dispatch (hipExtLaunchKernelGGL), so the recorded interval is the GPU
// execution of those kernels — first kernel's start to last kernel's end —
// without the dispatch gap a separately recorded event would include.
struct LaunchEvents {
    hipEvent_t start = nullptr, stop = nullptr;
    bool first = false, used = false;
};
LaunchEvents& launch_events();  // the calling thread's open scope, if any

struct ProfScope {
    focr_hip_ctx* ctx;
    const char* name;
    hipEvent_t start = nullptr, stop = nullptr;
    ProfScope(focr_hip_ctx* c, const char* n);
    ~ProfScope();
};

#define FOCR_LAUNCH(kernel, grid, block, lds, stream, ...)                                                  \
    do {                                                                                                   \
        focr::LaunchEvents& le_ = focr::launch_events();                                                   \
        if (le_.stop) {                                                                                    \
            hipExtLaunchKernelGGL(kernel, grid, block, lds, stream, le_.first ? le_.start : nullptr, le_.stop, \
                                  0, __VA_ARGS__);                                                          \
            le_.first = false;                                                                             \
            le_.used = true;                                                                               \
        } else {                                                                                           \
            hipLaunchKernelGGL(kernel, grid, block, lds, stream, __VA_ARGS__);                             \
        }                                                                                                  \
    } while (0)

constexpr int kNumHeads = 10;
constexpr int kHeadDim = 128;
constexpr int kRingWindow = 128;

// ---- launch functions (defined in the .hip kernel files) -----------------
// k_igemm.hip: drop-in tier i32 GEMM, out[M,N] += A[M,K] . B[N,K]^T.
hipError_t launch_igemm_i8(hipStream_t s, const void* a, bool a_unsigned, const int8_t* b,
                           int32_t* out, int m, int k, int n);
// batch independent s8s8 products in one launch: instance b reads
// a + b*m*k, b + b*n*k and accumulates into out + b*m*n. Needs k a multiple
// of 16 (<= 65536) and 16-byte aligned a and b.
// k_gemv.hip: the same products on the matrix cores (split-K GEMV, 16 rows
// per pass, out += wrapping); hipErrorNotSupported where the shape does not
// fit (m < 2, k < 64, not a multiple of 64 or > 8192, unaligned operands).
hipError_t launch_igemm_i8_mfma(hipStream_t s, const int8_t* a, const int8_t* b, int32_t* out, int batch, int m,
                                int k, int n);
hipError_t launch_igemm_i8_batched(hipStream_t s, const int8_t* a, const int8_t* b, int32_t* out, int batch, int m,
                                   int k, int n);

// k_gemv.hip
// rule: 0 quantize_row_i8 (half away), 1 quantize_row_i8_te (ties even), 2
// the dynamic activation rule of linear_int8_dynamic (true division, ties even).
constexpr int kQuantRuleDynamic = 2;
hipError_t launch_quantize_rows(hipStream_t s, const float* x, int m, int k, int8_t* xq,
                                float* a_scales, int rule);
// two row sets [m][K] (each row as launch_quantize_rows does it) in one launch
struct QuantRows {
    const float* x;
    int8_t* xq;
    float* scales;
    int m, K;
};
hipError_t launch_quantize_rows2(hipStream_t s, const QuantRows& r1, const QuantRows& r2, int rule);
// y[m,n] = ((f32)acc * a_scales[m]) * ws[n]; acc (nullable) gets raw i32;
// arg_keys (nullable) gets per-block argmax keys [m][nparts].
hipError_t launch_gemv_i8(hipStream_t s, const int8_t* w, const float* ws, int n, int k,
                          const int8_t* xq, const float* a_scales, int m, float* y, int32_t* acc,
                          uint64_t* arg_keys, int* nparts_out, int cu_count);
int gemv_i8_nparts(int n, int cu_count);
// The current device's dynamic-LDS limit per block (160 KB on gfx950).
size_t max_lds_per_block();
// The same GEMV with a per-row ban bitmap (ban_words u32 per row): a set bit
// n writes y[i][n] = -inf and keys see -inf.
// y = dequant(W . quantize_row_i8(x)) for m f32 rows x [m][k] (after
// rms_norm with weight norm_w and eps when norm_w is non-null): for small N
// and k <= 2048 one launch whose blocks quantize the rows themselves;
// otherwise the norm / quantize kernel into xq_tmp [m][k] / xs_tmp [m], then
// the GEMV. Any m >= 1 (rows in groups).
hipError_t launch_gemv_i8_f32(hipStream_t s, const int8_t* w, const float* ws, int n, int k, const float* x,
                              const float* norm_w, float eps, int m, float* y, int8_t* xq_tmp, float* xs_tmp,
                              int cu_count);
// The same (with per-block argmax keys) for m f32 rows x [m][k], quantized
// (quantize_row_i8) inside every block: no separate quantize launch. m = 1:
// k % 16 == 0, k <= 2048; m = 2..16: k % 256 == 0, k <= 1280 (the
// matrix-core form); x 16-byte aligned. hipErrorNotSupported outside those.
hipError_t launch_gemv_i8_f32_keys(hipStream_t s, const int8_t* w, const float* ws, int n, int k, const float* x,
                                   int m, float* y, uint64_t* arg_keys, int* nparts_out, int cu_count);
hipError_t launch_gemv_i8_banned(hipStream_t s, const int8_t* w, const float* ws, int n, int k,
                                 const int8_t* xq, const float* a_scales, int m, float* y, int32_t* acc,
                                 uint64_t* arg_keys, int* nparts_out, int cu_count, const uint32_t* ban_bits,
                                 int ban_words);
// The dense SwiGLU MLP in three launches (decode_layer step, layer 0): act =
// silu(g) * u with [g; u] = dequant(W_gu . quantize_row_i8(rms_norm(x + x2) *
// norm_w)) (W_gu: n gate rows then n up rows, k <= 1280), h = x + x2 written
// to h_out, in one launch; the quantize kernel; y = dequant(W . xq) + resid.
// Each returns hipErrorNotSupported where its shape is outside the one-launch
// form (the caller then runs the separate kernels).
// prefill-sized int8 products (1 <= m <= kRowsMaxM prequantized rows) on the
// split-K GEMV in 16-row groups: y = ((f32)acc * xs) * ws [m][n]; the SwiGLU
// form takes the gate rows then the up rows ([2n][k], scales [2n]) and
// writes act = silu(g) * u [m][n]
constexpr int kRowsMaxM = 256;
bool gemv_rows_supported(int n, int k, int m);
// whether that path is the faster one for the shape (its L2 re-reads grow with
// the block count)
bool gemv_rows_preferred(int n, int k, int m, bool swiglu);
hipError_t launch_gemv_i8_rows(hipStream_t s, const int8_t* w, const float* ws, int n, int k, const int8_t* xq,
                               const float* xs, int m, float* y);
hipError_t launch_swiglu_i8_f32_add(hipStream_t s, const int8_t* w_gu, const float* ws_gu, int n, int k,
                                    const float* x, const float* x2, float* h_out, const float* norm_w, float eps,
                                    int m, float* act, int cu_count);
hipError_t launch_gemv_i8_resid(hipStream_t s, const int8_t* w, const float* ws, int n, int k, const int8_t* xq,
                                const float* a_scales, int m, const float* resid, float* y, int cu_count);
hipError_t launch_argmax_reduce(hipStream_t s, const uint64_t* keys, int m, int nparts,
                                uint32_t* argmax);
// Per-block argmax keys [m][nparts] of a logits matrix (ban_bits nullable).
hipError_t launch_argmax_partial(hipStream_t s, const float* logits, int m, int n, uint64_t* keys, int nparts,
                                 const uint32_t* ban_bits, int ban_words);
hipError_t launch_argmax_rows(hipStream_t s, const float* logits, int m, int n, uint64_t* keys,
                              int nparts, uint32_t* argmax);

// k_moe.hip — decode MoE pipeline (route, gate_up, down + combine; down alone for a shared expert).
struct MoeDims {
    int t, hidden, inter, n_experts, top_k;
};
// route writes idx/gates [t][top_k], flag[t] = 1 when token t has fewer than
// top_k finite router scores, and — when sel is non-null — the routing in the
// layout the expert kernels read (moe_sel_bytes() of device scratch: token
// masks, per-expert slot and gate columns). Nothing is carried between calls.
size_t moe_sel_bytes();
// The decoder layer's residual + post-attention RMSNorm folded into the route
// kernel: it routes rms_norm(hidden + attn) * w and writes hidden + attn to
// h_out (hidden <= 1280).
struct MoeRouteNorm {
    const float* attn;
    const float* w;
    float eps;
    float* h_out;
};
// The route's exchange buffer for t tokens (bytes; zeroed once when
// allocated, then never cleared: calls are told apart by its counter) and
// the route itself (t <= 64 with the selection matrices sel, up to 16384
// without them: a prefill chunk's idx / gates);
// the gate/up launch given the same buffer advances the counter, and a route
// launched without a gate/up after it is followed by launch_route_epoch_bump.
size_t moe_route_xchg_bytes(size_t t);
hipError_t launch_moe_route(hipStream_t s, const MoeDims& d, const float* hidden, const float* router,
                            int norm_topk, float routed_scale, int8_t* xq, float* xs, uint32_t* idx, float* gates,
                            float* probs, int* flag, void* sel, void* xchg, unsigned wait_ticks,
                            const MoeRouteNorm* norm = nullptr);
hipError_t launch_route_epoch_bump(hipStream_t s, void* xchg);
// The many-row route (a prefill chunk, t <= 16384, hidden <= 1280): the split
// route's logits computed eight tokens per router read into logits [t][E],
// then its softmax / top-k per token; no exchange buffer, no quantized rows.
bool moe_route_rows_supported(int hidden);
hipError_t launch_moe_route_rows(hipStream_t s, const MoeDims& d, const float* hidden, const float* router,
                                 int norm_topk, float routed_scale, uint32_t* idx, float* gates, float* probs,
                                 int* flag, float* logits);
// The shared expert's gate/up weights, folded into the routed gate/up launch
// as extra blocks (every token a pair, act rows [t][inter]).
struct MoeSharedGateUp {
    const int8_t *wg, *wu;
    const float *sg, *su;
    float* act;
    int inter;
};
hipError_t launch_moe_gate_up(hipStream_t s, const MoeDims& d, const void* sel, const int8_t* xq, const float* xs,
                              const int8_t* wg, const float* sg, const int8_t* wu, const float* su, float* act,
                              int inter, bool shared, const MoeSharedGateUp* with_shared = nullptr,
                              void* route_xchg = nullptr);
hipError_t launch_moe_down(hipStream_t s, const MoeDims& d, const void* sel, const float* act, const int8_t* wd,
                           const float* sd, float* ybuf, int inter, bool shared);
// out[t] = slot-order sum of ybuf[t*top_k + j] (+ shared_y[t]); zero for a
// token whose flag is set; then resid[t] + that when resid is non-null (the
// decode layer's residual). Follows launch_moe_down over the routed experts.
hipError_t launch_moe_combine(hipStream_t s, const MoeDims& d, const float* ybuf, const int* flag,
                              const float* shared_y, const float* resid, float* out);
// Tokens per step from which the decode layer runs the expert-grouped down
// kernel (each down row read once per step) + combine instead of down +
// combine per token (each down row read once per token that routes to it).
// Measured on MI355X: per token 30.9 / 43.9 / 56.9 us at T = 32 / 48 / 64,
// grouped + combine 31.6 / 37.4 / 42.9 us.
constexpr int kMoeGroupedDownT = 40;
// Tokens per MoE decode call (the route kernel's selection matrices hold 64).
constexpr int kMoeMaxT = 64;
constexpr int kLayerPrefillMaxRows = 4096;  // rows of one decoder_layer_prefill chunk
// down + slot-order combine in one launch, reading the routing from idx /
// gates / flag ([t][top_k]) and the act rows of every pair (t*top_k + j).
hipError_t launch_moe_down_combine(hipStream_t s, const MoeDims& d, const uint32_t* idx, const float* gates,
                                   const int* flag, const float* act, const int8_t* wd, const float* sd,
                                   const float* shared_y, const float* resid, float* out, int inter);
// k_attn.hip — causal prefill attention on the f32 matrix cores (head_dim
// 128). Element (row i, head h) of q / out and (key j, head h) of k / v sit at
// base + i * ld + h * hstride (token-major: ld = heads * 128, hstride = 128).
struct AttnGeom {
    int ldq, hq, ldk, hk, ldv, hv, ldo, ho;
};
// Key ranges for a chunk of cs queries over a c1-key prefix: about two
// blocks per CU, in whole 64-key tiles.
int attn_pick_splits(int cs, int c1, int heads, int cu_count, int* split_len);
size_t attn_partials_bytes(int cs, int heads, int nsplit);
// qo (nullable): where the split merge may write the context rows quantized
// for the next int8 product instead of out (the dynamic rule, row-major or in
// the 256 x 128 GEMM's tiled order); done tells whether it did (a single key
// range writes out in f32, the caller quantizes).
struct AttnQuantOut {
    int8_t* xq;
    float* xs;
    bool tiled;
    bool done;
};
// part: attn_partials_bytes() of scratch when nsplit > 1 (unused otherwise).
hipError_t launch_attn_prefill(hipStream_t s, const AttnGeom& gm, const float* q, const float* k, const float* v,
                               float* out, int cs, int c0, int c1, int heads, int head_dim, int nsplit,
                               int split_len, float* part, AttnQuantOut* qo = nullptr);
// Token-major chunk rows [cs][heads*128] of K and V into head-major
// reference blocks [heads][cap][128] at rows c0 .. c0 + cs - 1.
hipError_t launch_attn_scatter_kv(hipStream_t s, const float* k_chunk, const float* v_chunk, int cs, int heads,
                                  float* ref_k, float* ref_v, int cap, int c0);
// k_layer.hip — the decode layer's ops around the GEMVs / attention / MoE.
// xq, xs = quantize_row_i8(rms_norm(x) * w) per row (n <= 4096).
hipError_t launch_rms_norm_quant(hipStream_t s, const float* x, const float* w, int rows, int n, float eps,
                                 int8_t* xq, float* xs);
// y = rms_norm(x) * w per row (w nullable).
hipError_t launch_rms_norm(hipStream_t s, const float* x, const float* w, int rows, int n, float eps, float* y);
// h = x + a; y = rms_norm(h) * w per row.
hipError_t launch_residual_rms_norm(hipStream_t s, const float* x, const float* a, const float* w, int rows, int n,
                                    float eps, float* h, float* y);
// Split fused qkv rows [streams][3 D] into q, k (RoPE at pos.p[stream]) and v.
struct RopePositions {
    static constexpr int kMax = 32;
    uint32_t p[kMax];
};
// Where the rotated k and the v rows go instead of contiguous k / v: stream
// s's ring slot, head h at k[s] + h * head_stride (the R-SWA ring layout,
// [head][W][head_dim] per stream, k[s] / v[s] already offset to the slot).
struct RopeRing {
    float* k[RopePositions::kMax];
    float* v[RopePositions::kMax];
    size_t head_stride;
};
// The qkv GEMV's RoPE epilogue: the weights' q and k rows are in the pair
// order of qkv_rope_row (each 16-row tile holds 8 (i, i + half) pairs of one
// head), rows >= 2 D in order; q goes to q [rows][D], k and v to the ring
// slots; row i of the launch is stream r0 + i.
struct RopeEpi {
    const float* inv_freq;
    RopePositions pos;
    RopeRing ring;
    float* q;
    int d_model;   // D = n_heads * head_dim
    int head_dim;
    int r0;
};
// Original row of permuted qkv row p (p < 2 D: pairs; else p).
__host__ __device__ inline int qkv_rope_row(int p, int D, int head_dim) {
    if (p >= 2 * D) return p;
    const int part = p / D, pl = p - part * D;
    const int hd = pl / head_dim, pr = pl - hd * head_dim;
    return part * D + hd * head_dim + (pr >> 1) + (pr & 1) * (head_dim >> 1);
}
hipError_t launch_permute_rows_i8(hipStream_t s, const int8_t* w, const float* ws, int n, int k, int D, int head_dim,
                                  int8_t* w_out, float* ws_out);
// qkv = quantized GEMV of the RMSNormed f32 rows (as launch_gemv_i8_f32) with
// RoPE and the q / ring-slot scatter in the epilogue; hipErrorNotSupported
// when the shape does not fit the one-launch form (the caller then runs the
// GEMV and launch_rope_split).
hipError_t launch_qkv_rope_f32(hipStream_t s, const int8_t* w_perm, const float* ws_perm, int n, int k,
                               const float* x, const float* norm_w, float eps, int m, RopeEpi epi, int cu_count);
hipError_t launch_rope_split(hipStream_t s, const float* qkv, const RopePositions& pos, const float* inv_freq,
                             int streams, int n_heads, int head_dim, float* q, float* k, float* v,
                             const RopeRing* ring);
// Prefill rows at positions c0 + r: fused qkv [rows][3 D] -> q [rows][D]
// (RoPE), k (RoPE) and v with element (r, head h, dim d) at
// k / v + r * kv_row_stride + h * kv_head_stride + d (token-major: D,
// head_dim; a head-major reference block at c0: head_dim, capacity *
// head_dim). head_dim a multiple of 8, strides multiples of 4.
hipError_t launch_rope_rows(hipStream_t s, const float* qkv, int rows, int c0, const float* inv_freq, int n_heads,
                            int head_dim, float* q, float* k, float* v, size_t kv_row_stride,
                            size_t kv_head_stride);
hipError_t launch_add_rows(hipStream_t s, const float* a, const float* b, float* out, size_t n);
hipError_t launch_silu_mul(hipStream_t s, const float* g, const float* u, float* act, size_t n);
// k_int4.hip
hipError_t launch_s4s8_packed(hipStream_t s, const int8_t* a, const uint8_t* b,
                              const float* scales, int group, int m, int k, int n, float* out,
                              int32_t* partials);
hipError_t launch_unpack_i4(hipStream_t s, const uint8_t* b, size_t nbytes, int8_t* out);

// k_s4mfma.hip — int4 x int8 GEMMs on the matrix cores and the int4 prefill
// MoE. The drop-in path uses the MFMA kernel when s4_mfma_supported().
bool s4_mfma_supported(int group, int k);
size_t s4_tile_pad_bytes();
hipError_t launch_s4s8_mfma(hipStream_t s, const int8_t* a, const uint8_t* b, const float* scales, int group, int m,
                            int k, int n, float* out);
// Device scratch of one prefill call (t tokens, top_k slots, TK = t*top_k):
// xq [t][H] i8, xs [t], act [TK][I] f32, aq [TK][I] i8, as [TK], ybuf
// [TK][H] f32, plan moe_i4_plan_ints(TK, E) ints, err one int.
struct MoeI4Scratch {
    int8_t* xq;
    float* xs;
    float* act;
    int8_t* aq;
    float* as;
    float* ybuf;
    int* plan;
    int* err;
};
size_t moe_i4_plan_ints(int tk, int n_experts);
// The prefill MoE plan (int4 and int8 layers): a stable counting sort of the
// (token, slot) pairs by expert into 64-row tiles, carved from moe_i4_plan_ints
// ints: perm [tk] (sorted row -> pair id), the tile list (expert, first row,
// rows), each expert's tile count and first tile, the tile count.
constexpr int kMoePlanTileRows = 64;
struct MoePlan {
    int* perm;
    int* tile_e;
    int* tile_r0;
    int* tile_nr;
    int* exp_nt;
    int* exp_t0;
    int* n_tiles;
    int max_tiles;
};
MoePlan moe_plan_view(int* plan, int tk, int n_experts);
// Quantize the t token rows of x by `rule` into xq/xs and build the plan from
// idx [t][top_k]; an expert id >= E sets *err. One launch.
hipError_t launch_moe_prefill_plan(hipStream_t s, const float* x, int t, int H, int rule, int8_t* xq, float* xs,
                                   const uint32_t* idx, int top_k, int E, const MoePlan& p, int* err);
// out[t] = the token's pair rows of ybuf [t*top_k][H] summed in ascending
// expert order (slot order among equal experts), + shared_y[t] if non-null;
// resid non-null: out[t] = resid[t] + that (the layer's residual add).
hipError_t launch_moe_prefill_combine(hipStream_t s, const float* ybuf, const uint32_t* idx, int t, int H,
                                      int top_k, const float* shared_y, float* out, const float* resid = nullptr);
// The int4 layer keeps its experts in the MFMA-tiled layout: b [E][n][k/2]
// packed and sc [E][n][k/group] are copied into b_tiled / s_tiled (same sizes,
// each allocation followed by s4_tile_pad_bytes() of readable padding).
hipError_t launch_retile_i4(hipStream_t s, const uint8_t* b, const float* sc, int n_experts, int n, int k, int group,
                            uint8_t* b_tiled, float* s_tiled);
hipError_t launch_moe_prefill_i4(hipStream_t s, const focr_hip_moe_layer_i4* L, const float* x, int t, int top_k,
                                 const uint32_t* idx, const float* gates, float* out, MoeI4Scratch& w,
                                 focr_hip_ctx* ctx);

// k_i8mfma.hip — int8 x int8 GEMMs on the matrix cores (prefill). K must be
// a multiple of 64. The weights are read in the fragment order that
// launch_retile_i8 writes: for matrix e of [n_mats][N][K], column tile nt =
// n / 32 (N padded to a multiple of 32 with zero columns), 32-byte K step ks,
// half h, column c = n % 32, the 16 bytes k = 32 ks + 16 h + [0, 16) of
// column n sit at 16-byte unit ((e * NT + nt) * KS + ks) * 64 + 32 h + c, so
// a wave's fragment load is 1 KB contiguous.
bool i8_mfma_supported(int k);
size_t i8_tiled_bytes(int n_mats, int n, int k);
hipError_t launch_retile_i8(hipStream_t s, const int8_t* src, int n_mats, int n, int k, int8_t* dst);
// y[m][n] = ((f32)(xq[m] . w[n]) * xs[m]) * ws[n] (+ bias[n]) — nn::linear_int8_dynamic
// on rows already quantized by the dynamic rule; w in fragment order.
hipError_t launch_linear_i8(hipStream_t s, const int8_t* xq, const float* xs, int m, int k, const int8_t* w,
                            const float* ws, int n, const float* bias, float* y);
// k_i8gemm.hip — the same product for large row counts: 256 x 128 block
// tiles, both operands in a tiled order (the activations written so by the
// quantizer, the weights retiled once). Needs m >= 256 and k a multiple of 64.
bool i8_gemm256_supported(int m, int n, int k);
size_t i8_gemm256_a_bytes(int m, int k);  // tiled activation buffer
size_t i8_gemm256_b_bytes(int n, int k);  // tiled weight buffer
hipError_t launch_i8_gemm256_retile_b(hipStream_t s, const int8_t* w, int n, int k, int8_t* wt);
hipError_t launch_quantize_rows_tiled(hipStream_t s, const float* x, int m, int k, int8_t* xt, float* xs, int rule);
// the same after the decoder's RMSNorm of each row (weight nw, k <= 4096)
hipError_t launch_rms_norm_quantize_rows_tiled(hipStream_t s, const float* x, const float* nw, float eps, int m,
                                              int k, int8_t* xt, float* xs, int rule);
hipError_t launch_i8_gemm256(hipStream_t s, const int8_t* xt, const float* xs, int m, int k, const int8_t* wt,
                             const float* ws, int n, const float* bias, float* y);
struct MoeI8Scratch {
    int8_t* xq;       // [t][hidden]
    float* xs;        // [t]
    float* act;       // [t*top_k][inter], sorted-row order
    int8_t* aq;       // [t*top_k][inter]
    float* as;        // [t*top_k]
    float* ybuf;      // [t*top_k][hidden], pair order
    int* plan;        // moe_i4_plan_ints(t*top_k, E)
    int* err;
    float* shared_act;  // with the shared expert: [t][shared_inter]
    int8_t* shared_aq;
    float* shared_as;
    float* shared_y;    // [t][hidden]
};
// moe_block_i8 over the routing idx/gates [t][top_k] (+ the shared expert),
// on the layer's fragment-ordered copies (moe_prefill_i8_prepare); resid
// non-null: out = resid + the block's output (added in the combine).
hipError_t launch_moe_prefill_i8(hipStream_t s, const focr_hip_moe_layer* L, const float* x, int t, int top_k,
                                 const uint32_t* idx, const float* gates, int with_shared, float* out,
                                 MoeI8Scratch& w, focr_hip_ctx* ctx, const float* resid = nullptr);

// k_sampler.hip — greedy decode sampler (sampler.rs): per-row ban bitmaps
// of the sliding-window no-repeat-ngram processor, then token / EOS / history
// append from the argmax keys.
struct SamplerArgs {
    const uint32_t* history;  // [m][cap] token ids
    uint32_t* history_mut;    // same array when appending, else null
    uint32_t* history_len;    // [m] (device)
    int cap;
    int ngram, window;
    const uint32_t* whitelist;
    int n_white;
    int vocab;
    uint32_t* ban_bits;  // [m][ban_words]
    int ban_words;
    int* err;  // [m]: 1 = history_len > cap, 2 = append past cap
};
// One block per row: optionally quantize x row r (decoder.rs:1588-1597) into
// xq/xs, then write row r's ban bitmap.
hipError_t launch_sampler_prep(hipStream_t s, int m, const float* x, int k, int8_t* xq, float* xs,
                               const SamplerArgs& a);
// keys [m][nparts] -> tokens [m], is_eos [m] (nullable), and with
// a.history_mut the token appended to each row's history.
hipError_t launch_sample_finish(hipStream_t s, int m, const uint64_t* keys, int nparts, uint32_t eos,
                                uint32_t* tokens, uint8_t* is_eos, const SamplerArgs& a);

// k_quant.hip — load/convert-time weight conversions. src is a stored
// payload of dtype dt (FOCR_HIP_DT_F32/F16/BF16) in device memory.
hipError_t launch_quant_weight_i8(hipStream_t s, const void* src, int dt, int n, int k, int8_t* q, float* scales);
hipError_t launch_pack_weight_i4(hipStream_t s, const void* src, int dt, int n, int k, int group, uint8_t* packed,
                                 float* scales);
hipError_t launch_widen(hipStream_t s, const void* src, int dt, size_t count, float* dst);

// k_rswa.hip
struct RswaStepArgs {
    static constexpr int kMax = 64;
    uint32_t n;
    uint32_t prefill_len[kMax];
    uint32_t ring_len[kMax];
    uint32_t slot[kMax];
};
hipError_t launch_rswa_write(hipStream_t s, const focr_hip_rswa* c, size_t s0,
                             const RswaStepArgs& a, const float* k_steps, const float* v_steps);
size_t rswa_partials_bytes(size_t n_streams, size_t max_keys);
hipError_t launch_rswa_attention(hipStream_t s, const focr_hip_rswa* c, size_t s0,
                                 const RswaStepArgs& a, const float* q, float* out,
                                 float* partials, int cu_count, focr_hip_ctx* ctx);

}  // namespace focr
