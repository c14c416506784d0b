// k_moe.hip — the MoE decode layer (decoder.rs:2199-2268 decode_mlp_i8 over
// T tokens) as five stream-ordered kernels:
//
//   router   logits[t][e] = f32(f64 dot(x_t, G_e)); x rows quantized
//            (quantize_row_i8) for the experts in the same launch.
//   topk     per token: f64 softmax -> f32 probs, greedy top-k (strict >,
//            lower index on ties, NaN skipped; moe.rs:209-266), optional
//            renorm and scale (moe.rs:226-236); then the expert-major pair
//            permutation (a counting sort over E buckets, tokens ascending
//            inside an expert, moe.rs:421-429).
//   gate_up  grid (active expert, row block): the expert's gate and up rows
//            streamed once for all of its tokens; epilogue dequant and
//            act = silu(g) * u (decoder.rs:1746-1752).
//   down     grid (active expert, row block): prologue re-quantizes each
//            pair's act row into LDS (quantize_row_i8), then streams the
//            down rows; epilogue y = dequant * gate (decoder.rs:2244-2246).
//   combine  out[t][c] = ((0 + y_slot0) + y_slot1) ... (+ shared), slot
//            order (decoder.rs:2253-2261) — deterministic, no atomics.
//
// Weight bytes dominate: each routed expert's 3.44 MB is read exactly once
// per layer step regardless of how many of the T tokens chose it.
#include "focr_internal.hpp"
#include "k_common.hpp"

namespace focr {
namespace {

constexpr int kThreads = 256;
constexpr int kGroups = kThreads / 16;
constexpr int kMaxT = 64;
constexpr int kMaxE = 64;
constexpr int kMaxK = 8;
constexpr int kMaxPairs = kMaxT * kMaxK;
constexpr int kPairStage = 32;  // pairs staged in LDS per pass
constexpr int kPC = 8;          // pairs accumulated in registers per pass

struct RouteTables {
    int n_active;
    int active_e[kMaxE];
    int offsets[kMaxE + 1];
    int pair_tok[kMaxPairs];
    float pair_gate[kMaxPairs];
    int tok_pair[kMaxPairs];
    // identity table for the shared expert: one "expert", pairs = tokens
    int sh_n_active;
    int sh_active_e[1];
    int sh_offsets[2];
    int sh_pair_tok[kMaxT];
    float sh_pair_gate[kMaxT];
};

struct TableView {
    const int* n_active;
    const int* active_e;
    const int* offsets;
    const int* pair_tok;
    const float* pair_gate;
};

__host__ __device__ inline TableView view(const RouteTables* t, bool shared) {
    if (shared) return {&t->sh_n_active, t->sh_active_e, t->sh_offsets, t->sh_pair_tok, t->sh_pair_gate};
    return {&t->n_active, t->active_e, t->offsets, t->pair_tok, t->pair_gate};
}

// ---- router: logits (f64 dots rounded to f32) + x quantization ------------
__global__ __launch_bounds__(kThreads) void moe_router_kernel(const float* __restrict__ x,
                                                              const float* __restrict__ G,
                                                              float* __restrict__ logits,
                                                              int8_t* __restrict__ xq,
                                                              float* __restrict__ xs, int T,
                                                              int H, int E) {
    __shared__ float red[kThreads / 64];
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int e = blockIdx.x * (kThreads / 64) + wave;
    if (e < E) {
        const float* g = G + static_cast<size_t>(e) * H;
        for (int t = 0; t < T; ++t) {
            const float* xr = x + static_cast<size_t>(t) * H;
            double acc = 0.0;
            for (int i = lane; i < H; i += 64) acc = fma(static_cast<double>(xr[i]), static_cast<double>(g[i]), acc);
            acc = wave_sum_d(acc);
            if (lane == 0) logits[static_cast<size_t>(t) * E + e] = static_cast<float>(acc);
        }
    }
    // quantize_row_i8 of the token rows (block-strided over tokens)
    for (int t = blockIdx.x; t < T; t += gridDim.x) {
        const float* xr = x + static_cast<size_t>(t) * H;
        float amax = 0.0f;
        for (int i = threadIdx.x; i < H; i += kThreads) amax = fmaxf(amax, fabsf(xr[i]));
        amax = wave_max_f(amax);
        __syncthreads();
        if (lane == 0) red[wave] = amax;
        __syncthreads();
        amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
        const float a_scale = amax > 0.0f ? amax / 127.0f : 1.0f;
        const float inv = 1.0f / a_scale;
        int8_t* q = xq + static_cast<size_t>(t) * H;
        for (int i = threadIdx.x; i < H; i += kThreads) q[i] = quant_i8(xr[i], inv, false);
        if (threadIdx.x == 0) xs[t] = a_scale;
    }
}

// ---- top-k + permutation (one block) --------------------------------------
__global__ __launch_bounds__(kThreads) void moe_topk_kernel(const float* __restrict__ logits, int T,
                                                            int E, int K, int norm_topk,
                                                            float routed_scale,
                                                            uint32_t* __restrict__ idx_out,
                                                            float* __restrict__ gates_out,
                                                            float* __restrict__ probs_out,
                                                            RouteTables* __restrict__ tb,
                                                            int* __restrict__ flag) {
    __shared__ int s_idx[kMaxPairs];
    __shared__ float s_w[kMaxPairs];
    __shared__ int s_cnt[kMaxE];
    __shared__ int s_base[kMaxE];
    __shared__ int s_bad;
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    if (threadIdx.x == 0) s_bad = 0;
    __syncthreads();
    for (int t = wave; t < T; t += kThreads / 64) {
        const bool valid = lane < E;
        const float lg = valid ? logits[static_cast<size_t>(t) * E + lane] : 0.0f;
        // softmax in f64 over the f32 logits, each probability rounded to f32
        const double mx = wave_max_d(valid && lg == lg ? static_cast<double>(lg) : -INFINITY);
        const double ex = valid ? exp(static_cast<double>(lg) - mx) : 0.0;
        const double sum = wave_sum_d(ex);
        const float p = valid ? static_cast<float>(ex / sum) : 0.0f;
        if (probs_out && valid) probs_out[static_cast<size_t>(t) * E + lane] = p;
        bool taken = false;
        float wsel[kMaxK];
        int esel[kMaxK];
        for (int slot = 0; slot < K; ++slot) {
            const uint64_t key = (valid && !taken) ? argmax_key(p, static_cast<uint32_t>(lane)) : 0ull;
            const uint64_t best = wave_max_u64(key);
            int e = 0;
            float w = 0.0f;
            if (best == 0ull) {
                if (lane == 0) s_bad = 1;
            } else {
                e = static_cast<int>(argmax_key_index(best));
                w = __shfl(p, e, 64);
            }
            if (lane == e && best != 0ull) taken = true;
            wsel[slot] = w;
            esel[slot] = e;
        }
        if (lane == 0) {
            if (norm_topk) {
                float s = 0.0f;
                for (int j = 0; j < K; ++j) s += wsel[j];
                const float denom = s + 1e-20f;
                for (int j = 0; j < K; ++j) wsel[j] = wsel[j] / denom;
            }
            for (int j = 0; j < K; ++j) {
                const float w = wsel[j] * routed_scale;
                s_idx[t * K + j] = esel[j];
                s_w[t * K + j] = w;
                if (idx_out) idx_out[t * K + j] = static_cast<uint32_t>(esel[j]);
                if (gates_out) gates_out[t * K + j] = w;
            }
        }
    }
    __syncthreads();
    // counting sort: thread e lists its pairs in token order
    if (threadIdx.x < E) {
        const int e = threadIdx.x;
        int c = 0;
        for (int i = 0; i < T * K; ++i) c += (s_idx[i] == e);
        s_cnt[e] = c;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        int off = 0, na = 0;
        for (int e = 0; e < E; ++e) {
            s_base[e] = off;
            if (s_cnt[e] > 0) {
                tb->active_e[na] = e;
                tb->offsets[na] = off;
                ++na;
            }
            off += s_cnt[e];
        }
        tb->offsets[na] = off;
        tb->n_active = na;
        tb->sh_n_active = 1;
        tb->sh_active_e[0] = 0;
        tb->sh_offsets[0] = 0;
        tb->sh_offsets[1] = T;
        if (flag) *flag = s_bad;
    }
    __syncthreads();
    if (threadIdx.x < E) {
        const int e = threadIdx.x;
        int p = s_base[e];
        for (int i = 0; i < T * K; ++i) {
            if (s_idx[i] == e) {
                tb->pair_tok[p] = i / K;
                tb->pair_gate[p] = s_w[i];
                tb->tok_pair[i] = p;
                ++p;
            }
        }
    }
    for (int t = threadIdx.x; t < T; t += kThreads) {
        tb->sh_pair_tok[t] = t;
        tb->sh_pair_gate[t] = 1.0f;
    }
}

// ---- gate/up: act[p][r] = silu(g) * u --------------------------------------
// Block = (active expert a, row block). 16 lanes per row; each lane holds its
// gate-row and up-row chunks in registers and reuses them for every pair.
template <int JB>
__global__ __launch_bounds__(kThreads) void moe_gate_up_kernel(
    const RouteTables* __restrict__ tb, int shared_mode, const int8_t* __restrict__ xq,
    const float* __restrict__ xs, const int8_t* __restrict__ wg, const float* __restrict__ sg,
    const int8_t* __restrict__ wu, const float* __restrict__ su, float* __restrict__ act, int H,
    int I, int rows_per_block) {
    extern __shared__ int4 lds_x[];  // [kPairStage][H/16]
    const TableView tv = view(tb, shared_mode != 0);
    const int a = blockIdx.x;
    if (a >= *tv.n_active) return;
    const int e = tv.active_e[a];
    const int p0 = tv.offsets[a];
    const int P = tv.offsets[a + 1] - p0;
    const int group = threadIdx.x >> 4;
    const int lane = threadIdx.x & 15;
    const int C = H >> 4;
    const int r_begin = blockIdx.y * rows_per_block;
    const int r_end = min(r_begin + rows_per_block, I);
    const int8_t* wg_e = wg + static_cast<size_t>(e) * I * H;
    const int8_t* wu_e = wu + static_cast<size_t>(e) * I * H;

    for (int pb = 0; pb < P; pb += kPairStage) {
        const int pc_n = min(kPairStage, P - pb);
        __syncthreads();
        for (int i = threadIdx.x; i < pc_n * C; i += kThreads) {
            const int pp = i / C, c = i - pp * C;
            const int tok = tv.pair_tok[p0 + pb + pp];
            lds_x[i] = reinterpret_cast<const int4*>(xq + static_cast<size_t>(tok) * H)[c];
        }
        __syncthreads();
        for (int r0 = r_begin; r0 < r_end; r0 += kGroups) {
            const int r = r0 + group;
            const bool live = r < r_end;
            int4 wgv[JB], wuv[JB];
            const int4* grow = reinterpret_cast<const int4*>(wg_e + static_cast<size_t>(live ? r : r_begin) * H);
            const int4* urow = reinterpret_cast<const int4*>(wu_e + static_cast<size_t>(live ? r : r_begin) * H);
#pragma unroll
            for (int j = 0; j < JB; ++j) {
                const int c = lane + 16 * j;
                wgv[j] = (live && c < C) ? grow[c] : make_int4(0, 0, 0, 0);
                wuv[j] = (live && c < C) ? urow[c] : make_int4(0, 0, 0, 0);
            }
            const float sgr = live ? sg[static_cast<size_t>(e) * I + r] : 0.0f;
            const float sur = live ? su[static_cast<size_t>(e) * I + r] : 0.0f;
            for (int q0 = 0; q0 < pc_n; q0 += kPC) {
                int ga[kPC], ua[kPC];
#pragma unroll
                for (int i = 0; i < kPC; ++i) ga[i] = ua[i] = 0;
#pragma unroll
                for (int j = 0; j < JB; ++j) {
                    const int c = lane + 16 * j;
                    if (c < C) {
#pragma unroll
                        for (int i = 0; i < kPC; ++i) {
                            if (q0 + i < pc_n) {
                                const int4 xv = lds_x[(q0 + i) * C + c];
                                ga[i] = dot16_i8(wgv[j], xv, ga[i]);
                                ua[i] = dot16_i8(wuv[j], xv, ua[i]);
                            }
                        }
                    }
                }
#pragma unroll
                for (int i = 0; i < kPC; ++i) {
                    const int gv = reduce16_add(ga[i]);
                    const int uv = reduce16_add(ua[i]);
                    if (live && lane == i && q0 + i < pc_n) {
                        const int p = p0 + pb + q0 + i;
                        const float as = xs[tv.pair_tok[p]];
                        const float g = (static_cast<float>(gv) * as) * sgr;
                        const float u = (static_cast<float>(uv) * as) * sur;
                        act[static_cast<size_t>(p) * I + r] = silu_f(g) * u;
                    }
                }
            }
        }
    }
}

// ---- down: ybuf[p][r] = dequant(Wd[e][r] . q(act[p])) * gate[p] ------------
template <int JB>
__global__ __launch_bounds__(kThreads) void moe_down_kernel(
    const RouteTables* __restrict__ tb, int shared_mode, const float* __restrict__ act,
    const int8_t* __restrict__ wd, const float* __restrict__ sd, float* __restrict__ ybuf, int H,
    int I, int rows_per_block) {
    extern __shared__ int4 lds_a[];  // [kPairStage][I/16]
    __shared__ float lds_as[kPairStage];
    const TableView tv = view(tb, shared_mode != 0);
    const int a = blockIdx.x;
    if (a >= *tv.n_active) return;
    const int e = tv.active_e[a];
    const int p0 = tv.offsets[a];
    const int P = tv.offsets[a + 1] - p0;
    const int group = threadIdx.x >> 4;
    const int lane = threadIdx.x & 15;
    const int wave = threadIdx.x >> 6;
    const int wl = threadIdx.x & 63;
    const int C = I >> 4;
    const int r_begin = blockIdx.y * rows_per_block;
    const int r_end = min(r_begin + rows_per_block, H);
    const int8_t* wd_e = wd + static_cast<size_t>(e) * H * I;
    int8_t* lds_b = reinterpret_cast<int8_t*>(lds_a);

    for (int pb = 0; pb < P; pb += kPairStage) {
        const int pc_n = min(kPairStage, P - pb);
        __syncthreads();
        // quantize_row_i8 of each pair's act row: one wave per pair
        for (int pp = wave; pp < pc_n; pp += kThreads / 64) {
            const float* ar = act + static_cast<size_t>(p0 + pb + pp) * I;
            float amax = 0.0f;
            for (int i = wl; i < I; i += 64) amax = fmaxf(amax, fabsf(ar[i]));
            amax = wave_max_f(amax);
            const float a_scale = amax > 0.0f ? amax / 127.0f : 1.0f;
            const float inv = 1.0f / a_scale;
            for (int i = wl; i < I; i += 64) lds_b[pp * I + i] = quant_i8(ar[i], inv, false);
            if (wl == 0) lds_as[pp] = a_scale;
        }
        __syncthreads();
        for (int r0 = r_begin; r0 < r_end; r0 += kGroups) {
            const int r = r0 + group;
            const bool live = r < r_end;
            int4 wv[JB];
            const int4* drow = reinterpret_cast<const int4*>(wd_e + static_cast<size_t>(live ? r : r_begin) * I);
#pragma unroll
            for (int j = 0; j < JB; ++j) {
                const int c = lane + 16 * j;
                wv[j] = (live && c < C) ? drow[c] : make_int4(0, 0, 0, 0);
            }
            const float sdr = live ? sd[static_cast<size_t>(e) * H + r] : 0.0f;
            for (int q0 = 0; q0 < pc_n; q0 += kPC) {
                int da[kPC];
#pragma unroll
                for (int i = 0; i < kPC; ++i) da[i] = 0;
#pragma unroll
                for (int j = 0; j < JB; ++j) {
                    const int c = lane + 16 * j;
                    if (c < C) {
#pragma unroll
                        for (int i = 0; i < kPC; ++i)
                            if (q0 + i < pc_n) da[i] = dot16_i8(wv[j], lds_a[(q0 + i) * C + c], da[i]);
                    }
                }
#pragma unroll
                for (int i = 0; i < kPC; ++i) {
                    const int dv = reduce16_add(da[i]);
                    if (live && lane == i && q0 + i < pc_n) {
                        const int p = p0 + pb + q0 + i;
                        const float yv = (static_cast<float>(dv) * lds_as[q0 + i]) * sdr;
                        ybuf[static_cast<size_t>(p) * H + r] = yv * tv.pair_gate[p];
                    }
                }
            }
        }
    }
}

// ---- combine (slot order) ---------------------------------------------------
__global__ __launch_bounds__(kThreads) void moe_combine_kernel(const RouteTables* __restrict__ tb,
                                                               const float* __restrict__ ybuf,
                                                               const float* __restrict__ shared_y,
                                                               float* __restrict__ out, int H,
                                                               int K) {
    const int t = blockIdx.y;
    const int c = blockIdx.x * kThreads + threadIdx.x;
    if (c >= H) return;
    float o = 0.0f;
    for (int j = 0; j < K; ++j) o += ybuf[static_cast<size_t>(tb->tok_pair[t * K + j]) * H + c];
    if (shared_y) o += shared_y[static_cast<size_t>(t) * H + c];
    out[static_cast<size_t>(t) * H + c] = o;
}

constexpr int kGateUpRows = 32;
constexpr int kDownRows = 64;

}  // namespace

size_t moe_route_table_bytes(const MoeDims&) { return sizeof(RouteTables); }

hipError_t launch_moe_router(hipStream_t s, const MoeDims& d, const float* hidden,
                             const float* router, float* logits, int8_t* xq, float* xs) {
    if (d.t < 1 || d.t > kMaxT || d.n_experts < 1 || d.n_experts > kMaxE) return hipErrorInvalidValue;
    const int grid = (d.n_experts + 3) / 4;
    hipLaunchKernelGGL(moe_router_kernel, dim3(grid), dim3(kThreads), 0, s, hidden, router, logits,
                       xq, xs, d.t, d.hidden, d.n_experts);
    return hipGetLastError();
}

hipError_t launch_moe_topk(hipStream_t s, const MoeDims& d, const float* logits, int norm_topk,
                           float routed_scale, uint32_t* idx, float* gates, float* probs,
                           void* tables, int* flag) {
    if (d.top_k < 1 || d.top_k > kMaxK || d.top_k > d.n_experts) return hipErrorInvalidValue;
    hipLaunchKernelGGL(moe_topk_kernel, dim3(1), dim3(kThreads), 0, s, logits, d.t, d.n_experts,
                       d.top_k, norm_topk, routed_scale, idx, gates, probs,
                       static_cast<RouteTables*>(tables), flag);
    return hipGetLastError();
}

hipError_t launch_moe_gate_up(hipStream_t s, const MoeDims& d, const void* tables,
                              const int8_t* xq, const float* xs, const int8_t* wg,
                              const float* sg, const int8_t* wu, const float* su, float* act,
                              int inter, int max_active, bool shared) {
    if (d.hidden % 16 != 0 || d.hidden > 16 * 16 * 8) return hipErrorInvalidValue;
    const dim3 grid(max_active, (inter + kGateUpRows - 1) / kGateUpRows);
    const size_t lds = static_cast<size_t>(kPairStage) * d.hidden;
    hipLaunchKernelGGL(moe_gate_up_kernel<8>, grid, dim3(kThreads), lds, s,
                       static_cast<const RouteTables*>(tables), shared ? 1 : 0, xq, xs, wg, sg, wu,
                       su, act, d.hidden, inter, kGateUpRows);
    return hipGetLastError();
}

hipError_t launch_moe_down(hipStream_t s, const MoeDims& d, const void* tables, const float* act,
                           const int8_t* wd, const float* sd, const float*, float* ybuf, int inter,
                           int max_active, bool shared) {
    if (inter % 16 != 0 || inter > 16 * 16 * 8) return hipErrorInvalidValue;
    const dim3 grid(max_active, (d.hidden + kDownRows - 1) / kDownRows);
    const size_t lds = static_cast<size_t>(kPairStage) * inter;
    hipLaunchKernelGGL(moe_down_kernel<8>, grid, dim3(kThreads), lds, s,
                       static_cast<const RouteTables*>(tables), shared ? 1 : 0, act, wd, sd, ybuf,
                       d.hidden, inter, kDownRows);
    return hipGetLastError();
}

hipError_t launch_moe_combine(hipStream_t s, const MoeDims& d, const void* tables,
                              const float* ybuf, const float* shared_y, float* out) {
    const dim3 grid((d.hidden + kThreads - 1) / kThreads, d.t);
    hipLaunchKernelGGL(moe_combine_kernel, grid, dim3(kThreads), 0, s,
                       static_cast<const RouteTables*>(tables), ybuf, shared_y, out, d.hidden,
                       d.top_k);
    return hipGetLastError();
}

}  // namespace focr
