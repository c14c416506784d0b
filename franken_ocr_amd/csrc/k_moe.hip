// k_moe.hip — the MoE decode layer (decoder.rs:2199-2268 decode_mlp_i8 over
// T tokens) as four stream-ordered kernels:
//
//   route    one block per token: router logits as f64 dot products rounded
//            to f32, quantize_row_i8 of the token row, f64 softmax rounded to
//            f32, greedy top-k (= rank by (prob desc, index asc), NaN
//            skipped; moe.rs:209-266), optional renorm and scale
//            (moe.rs:226-236). Writes idx/gates [t][k] and appends each
//            (token, slot) pair to its expert's list in the step plan (an
//            active-expert bitmask plus per-expert pair lists, built with
//            device atomics; the next kernel launch orders the reads).
//   gate_up  grid (active expert, row block): finds its expert with one
//            scalar load of the plan's active mask, issues the expert's gate
//            and up row loads, stages the routed tokens' int8 rows in LDS
//            meanwhile, and writes act[t*K + j][r] = silu(g) * u
//            (decoder.rs:1746-1752).
//   down     grid (active expert, row block): issues the down row loads,
//            re-quantizes each pair's act row into LDS (quantize_row_i8)
//            meanwhile, writes y[t*K + j][r] = dequant * gate
//            (decoder.rs:2244-2246).
//   combine  out[t][c] = ((0 + y[t,0]) + y[t,1]) ... (+ shared), slot order
//            (decoder.rs:2253-2261); deterministic, no atomics. It also
//            clears the plan for the next step.
//
// Each routed expert's 3.44 MB of weights is read exactly once per step, by
// exactly as many blocks as it has row blocks. The order of pairs inside an
// expert's list depends on block timing, but every pair's result is computed
// independently and stored at its own (token, slot) slot, so outputs are
// bit-reproducible run to run. GEMV rows use LPR lanes per row (16 for K =
// 1280 -> 5 chunks of 16 B per lane; 8 for K = 896 -> 7 chunks) and one row
// per lane group: with few pairs per expert the kernels are latency-bound,
// and the smaller register footprint buys the occupancy that hides it.
#include "focr_internal.hpp"
#include "k_common.hpp"

namespace focr {
namespace {

constexpr int kMaxT = 64;
constexpr int kMaxE = 64;
constexpr int kMaxK = 8;
constexpr int kPairStage = 32;  // pairs staged in LDS per pass

struct MoePlan {
    unsigned long long mask;   // bit e: expert e has pairs this step
    int cnt[kMaxE];            // pairs per expert
    int list[kMaxE][kMaxT];    // pair ids t*K + j, per expert
};

template <int LPR>
__device__ __forceinline__ int reduce_lanes(int v) {
#pragma unroll
    for (int o = LPR / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, LPR);
    return v;
}

// Index of the a-th set bit of m (a is block-uniform), or -1.
__device__ __forceinline__ int nth_set_bit(unsigned long long m, int a) {
    for (int i = 0; i < a && m; ++i) m &= m - 1ull;
    return m ? __ffsll(static_cast<long long>(m)) - 1 : -1;
}

// ---- route: one block (16 waves) per token ---------------------------------
constexpr int kRouteThreads = 1024;
constexpr int kRouteWaves = kRouteThreads / 64;

template <int NI>  // float4 chunks of a router row per thread, in batches (H <= 64 * 4 * NI)
__global__ __launch_bounds__(kRouteThreads) void moe_route_kernel(
    const float* __restrict__ x, const float* __restrict__ G, int H, int E, int K, int norm_topk,
    float routed_scale, int8_t* __restrict__ xq, float* __restrict__ xs, uint32_t* __restrict__ idx_out,
    float* __restrict__ gates_out, float* __restrict__ probs_out, int* __restrict__ flag,
    MoePlan* __restrict__ plan) {
    __shared__ float4 s_x[512];
    __shared__ float s_logit[kMaxE];
    __shared__ double s_ex[kMaxE];
    __shared__ float s_p[kMaxE];
    __shared__ int s_sel_e[kMaxK];
    __shared__ float s_sel_w[kMaxK];
    __shared__ float s_red[kRouteWaves];
    const int t = blockIdx.x;
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const float* xr = x + static_cast<size_t>(t) * H;
    const int H4 = H >> 2;
    const float4* x4 = reinterpret_cast<const float4*>(xr);
    for (int c = threadIdx.x; c < H4; c += kRouteThreads) s_x[c] = x4[c];
    __syncthreads();

    // 1. logits: 16 threads per expert; thread (e, l) covers float4 chunks
    //    c = l + 16 i of the router row, NI loads in flight per batch.
    {
        const int e = threadIdx.x >> 4;
        const int l = threadIdx.x & 15;
        double acc = 0.0;
        if (e < E) {
            const float4* gr = reinterpret_cast<const float4*>(G + static_cast<size_t>(e) * H);
#pragma unroll 1
            for (int c0 = l; c0 < H4; c0 += 16 * NI) {
                float4 g[NI];
#pragma unroll
                for (int i = 0; i < NI; ++i) {
                    const int c = c0 + 16 * i;
                    g[i] = c < H4 ? gr[c] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                }
#pragma unroll
                for (int i = 0; i < NI; ++i) {
                    const int c = c0 + 16 * i;
                    const float4 xv = c < H4 ? s_x[c] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                    acc = fma(static_cast<double>(xv.x), static_cast<double>(g[i].x), acc);
                    acc = fma(static_cast<double>(xv.y), static_cast<double>(g[i].y), acc);
                    acc = fma(static_cast<double>(xv.z), static_cast<double>(g[i].z), acc);
                    acc = fma(static_cast<double>(xv.w), static_cast<double>(g[i].w), acc);
                }
            }
        }
#pragma unroll
        for (int o = 8; o > 0; o >>= 1) acc += __shfl_xor(acc, o, 16);
        if (l == 0 && e < E) s_logit[e] = static_cast<float>(acc);
    }

    // 2. quantize_row_i8 of the token row
    float amax = 0.0f;
    for (int i = threadIdx.x; i < H; i += kRouteThreads) amax = fmaxf(amax, fabsf(xr[i]));
    amax = wave_max_f(amax);
    if (lane == 0) s_red[wave] = amax;
    __syncthreads();
    amax = 0.0f;
#pragma unroll
    for (int w = 0; w < kRouteWaves; ++w) amax = fmaxf(amax, s_red[w]);
    const float a_scale = amax > 0.0f ? amax / 127.0f : 1.0f;
    const float inv = 1.0f / a_scale;
    for (int i = threadIdx.x; i < H; i += kRouteThreads)
        xq[static_cast<size_t>(t) * H + i] = quant_i8(xr[i], inv, false);
    if (threadIdx.x == 0) xs[t] = a_scale;

    // 3. softmax in f64 over the f32 logits: max, exp, then a sequential sum
    //    in expert order; each probability rounded to f32.
    const bool valid = wave == 0 && lane < E;
    double ex = 0.0;
    if (valid) {
        double mx = -INFINITY;
        for (int e = 0; e < E; ++e) {
            const double v = static_cast<double>(s_logit[e]);
            mx = v > mx ? v : mx;
        }
        ex = exp(static_cast<double>(s_logit[lane]) - mx);
        s_ex[lane] = ex;
    }
    __syncthreads();
    float p = 0.0f;
    if (valid) {
        double sum = 0.0;
        for (int e = 0; e < E; ++e) sum += s_ex[e];
        p = static_cast<float>(ex / sum);
        s_p[lane] = p;
        if (probs_out) probs_out[static_cast<size_t>(t) * E + lane] = p;
    }
    __syncthreads();
    // 4. greedy top-k == rank by (prob desc, index asc) among non-NaN probs
    int n_valid = 0;
    if (valid) {
        int rank = 0;
        for (int e = 0; e < E; ++e) {
            const float q = s_p[e];
            if (q != q) continue;
            ++n_valid;
            rank += (q > p || (q == p && e < lane)) ? 1 : 0;
        }
        if (p == p && rank < K) {
            s_sel_e[rank] = lane;
            s_sel_w[rank] = p;
        }
    }
    __syncthreads();
    // 5. renormalise (sequential f32 sum in slot order) and scale
    __shared__ float s_denom;
    __shared__ int s_bad;
    if (threadIdx.x == 0) {
        const bool bad = n_valid < K;
        s_bad = bad ? 1 : 0;
        flag[t] = bad ? 1 : 0;
        float s = 0.0f;
        for (int j = 0; j < K; ++j) s += bad ? 0.0f : s_sel_w[j];
        s_denom = s + 1e-20f;
    }
    __syncthreads();
    // 6. publish: one thread per slot (the plan's device atomics run in
    //    parallel rather than as a serial chain of round trips)
    if (threadIdx.x < K) {
        const int j = threadIdx.x;
        const bool bad = s_bad != 0;
        const int e = bad ? 0 : s_sel_e[j];
        float w = bad ? 0.0f : s_sel_w[j];
        if (norm_topk) w = w / s_denom;
        idx_out[t * K + j] = static_cast<uint32_t>(e);
        gates_out[t * K + j] = w * routed_scale;
        if (plan) {
            atomicOr(&plan->mask, 1ull << e);
            const int pos = atomicAdd(&plan->cnt[e], 1);
            if (pos < kMaxT) plan->list[e][pos] = t * K + j;
        }
    }
}

// Expert of this block: routed mode takes the a-th set bit of the plan's
// active mask (one scalar load, so the weight loads can issue right after);
// shared mode is one expert whose pairs are the tokens.
__device__ __forceinline__ int block_expert(const MoePlan* __restrict__ plan, int shared_T) {
    if (shared_T > 0) return 0;
    return nth_set_bit(plan->mask, blockIdx.x);
}

__device__ __forceinline__ int block_pairs(const MoePlan* __restrict__ plan, int e, int shared_T) {
    return shared_T > 0 ? shared_T : min(plan->cnt[e], kMaxT);
}

// Stage the token rows a block needs into LDS: every token row when T fits
// (no dependence on the plan, so these loads start immediately), else the
// rows of the block's pairs [pb, pb + n).
__device__ __forceinline__ void stage_rows(int4* lds, const int8_t* __restrict__ xq, int H, int C, int nrows,
                                          const int* rows) {
    for (int i = threadIdx.x; i < nrows * C; i += 256) {
        const int pp = i / C, c = i - pp * C;
        const int tok = rows ? rows[pp] : pp;
        lds[i] = reinterpret_cast<const int4*>(xq + static_cast<size_t>(tok) * H)[c];
    }
}

constexpr int kAllTok = 32;  // stage every token row when T <= kAllTok

// ---- gate/up ------------------------------------------------------------------
// Block = 256 threads = (256 / LPR) row groups, one weight row per group held
// in registers (2 * JC 16-byte loads in flight per lane); the block's routed
// pairs are then taken one at a time against the staged token rows.
template <int LPR, int JC>
__global__ __launch_bounds__(256) void moe_gate_up_kernel(
    const MoePlan* __restrict__ plan, int T, int K, const int8_t* __restrict__ xq,
    const float* __restrict__ xs, const int8_t* __restrict__ wg, const float* __restrict__ sg,
    const int8_t* __restrict__ wu, const float* __restrict__ su, float* __restrict__ act, int H, int I,
    int shared_T) {
    extern __shared__ int4 lds_x[];  // [rows staged][H/16]
    __shared__ int s_pid[kMaxT];
    __shared__ int s_tok[kMaxT];
    __shared__ float s_xs[kMaxT];
    constexpr int G = 256 / LPR;  // rows per block
    const int e = block_expert(plan, shared_T);
    if (e < 0) return;
    const int grp = threadIdx.x / LPR;
    const int lane = threadIdx.x % LPR;
    const int C = H >> 4;
    const int r = blockIdx.y * G + grp;
    const bool live = r < I;
    const size_t row = static_cast<size_t>(e) * I + (live ? r : 0);
    int4 wgv[JC], wuv[JC];
    {
        const int4* grow = reinterpret_cast<const int4*>(wg + row * H);
        const int4* urow = reinterpret_cast<const int4*>(wu + row * H);
#pragma unroll
        for (int j = 0; j < JC; ++j) {
            const int c = lane + LPR * j;
            wgv[j] = (live && c < C) ? ld_stream(grow + c) : make_int4(0, 0, 0, 0);
            wuv[j] = (live && c < C) ? ld_stream(urow + c) : make_int4(0, 0, 0, 0);
        }
    }
    const float sgr = live ? sg[row] : 0.0f;
    const float sur = live ? su[row] : 0.0f;
    const bool all_tok = T <= kAllTok;
    if (all_tok) stage_rows(lds_x, xq, H, C, T, nullptr);
    if (threadIdx.x < T) s_xs[threadIdx.x] = xs[threadIdx.x];
    const int P = block_pairs(plan, e, shared_T);
    if (threadIdx.x < P) {
        const int pid = shared_T > 0 ? threadIdx.x : plan->list[e][threadIdx.x];
        s_pid[threadIdx.x] = pid;
        s_tok[threadIdx.x] = shared_T > 0 ? pid : pid / K;
    }
    __syncthreads();

    for (int pb = 0; pb < P; pb += kPairStage) {
        const int pc_n = min(kPairStage, P - pb);
        if (!all_tok) {
            if (pb) __syncthreads();
            stage_rows(lds_x, xq, H, C, pc_n, s_tok + pb);
            __syncthreads();
        }
        for (int i = 0; i < pc_n; ++i) {
            const int pp = pb + i;
            const int srow = all_tok ? s_tok[pp] : i;
            int ga = 0, ua = 0;
#pragma unroll
            for (int j = 0; j < JC; ++j) {
                const int c = lane + LPR * j;
                if (c < C) {
                    const int4 xv = lds_x[srow * C + c];
                    ga = dot16_i8(wgv[j], xv, ga);
                    ua = dot16_i8(wuv[j], xv, ua);
                }
            }
            ga = reduce_lanes<LPR>(ga);
            ua = reduce_lanes<LPR>(ua);
            if (live && lane == 0) {
                const float as = s_xs[s_tok[pp]];
                const float g = (static_cast<float>(ga) * as) * sgr;
                const float u = (static_cast<float>(ua) * as) * sur;
                act[static_cast<size_t>(s_pid[pp]) * I + r] = silu_f(g) * u;
            }
        }
    }
}

// ---- down ----------------------------------------------------------------------
constexpr int NQ = 16;  // act values per lane held in registers when a wave quantizes a row

template <int LPR, int JC>
__global__ __launch_bounds__(256) void moe_down_kernel(
    const MoePlan* __restrict__ plan, const float* __restrict__ gates, const float* __restrict__ act,
    const int8_t* __restrict__ wd, const float* __restrict__ sd, float* __restrict__ ybuf, int H, int I,
    int shared_T) {
    extern __shared__ int4 lds_a[];  // [kPairStage][I/16]
    __shared__ float lds_as[kPairStage];
    __shared__ int s_pid[kMaxT];
    constexpr int G = 256 / LPR;
    const int e = block_expert(plan, shared_T);
    if (e < 0) return;
    const int grp = threadIdx.x / LPR;
    const int lane = threadIdx.x % LPR;
    const int wave = threadIdx.x >> 6;
    const int wl = threadIdx.x & 63;
    const int C = I >> 4;
    const int r = blockIdx.y * G + grp;
    const bool live = r < H;
    const size_t row = static_cast<size_t>(e) * H + (live ? r : 0);
    int4 wv[JC];
    {
        const int4* drow = reinterpret_cast<const int4*>(wd + row * I);
#pragma unroll
        for (int j = 0; j < JC; ++j) {
            const int c = lane + LPR * j;
            wv[j] = (live && c < C) ? ld_stream(drow + c) : make_int4(0, 0, 0, 0);
        }
    }
    const float sdr = live ? sd[row] : 0.0f;
    const int P = block_pairs(plan, e, shared_T);
    if (threadIdx.x < P) s_pid[threadIdx.x] = shared_T > 0 ? threadIdx.x : plan->list[e][threadIdx.x];
    __syncthreads();
    int8_t* lds_b = reinterpret_cast<int8_t*>(lds_a);

    for (int pb = 0; pb < P; pb += kPairStage) {
        const int pc_n = min(kPairStage, P - pb);
        if (pb) __syncthreads();
        // quantize_row_i8 of each pair's act row: one wave per pair, the
        // row held in registers (NQ values per lane) between the two passes
        for (int pp = wave; pp < pc_n; pp += 4) {
            const float* ar = act + static_cast<size_t>(s_pid[pb + pp]) * I;
            if (I > 64 * NQ) {  // long rows (a wide shared expert): two passes over L2
                float amax = 0.0f;
                for (int i = wl; i < I; i += 64) amax = fmaxf(amax, fabsf(ar[i]));
                amax = wave_max_f(amax);
                const float a_scale = amax > 0.0f ? amax / 127.0f : 1.0f;
                const float inv = 1.0f / a_scale;
                for (int i = wl; i < I; i += 64) lds_b[pp * I + i] = quant_i8(ar[i], inv, false);
                if (wl == 0) lds_as[pp] = a_scale;
                continue;
            }
            float v[NQ];
#pragma unroll
            for (int q = 0; q < NQ; ++q) v[q] = wl + 64 * q < I ? ar[wl + 64 * q] : 0.0f;
            float amax = 0.0f;
#pragma unroll
            for (int q = 0; q < NQ; ++q) amax = fmaxf(amax, fabsf(v[q]));
            amax = wave_max_f(amax);
            const float a_scale = amax > 0.0f ? amax / 127.0f : 1.0f;
            const float inv = 1.0f / a_scale;
#pragma unroll
            for (int q = 0; q < NQ; ++q)
                if (wl + 64 * q < I) lds_b[pp * I + wl + 64 * q] = quant_i8(v[q], inv, false);
            if (wl == 0) lds_as[pp] = a_scale;
        }
        __syncthreads();
        for (int i = 0; i < pc_n; ++i) {
            int d = 0;
#pragma unroll
            for (int j = 0; j < JC; ++j) {
                const int c = lane + LPR * j;
                if (c < C) d = dot16_i8(wv[j], lds_a[i * C + c], d);
            }
            d = reduce_lanes<LPR>(d);
            if (live && lane == 0) {
                const int pid = s_pid[pb + i];
                const float yv = (static_cast<float>(d) * lds_as[i]) * sdr;
                const float gate = shared_T > 0 ? 1.0f : gates[pid];
                ybuf[static_cast<size_t>(pid) * H + r] = yv * gate;
            }
        }
    }
}

// ---- combine (slot order) ---------------------------------------------------------
__global__ __launch_bounds__(256) void moe_combine_kernel(const float* __restrict__ ybuf,
                                                          const float* __restrict__ shared_y,
                                                          float* __restrict__ out, int H, int K,
                                                          MoePlan* __restrict__ plan, int E) {
    const int t = blockIdx.y;
    const int c = blockIdx.x * 256 + threadIdx.x;
    if (plan && blockIdx.x == 0 && blockIdx.y == 0) {
        // every reader of the plan (gate_up, down) finished before this launch
        if (threadIdx.x < E) plan->cnt[threadIdx.x] = 0;
        if (threadIdx.x == 0) plan->mask = 0ull;
    }
    if (c >= H) return;
    float v[kMaxK];
#pragma unroll
    for (int j = 0; j < kMaxK; ++j) v[j] = j < K ? ybuf[(static_cast<size_t>(t) * K + j) * H + c] : 0.0f;
    const float sh = shared_y ? shared_y[static_cast<size_t>(t) * H + c] : 0.0f;
    float o = 0.0f;
#pragma unroll
    for (int j = 0; j < kMaxK; ++j)
        if (j < K) o += v[j];
    if (shared_y) o += sh;
    out[static_cast<size_t>(t) * H + c] = o;
}

template <int LPR>
hipError_t launch_gate_up_lpr(hipStream_t s, dim3 grid, size_t lds, int JC, const MoePlan* plan, int T, int K,
                              const int8_t* xq, const float* xs, const int8_t* wg, const float* sg,
                              const int8_t* wu, const float* su, float* act, int H, int I, int shared_T) {
#define FOCR_GU(J)                                                                                              \
    case J:                                                                                                     \
        hipLaunchKernelGGL((moe_gate_up_kernel<LPR, J>), grid, dim3(256), lds, s, plan, T, K, xq, xs, wg, sg, wu, \
                           su, act, H, I, shared_T);                                                            \
        break;
    switch (JC) {
        FOCR_GU(1) FOCR_GU(2) FOCR_GU(3) FOCR_GU(4) FOCR_GU(5) FOCR_GU(6) FOCR_GU(7) FOCR_GU(8)
        default:
            return hipErrorInvalidValue;
    }
#undef FOCR_GU
    return hipGetLastError();
}

template <int LPR>
hipError_t launch_down_lpr(hipStream_t s, dim3 grid, size_t lds, int JC, const MoePlan* plan,
                           const float* gates, const float* act, const int8_t* wd, const float* sd, float* ybuf, int H,
                           int I, int shared_T) {
#define FOCR_DN(J)                                                                                                \
    case J:                                                                                                       \
        hipLaunchKernelGGL((moe_down_kernel<LPR, J>), grid, dim3(256), lds, s, plan, gates, act, wd, sd, ybuf, H, I, \
                           shared_T);                                                                             \
        break;
    switch (JC) {
        FOCR_DN(1) FOCR_DN(2) FOCR_DN(3) FOCR_DN(4) FOCR_DN(5) FOCR_DN(6) FOCR_DN(7) FOCR_DN(8)
        default:
            return hipErrorInvalidValue;
    }
#undef FOCR_DN
    return hipGetLastError();
}

// Lanes per row for a K-byte row: 16 when the 16-byte chunk count is a
// multiple of 16 or large (K = 1280: 5 per lane), else 8 (K = 896: 7 per lane).
void pick_lpr(int K, int* lpr, int* jc) {
    const int C = K / 16;
    if (C % 16 == 0 || C > 64) {
        *lpr = 16;
        *jc = (C + 15) / 16;
    } else {
        *lpr = 8;
        *jc = (C + 7) / 8;
    }
}

}  // namespace

size_t moe_plan_bytes() { return sizeof(MoePlan); }

hipError_t launch_moe_route(hipStream_t s, const MoeDims& d, const float* hidden, const float* router,
                            int norm_topk, float routed_scale, int8_t* xq, float* xs, uint32_t* idx, float* gates,
                            float* probs, int* flag, void* plan) {
    if (d.t < 1 || d.t > kMaxT || d.n_experts < 1 || d.n_experts > kMaxE || d.top_k < 1 || d.top_k > kMaxK ||
        d.top_k > d.n_experts || d.hidden % 4 != 0 || d.hidden > 2048)
        return hipErrorInvalidValue;
    MoePlan* pl = static_cast<MoePlan*>(plan);
    hipLaunchKernelGGL((moe_route_kernel<5>), dim3(d.t), dim3(kRouteThreads), 0, s, hidden, router, d.hidden,
                       d.n_experts, d.top_k, norm_topk, routed_scale, xq, xs, idx, gates, probs, flag, pl);
    return hipGetLastError();
}

hipError_t launch_moe_gate_up(hipStream_t s, const MoeDims& d, const void* plan, const int8_t* xq, const float* xs,
                              const int8_t* wg, const float* sg, const int8_t* wu, const float* su, float* act,
                              int inter, bool shared) {
    int lpr, jc;
    pick_lpr(d.hidden, &lpr, &jc);
    if (d.hidden % 16 != 0 || jc > 8) return hipErrorInvalidValue;
    const int rows_per_block = 256 / lpr;
    const int max_active = shared ? 1 : (d.n_experts < d.t * d.top_k ? d.n_experts : d.t * d.top_k);
    const dim3 grid(max_active, (inter + rows_per_block - 1) / rows_per_block);
    const int staged = d.t <= kAllTok ? d.t : kPairStage;
    const size_t lds = static_cast<size_t>(staged) * d.hidden;
    const int sh = shared ? d.t : 0;
    const MoePlan* pl = static_cast<const MoePlan*>(plan);
    if (lpr == 16)
        return launch_gate_up_lpr<16>(s, grid, lds, jc, pl, d.t, d.top_k, xq, xs, wg, sg, wu, su, act,
                                      d.hidden, inter, sh);
    return launch_gate_up_lpr<8>(s, grid, lds, jc, pl, d.t, d.top_k, xq, xs, wg, sg, wu, su, act,
                                 d.hidden, inter, sh);
}

hipError_t launch_moe_down(hipStream_t s, const MoeDims& d, const void* plan, const float* gates, const float* act,
                           const int8_t* wd, const float* sd, float* ybuf, int inter, bool shared) {
    int lpr, jc;
    pick_lpr(inter, &lpr, &jc);
    if (inter % 16 != 0 || jc > 8) return hipErrorInvalidValue;
    const int rows_per_block = 256 / lpr;
    const int max_active = shared ? 1 : (d.n_experts < d.t * d.top_k ? d.n_experts : d.t * d.top_k);
    const dim3 grid(max_active, (d.hidden + rows_per_block - 1) / rows_per_block);
    const size_t lds = static_cast<size_t>(kPairStage) * inter;
    const int sh = shared ? d.t : 0;
    const MoePlan* pl = static_cast<const MoePlan*>(plan);
    if (lpr == 16)
        return launch_down_lpr<16>(s, grid, lds, jc, pl, gates, act, wd, sd, ybuf, d.hidden, inter, sh);
    return launch_down_lpr<8>(s, grid, lds, jc, pl, gates, act, wd, sd, ybuf, d.hidden, inter, sh);
}

hipError_t launch_moe_combine(hipStream_t s, const MoeDims& d, const float* ybuf, const float* shared_y, float* out,
                              void* plan) {
    const dim3 grid((d.hidden + 255) / 256, d.t);
    hipLaunchKernelGGL(moe_combine_kernel, grid, dim3(256), 0, s, ybuf, shared_y, out, d.hidden, d.top_k,
                       static_cast<MoePlan*>(plan), d.n_experts);
    return hipGetLastError();
}

}  // namespace focr
