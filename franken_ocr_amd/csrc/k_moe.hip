// k_moe.hip — the MoE decode layer (decoder.rs:2199-2268 decode_mlp_i8 over
// T tokens) as four stream-ordered kernels:
//
//   route    eight blocks per token on one XCD (below): router logits as f64
//            dot products rounded to f32, quantize_row_i8 of the token row,
//            f64 softmax rounded to f32, greedy top-k (= rank by (prob desc,
//            index asc), NaN skipped; moe.rs:209-266), optional renorm and
//            scale (moe.rs:226-236). Writes idx/gates [t][k] and the
//            selection matrices slot[e][t] / gate[e][t]; no atomics; the only
//            state between calls is the logit exchange's tag counter.
//   gate_up  grid (active-expert slot a, row block): one ballot over the
//            experts' slot rows gives the active set and the a-th expert;
//            issues the expert's gate and up row loads, stages the token rows
//            in LDS, takes its (token, slot) pairs from column e of the slot
//            matrix in token order; writes act[t*K + j][r] = silu(g) * u
//            (decoder.rs:1746-1752).
//   down     grid (active-expert slot a, row block): issues the down row
//            loads, collects the pairs the same way, re-quantizes each pair's
//            act row into LDS (quantize_row_i8), writes y[t*K + j][r] =
//            dequant * gate (decoder.rs:2244-2246).
//   combine  out[t][c] = ((0 + y[t,0]) + y[t,1]) ... (+ shared), slot order
//            (decoder.rs:2253-2261); deterministic, no atomics.
//
// Each routed expert's 3.44 MB of weights is read exactly once per step, by
// exactly as many blocks as it has row blocks. Every pair's result is
// computed independently and stored at its own (token, slot) slot, so
// outputs are bit-reproducible run to run. GEMV rows use LPR lanes per row
// (16 for K = 1280 -> 5 chunks of 16 B per lane; 8 for K = 896 -> 7 chunks)
// and one row per lane group: with few pairs per expert the kernels are
// latency-bound, and the smaller register footprint buys the occupancy that
// hides it.
#include "focr_internal.hpp"
#include "k_common.hpp"

namespace focr {
namespace {

constexpr int kMaxT = 64;
constexpr int kMaxE = 64;
constexpr int kMaxK = 8;
constexpr int kPairStage = 32;  // pairs staged in LDS per pass

// The step's routing in the layout the expert kernels consume, written by
// route without atomics: slot[e][t] = 1 + the slot j at which token t chose
// expert e, 0 if it did not (every entry is written each call: the token's
// block writes column t for e < E, block 0 zeroes the rest); gate[e][t] =
// that pair's gate (valid where slot != 0).
struct MoeSel {
    uint8_t* slot;  // [kMaxE][kMaxT]
    float* gate;    // [kMaxE][kMaxT]
};


// Index of the a-th set bit of m (a is block-uniform), or -1.
__device__ __forceinline__ int nth_set_bit(unsigned long long m, int a) {
    for (int i = 0; i < a && m; ++i) m &= m - 1ull;
    return m ? __ffsll(static_cast<long long>(m)) - 1 : -1;
}

// ---- route: kRouteParts blocks per token, on one XCD -----------------------
// Pulling the whole 327 KB router through one CU takes ~4.8 us (the per-CU
// load path, not HBM), so each token's router rows are split over
// kRouteParts blocks of kRouteThreads threads: part p computes the logits of
// experts [p*EP, (p+1)*EP), EP = ceil(E / kRouteParts). The parts of a token
// are placed on one XCD (workgroups go to the 8 XCDs round-robin, block b to
// XCD b % 8), so they share that XCD's L2. Each part publishes its logits as
// 8-byte words (f32 logit bits | the call's 32-bit tag << 32), one aligned
// store each, so a word is either the old one or the new one; part 0 (the
// leader) polls them with agent-scope loads (sc1: past the CU's L1, which
// would otherwise serve a stale line on every poll after the first; a
// workgroup-scope sc0 load did not see half of them) and gets the logit
// with its tag. No atomic read-modify-writes, no fences. The wait is
// bounded by the real-time clock: a part whose words have not all appeared
// after wait_ticks (s_memrealtime runs at 100 MHz; 1000 = 10 us by default)
// is computed by the leader itself, so the result
// never depends on the placement or on the other blocks being resident.
// Either way each logit is the same f64 dot product in the same lane order
// (lane l: float4 chunks l + 64 i, then the DPP tree), so the routing is
// that of one block doing it all.
//
// Tags: a call's tag is the low 32 bits of 2 * counter + 1, counter = the
// exchange buffer's header word, read by every block at its start and
// advanced by the next kernel of the call (route_epoch_bump / the gate/up
// kernel), so no word of an earlier call (or of the zeroed buffer) matches.
// A graph that replays the call replays the bump too.
//
// Per-phase timestamps (s_memrealtime, one T = 8 step, from the first
// block's start): blocks start over 0 - 1.4 us, the parts' dots end by
// ~2.8 us; publishing before the token row's quantize and without a store
// acknowledgement wait, and the softmax, rank and renorm in one wave with
// cross-lane reads, keep the leader's tail short.
constexpr int kRouteParts = 8;
constexpr int kRouteThreads = 256;
constexpr int kRouteWaves = kRouteThreads / 64;
constexpr int kRouteRPW = 2;   // router rows per wave: kRouteWaves x 2 = 8 = E / kRouteParts at E = 64
constexpr int kRouteNC = 5;    // float4 chunks per lane per batch: 64 x 5 x 4 = 1280 floats
constexpr int kRouteEPP = kRouteWaves * kRouteRPW;  // experts per part (max)
static_assert(kRouteEPP * kRouteParts >= kMaxE, "the parts cover every expert");
static_assert(kRouteRPW == 2, "route_dots results are taken as d[0] / d[1]");

// The exchange buffer: this header, then the words [T][kRouteParts][kRouteEPP]
// (logit bits | tag << 32) of a call over T tokens.
struct RouteXchg {
    unsigned long long counter;  // advanced once per call, after the route kernel
    unsigned long long pad[15];
};
__device__ __forceinline__ unsigned long long* route_word(RouteXchg* x, int t, int part, int i) {
    return reinterpret_cast<unsigned long long*>(x + 1) + (static_cast<size_t>(t) * kRouteParts + part) * kRouteEPP + i;
}
constexpr int kRouteMaxT = 16384;  // tokens of one route call without the selection matrices (prefill)

struct RouteNorm {
    const float* attn;  // [T][H]
    const float* w;     // [H]
    float eps;
    float* h_out;       // [T][H]
};

__device__ __forceinline__ unsigned long long realtime() { return __builtin_amdgcn_s_memrealtime(); }

// The f64 logits of router rows r[0..kRouteRPW) (clamped in range by the
// caller) against the routed row, in this wave: lane l owns float4 chunks
// l + 64 i; every load of a batch is issued before its first use. Returns
// the wave sums (every lane) and max|row| over the wave.
template <bool NORM>
__device__ __forceinline__ void route_dots(const float4* __restrict__ xr, const float4 (&nv)[kRouteNC],
                                           const float* __restrict__ G, const int (&r)[kRouteRPW], int H4,
                                           int lane, double (&out)[kRouteRPW], float& amax_out) {
    const float4* gr[kRouteRPW];
#pragma unroll
    for (int k = 0; k < kRouteRPW; ++k) gr[k] = reinterpret_cast<const float4*>(G + static_cast<size_t>(r[k]) * H4 * 4);
    auto masked = [](float4 v, unsigned m) {
        return make_float4(__uint_as_float(__float_as_uint(v.x) & m), __uint_as_float(__float_as_uint(v.y) & m),
                           __uint_as_float(__float_as_uint(v.z) & m), __uint_as_float(__float_as_uint(v.w) & m));
    };
    double acc[kRouteRPW];
#pragma unroll
    for (int k = 0; k < kRouteRPW; ++k) acc[k] = 0.0;
    float amax = 0.0f;
#pragma unroll 1
    for (int c0 = lane; c0 < H4 + lane; c0 += 64 * kRouteNC) {
        float4 xv[kRouteNC];
        float4 gv[kRouteRPW][kRouteNC];
        unsigned m[kRouteNC];
#pragma unroll
        for (int i = 0; i < kRouteNC; ++i) {
            const int c = c0 + 64 * i;
            m[i] = c < H4 ? 0xFFFFFFFFu : 0u;
            if constexpr (NORM) xv[i] = nv[i];
            else xv[i] = xr[c < H4 ? c : H4 - 1];
        }
#pragma unroll
        for (int i = 0; i < kRouteNC; ++i)
#pragma unroll
            for (int k = 0; k < kRouteRPW; ++k) {
                const int c = c0 + 64 * i;
                gv[k][i] = gr[k][c < H4 ? c : H4 - 1];
            }
        __builtin_amdgcn_sched_barrier(0);  // every load of the batch is issued before the first use
#pragma unroll
        for (int i = 0; i < kRouteNC; ++i) {
            const float4 xc = masked(xv[i], m[i]);
            amax = fmaxf(amax, fmaxf(fmaxf(fabsf(xc.x), fabsf(xc.y)), fmaxf(fabsf(xc.z), fabsf(xc.w))));
            const double x0 = xc.x, x1 = xc.y, x2 = xc.z, x3 = xc.w;
#pragma unroll
            for (int k = 0; k < kRouteRPW; ++k) {
                const float4 g = gv[k][i];
                acc[k] = fma(x0, static_cast<double>(g.x), acc[k]);
                acc[k] = fma(x1, static_cast<double>(g.y), acc[k]);
                acc[k] = fma(x2, static_cast<double>(g.z), acc[k]);
                acc[k] = fma(x3, static_cast<double>(g.w), acc[k]);
            }
        }
    }
#pragma unroll
    for (int k = 0; k < kRouteRPW; ++k) out[k] = wave_sum_d_full(acc[k]);
    amax_out = wave_max_f_full(amax);
}

// Steps 6-8 of the route for token t in one wave (lane = expert, lg = its
// logit for lane < E): the f64 softmax, the greedy top-k and the renormalised
// gates, the outputs and the selection entries. The split route's leader and
// the many-row route's rank kernel both end here, so their routing is the
// same arithmetic.
__device__ __forceinline__ void route_rank(float lg_in, int lane, int t, int E, int K, int norm_topk,
                                           float routed_scale, uint32_t* __restrict__ idx_out,
                                           float* __restrict__ gates_out, float* __restrict__ probs_out,
                                           int* __restrict__ flag, const MoeSel& sel) {
    // 6. softmax in f64 over the f32 logits (lane = expert): max, exp,
    //    DPP-tree sum (the oracle's wave_tree_sum64 order), divide, round to
    //    f32; a lane past E is NaN and never ranked
    const bool valid = lane < E;
    const float lg = valid ? lg_in : -INFINITY;
    const double mx = static_cast<double>(wave_max_f_full(lg));
    const double ex = valid ? exp(static_cast<double>(lg) - mx) : 0.0;
    const double sum = wave_sum_d_full(ex);
    const float pr = valid ? static_cast<float>(ex / sum) : __int_as_float(0x7fc00000);
    if (valid && probs_out) probs_out[static_cast<size_t>(t) * E + lane] = pr;
    const int nvalid = __popcll(__ballot(pr == pr));

    // 7. greedy top-k (moe.rs:209-266): K times the largest remaining
    //    probability, the lowest index among equal ones, NaN never; slot j is
    //    the j-th pick. A probability is finite and >= +0 (ex >= 0, sum > 0),
    //    so -inf marks a lane out of the running (NaN, past E, or picked).
    //    Fewer than K finite probabilities: the token's routing failed
    //    (flag), every output of it zero.
    float pk = valid && pr == pr ? pr : -INFINITY;
    int my_slot = -1;
    int ej_mine = 0;
    float wj_mine = 0.0f;
    float den = 0.0f;
    const bool bad = nvalid < K;
    for (int j = 0; j < K; ++j) {
        const float mv = wave_max_f_full(pk);
        const unsigned long long mm = __ballot(pk == mv && mv != -INFINITY);
        const int lj = mm ? __ffsll(static_cast<long long>(mm)) - 1 : 0;
        const float wj = mm ? mv : 0.0f;
        den += bad ? 0.0f : wj;  // sequential f32 sum in slot order
        if (mm && lane == lj) {
            pk = -INFINITY;
            my_slot = j;
        }
        if (lane == j) {
            ej_mine = lj;
            wj_mine = wj;
        }
    }
    const bool chosen = my_slot >= 0;

    // 8. renormalise (the slot-order sum above + 1e-20), scale, publish
    den += 1e-20f;
    if (lane < K) {
        const int ej = bad ? 0 : ej_mine;
        float w = bad ? 0.0f : wj_mine;
        if (norm_topk) w = w / den;
        idx_out[t * K + lane] = static_cast<uint32_t>(ej);
        gates_out[t * K + lane] = w * routed_scale;
        if (sel.slot && !bad) sel.gate[ej * kMaxT + t] = w * routed_scale;
        if (lane == 0) flag[t] = bad ? 1 : 0;
    }
    if (sel.slot && valid) sel.slot[lane * kMaxT + t] = static_cast<uint8_t>(chosen && !bad ? my_slot + 1 : 0);
}

// Grid: 8 * S blocks, S = ceil(T / 8) * kRouteParts. Block b sits on XCD
// x = b % 8; its slot s = b / 8 is part s % kRouteParts of token
// (s / kRouteParts) * 8 + x (blocks of tokens >= T exit at once). Part 0 of
// a token is its leader: it gathers the logits and writes the token's
// routing; part 1 (part 0 when kRouteParts == 1) quantizes the token row
// after publishing; token 0's other parts zero the selection entries no
// token owns.
// NORM: the decoder layer's residual + post-attention RMSNorm first
// (decoder.rs:2596-2600): the routed row is rms_norm(x + attn) * w, as
// rms_norm_rows_kernel<1> computes it (f32 h, f64 sum of squares, f32
// rstd); every wave holds the whole row and reduces it itself; the quantizer
// part writes h = x + attn to h_out for the layer's final residual.
template <bool NORM>
__global__ __launch_bounds__(kRouteThreads) void moe_route_kernel(
    const float* __restrict__ x, const float* __restrict__ G, int T, int H, int E, int K, int norm_topk,
    float routed_scale, int8_t* __restrict__ xq, float* __restrict__ xs, uint32_t* __restrict__ idx_out,
    float* __restrict__ gates_out, float* __restrict__ probs_out, int* __restrict__ flag, MoeSel sel,
    const RouteNorm rn, RouteXchg* __restrict__ xch, unsigned wait_ticks) {
    __shared__ float s_logit[kMaxE];
    __shared__ unsigned s_missing;  // leader: parts it computes itself (bit p)
    const int xcd = blockIdx.x & 7;
    const int slot = blockIdx.x >> 3;
    const int part = slot % kRouteParts;
    const int t = (slot / kRouteParts) * 8 + xcd;
    if (t >= T) return;
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int H4 = H >> 2;
    const int EP = (E + kRouteParts - 1) / kRouteParts;
    const unsigned tag = static_cast<unsigned>(
        2ull * __hip_atomic_load(&xch->counter, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1ull);
    const float4* xr = reinterpret_cast<const float4*>(x + static_cast<size_t>(t) * H);

    // NORM: the routed row's chunks (one batch: NORM requires H <= 64 * 4 * kRouteNC)
    const float4* ar = NORM ? reinterpret_cast<const float4*>(rn.attn + static_cast<size_t>(t) * H) : nullptr;
    float4 nv[kRouteNC];
    float rstd = 1.0f;
    if constexpr (NORM) {
        const float4* wr = reinterpret_cast<const float4*>(rn.w);
        float4 hv[kRouteNC], gw[kRouteNC];
#pragma unroll
        for (int i = 0; i < kRouteNC; ++i) {
            const int c = lane + 64 * i;
            const float4 a = xr[c < H4 ? c : H4 - 1], b = ar[c < H4 ? c : H4 - 1];
            gw[i] = wr[c < H4 ? c : H4 - 1];
            hv[i] = make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
        }
        double ss = 0.0;
#pragma unroll
        for (int i = 0; i < kRouteNC; ++i) {
            if (lane + 64 * i < H4) {
                ss = fma(static_cast<double>(hv[i].x), static_cast<double>(hv[i].x), ss);
                ss = fma(static_cast<double>(hv[i].y), static_cast<double>(hv[i].y), ss);
                ss = fma(static_cast<double>(hv[i].z), static_cast<double>(hv[i].z), ss);
                ss = fma(static_cast<double>(hv[i].w), static_cast<double>(hv[i].w), ss);
            }
        }
        ss = wave_sum_d_full(ss);
        rstd = static_cast<float>(1.0 / sqrt(ss / static_cast<double>(H) + static_cast<double>(rn.eps)));
#pragma unroll
        for (int i = 0; i < kRouteNC; ++i) {
            const float4 g = gw[i];
            nv[i] = make_float4((hv[i].x * rstd) * g.x, (hv[i].y * rstd) * g.y, (hv[i].z * rstd) * g.z,
                                (hv[i].w * rstd) * g.w);
        }
    }

    // 1. this part's logits: wave w owns rows e0 + kRouteRPW w + k
    const bool quantizer = part == (kRouteParts > 1 ? 1 : 0);
    const int e0 = part * EP;
    float amax = 0.0f;
    {
        int r[kRouteRPW];
#pragma unroll
        for (int k = 0; k < kRouteRPW; ++k) {
            const int e = e0 + wave * kRouteRPW + k;
            r[k] = e < E ? e : E - 1;
        }
        double d[kRouteRPW];
        route_dots<NORM>(xr, nv, G, r, H4, lane, d, amax);
        if (lane < kRouteRPW) {
            const int el = wave * kRouteRPW + lane;
            const double v = lane == 0 ? d[0] : d[1];
            if (el < EP && e0 + el < E) s_logit[e0 + el] = static_cast<float>(v);
        }
    }
    __syncthreads();

    if (part != 0) {
        // 2. publish: one 8-byte word per logit (the logit's bits and the tag)
        if (wave == 0 && lane < EP) {
            const float lg = e0 + lane < E ? s_logit[e0 + lane] : 0.0f;
            *route_word(xch, t, part, lane) = static_cast<unsigned long long>(__float_as_uint(lg)) |
                                              (static_cast<unsigned long long>(tag) << 32);
        }
        // 3. quantize_row_i8 of the token row (wave 0 of the quantizer part
        //    holds the whole row's max|x|), after publishing
        if (quantizer && wave == 0) {
            const float a_scale = amax > 0.0f ? amax / 127.0f : 1.0f;
            const float inv = 1.0f / a_scale;
#pragma unroll 1
            for (int c = lane; c < H4; c += 64) {
                float4 v;
                if constexpr (NORM) {
                    const float4 a = xr[c], b = ar[c], g = reinterpret_cast<const float4*>(rn.w)[c];
                    const float4 h = make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
                    reinterpret_cast<float4*>(rn.h_out + static_cast<size_t>(t) * H)[c] = h;
                    v = make_float4((h.x * rstd) * g.x, (h.y * rstd) * g.y, (h.z * rstd) * g.z, (h.w * rstd) * g.w);
                } else {
                    v = xr[c];
                }
                char4 q;
                q.x = quant_i8(v.x, inv, false);
                q.y = quant_i8(v.y, inv, false);
                q.z = quant_i8(v.z, inv, false);
                q.w = quant_i8(v.w, inv, false);
                reinterpret_cast<char4*>(xq + static_cast<size_t>(t) * H)[c] = q;
            }
            if (lane == 0) xs[t] = a_scale;
        }
        // 4. token 0's non-leader parts zero the selection entries no token
        //    owns (e >= E or t >= T), one 4-byte word (an expert row, tokens
        //    t0..t0+3) at a time, byte by byte where a token owns part of it
        if (sel.slot && t == 0) {
            const int workers = kRouteParts - 1;
#pragma unroll 1
            for (int wi = (part - 1) * kRouteThreads + static_cast<int>(threadIdx.x); wi < kMaxE * kMaxT / 4;
                 wi += workers * kRouteThreads) {
                const int ei = wi / (kMaxT / 4), t0 = 4 * (wi % (kMaxT / 4));
                uint8_t* w = sel.slot + 4 * wi;
                if (ei >= E || t0 >= T) {
                    *reinterpret_cast<uint32_t*>(w) = 0u;
                } else {
                    for (int ti = T; ti < t0 + 4; ++ti) w[ti - t0] = 0;
                }
            }
        }
        return;
    }

    // 5. leader: the other parts' logits (bounded wait); lane e >= EP polls
    //    the word of expert e
    const int nparts = (E + EP - 1) / EP;
    if (wave == 0) {
        const int pe = lane / EP, ie = lane % EP;
        const bool watch = lane >= EP && lane < E;
        bool ready = !watch;
        float got = 0.0f;
        const unsigned long long t_end = realtime() + wait_ticks;
        while (wait_ticks) {  // 0: no wait, every part computed below
            if (!ready) {
                const unsigned long long w =
                    __hip_atomic_load(route_word(xch, t, pe, ie), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                if (static_cast<unsigned>(w >> 32) == tag) {
                    ready = true;
                    got = __uint_as_float(static_cast<unsigned>(w));
                }
            }
            if (__ballot(!ready) == 0ull || realtime() > t_end) break;
            __builtin_amdgcn_s_sleep(1);
        }
        if (watch && ready) s_logit[lane] = got;
        // a part is computed here if any of its words is missing
        unsigned long long miss_lanes = __ballot(watch && !ready);
        unsigned miss = 0;
        for (int pm = 1; pm < nparts; ++pm)
            if ((miss_lanes >> (pm * EP)) & ((1ull << EP) - 1ull)) miss |= 1u << pm;
        if (lane == 0) s_missing = miss;
    }
    if (!(kRouteParts > 1)) {
        // one part: the leader is the quantizer (its wave 0 holds max|x|)
        if (wave == 0) {
            const float a_scale = amax > 0.0f ? amax / 127.0f : 1.0f;
            const float inv = 1.0f / a_scale;
#pragma unroll 1
            for (int c = lane; c < H4; c += 64) {
                float4 v;
                if constexpr (NORM) {
                    const float4 a = xr[c], b = ar[c], g = reinterpret_cast<const float4*>(rn.w)[c];
                    const float4 h = make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
                    reinterpret_cast<float4*>(rn.h_out + static_cast<size_t>(t) * H)[c] = h;
                    v = make_float4((h.x * rstd) * g.x, (h.y * rstd) * g.y, (h.z * rstd) * g.z, (h.w * rstd) * g.w);
                } else {
                    v = xr[c];
                }
                char4 q;
                q.x = quant_i8(v.x, inv, false);
                q.y = quant_i8(v.y, inv, false);
                q.z = quant_i8(v.z, inv, false);
                q.w = quant_i8(v.w, inv, false);
                reinterpret_cast<char4*>(xq + static_cast<size_t>(t) * H)[c] = q;
            }
            if (lane == 0) xs[t] = a_scale;
        }
    }
    __syncthreads();
    // a part that never published: its rows, computed here (same lanes, same order)
    for (unsigned miss = s_missing; miss; miss &= miss - 1u) {
        const int pm = __ffs(static_cast<int>(miss)) - 1;
        int r[kRouteRPW];
#pragma unroll
        for (int k = 0; k < kRouteRPW; ++k) {
            const int e = pm * EP + wave * kRouteRPW + k;
            r[k] = e < E ? e : E - 1;
        }
        double d[kRouteRPW];
        float amax_unused;
        route_dots<NORM>(xr, nv, G, r, H4, lane, d, amax_unused);
        if (lane < kRouteRPW) {
            const int el = wave * kRouteRPW + lane;
            const double v = lane == 0 ? d[0] : d[1];
            if (el < EP && pm * EP + el < E) s_logit[pm * EP + el] = static_cast<float>(v);
        }
        __syncthreads();
    }
    if (wave != 0) return;
    route_rank(s_logit[lane < kMaxE ? lane : 0], lane, t, E, K, norm_topk, routed_scale, idx_out, gates_out,
               probs_out, flag, sel);
}

// Advances the route exchange's counter once the route kernel of a call has
// finished (stream order): the next call's records carry a new tag.
__global__ void route_epoch_bump_kernel(RouteXchg* __restrict__ xch) {
    if (threadIdx.x == 0 && blockIdx.x == 0) xch->counter = xch->counter + 1ull;
}

// ---- route of many rows (a prefill chunk): logits, then the rank ------------
// The split route reads the router once per token (327 KB each, through the
// token's XCD L2), which is what a 256-1024-row chunk pays for. Here a block
// holds two router rows per wave in registers (eight experts) and runs them
// against kRowsTB token rows staged in LDS (all their loads in flight at
// once): the router is read once per kRowsTB tokens (4 up to 512 rows, where
// the blocks are few, else 8). Each logit is route_dots' f64 dot in the same
// lane order (lane l: float4 chunks l + 64 i, x, y, z, w in turn) and the
// same DPP tree, so the logits are the split route's bit for bit;
// route_rank_kernel then runs the split route's own softmax / top-k
// (route_rank) on them, one wave per token. The f64 FMAs, converts and DPP
// trees bound it (about 10 us of VALU at 1024 rows). Rows up to 1280
// wide (one batch of kRouteNC float4 per lane); no exchange buffer, no
// quantized rows.
template <int kRowsTB>
__global__ __launch_bounds__(256) void route_logits_kernel(const float* __restrict__ x, const float* __restrict__ G,
                                                           int T, int H, int E, float* __restrict__ logits) {
    // the block's kRowsTB token rows, staged at once (every load in flight
    // together), then read per token from LDS
    __shared__ float4 s_x[kRowsTB][64 * kRouteNC];
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int H4 = H >> 2;
    const int t0 = static_cast<int>(blockIdx.x) * kRowsTB;
    const int e0 = static_cast<int>(blockIdx.y) * kRouteEPP + wave * kRouteRPW;
    float4 gv[kRouteRPW][kRouteNC];
    unsigned m[kRouteNC];
#pragma unroll
    for (int i = 0; i < kRouteNC; ++i) {
        const int c = lane + 64 * i;
        m[i] = c < H4 ? 0xFFFFFFFFu : 0u;
#pragma unroll
        for (int k = 0; k < kRouteRPW; ++k) {
            const int e = e0 + k < E ? e0 + k : E - 1;
            gv[k][i] = reinterpret_cast<const float4*>(G + static_cast<size_t>(e) * H)[c < H4 ? c : H4 - 1];
        }
    }
    constexpr int kPer = kRowsTB * 64 * kRouteNC / 256;  // float4 per thread
    float4 st[kPer];
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
        const int q = static_cast<int>(threadIdx.x) + 256 * j;
        const int u = q / (64 * kRouteNC), c = q % (64 * kRouteNC);
        const int t = t0 + u < T ? t0 + u : T - 1;
        st[j] = reinterpret_cast<const float4*>(x + static_cast<size_t>(t) * H)[c < H4 ? c : H4 - 1];
    }
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
        const int q = static_cast<int>(threadIdx.x) + 256 * j;
        s_x[q / (64 * kRouteNC)][q % (64 * kRouteNC)] = st[j];
    }
    __syncthreads();
#pragma unroll 1
    for (int u = 0; u < kRowsTB; ++u) {
        const int t = t0 + u;
        double acc[kRouteRPW];
#pragma unroll
        for (int k = 0; k < kRouteRPW; ++k) acc[k] = 0.0;
#pragma unroll
        for (int i = 0; i < kRouteNC; ++i) {
            const float4 xv = s_x[u][lane + 64 * i];
            const float4 xc = make_float4(__uint_as_float(__float_as_uint(xv.x) & m[i]),
                                          __uint_as_float(__float_as_uint(xv.y) & m[i]),
                                          __uint_as_float(__float_as_uint(xv.z) & m[i]),
                                          __uint_as_float(__float_as_uint(xv.w) & m[i]));
            const double x0 = xc.x, x1 = xc.y, x2 = xc.z, x3 = xc.w;
#pragma unroll
            for (int k = 0; k < kRouteRPW; ++k) {
                const float4 g = gv[k][i];
                acc[k] = fma(x0, static_cast<double>(g.x), acc[k]);
                acc[k] = fma(x1, static_cast<double>(g.y), acc[k]);
                acc[k] = fma(x2, static_cast<double>(g.z), acc[k]);
                acc[k] = fma(x3, static_cast<double>(g.w), acc[k]);
            }
        }
        double d[kRouteRPW];
#pragma unroll
        for (int k = 0; k < kRouteRPW; ++k) d[k] = wave_sum_d_full(acc[k]);
        if (t < T && lane < kRouteRPW && e0 + lane < E)
            logits[static_cast<size_t>(t) * E + e0 + lane] = static_cast<float>(lane == 0 ? d[0] : d[1]);
    }
}

// One wave per token: its E logits (lane = expert) through route_rank.
__global__ __launch_bounds__(256) void route_rank_kernel(const float* __restrict__ logits, int T, int E, int K,
                                                         int norm_topk, float routed_scale,
                                                         uint32_t* __restrict__ idx_out,
                                                         float* __restrict__ gates_out,
                                                         float* __restrict__ probs_out, int* __restrict__ flag) {
    const int t = static_cast<int>(blockIdx.x) * 4 + static_cast<int>(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (t >= T) return;
    const float lg = logits[static_cast<size_t>(t) * E + (lane < E ? lane : 0)];
    route_rank(lg, lane, t, E, K, norm_topk, routed_scale, idx_out, gates_out, probs_out, flag, MoeSel{});
}

// Expert of this block: lane e loads expert e's 64-byte slot row (four
// 16-byte loads in flight) and one ballot gives the set of experts with
// pairs; the a-th set bit (a = blockIdx.y) is found with one more ballot.
// The row block is blockIdx.x: with linear block id x + X y and blocks dealt
// to the eight XCDs round-robin, an expert's row blocks spread over all of
// them (X = 56 is a multiple of 8), where blockIdx.x = expert would put all of
// an expert's weights through one XCD and leave the XCDs a whole expert
// apart in load.
// Shared mode is one expert whose pairs are the tokens. Slots past the number
// of active experts get -1.
// Route zeroes every entry t >= T, so for T <= 16 the first 16 bytes of a
// row decide it: one load per lane instead of four (every wave of the
// launch reads the 64 rows before its first weight load; T = 8 gate/up
// 16.8 -> 15.7 us).
__device__ __forceinline__ int block_expert(const MoeSel& sel, int shared_T, int T, int slot = -1) {
    if (shared_T > 0) return 0;
    if (slot < 0) slot = static_cast<int>(blockIdx.y);
    const int lane = threadIdx.x & 63;
    const uint4* row = reinterpret_cast<const uint4*>(sel.slot + lane * kMaxT);
    unsigned any;
    if (T <= 16) {  // kernel argument: a uniform branch
        const uint4 r0 = row[0];
        any = r0.x | r0.y | r0.z | r0.w;
    } else {
        const uint4 r0 = row[0], r1 = row[1], r2 = row[2], r3 = row[3];
        any = (r0.x | r0.y | r0.z | r0.w) | (r1.x | r1.y | r1.z | r1.w) | (r2.x | r2.y | r2.z | r2.w) |
              (r3.x | r3.y | r3.z | r3.w);
    }
    const unsigned long long m = __ballot(any != 0u);
    const int below = __popcll(m & ((1ull << lane) - 1ull));
    const unsigned long long hit = __ballot(any != 0u && below == slot);
    return hit ? __ffsll(static_cast<long long>(hit)) - 1 : -1;
}

// Wave 0 collects the block's pairs (t*K + j) in increasing token order from
// column e of the slot matrix — one load per lane and one ballot — with their
// gates when s_gate is non-null (1.0 for the shared expert). The caller
// synchronises before reading them. All loads on these kernels' critical path
// are issued unconditionally from clamped addresses, with invalid lanes masked
// arithmetically: a select between a load and a constant tends to become a
// branch around the load with a full wait inside it, which serialises the
// memory round trips these kernels depend on overlapping.
__device__ __forceinline__ void block_pairs(const MoeSel& sel, int T, int K, int e, int shared_T, int* s_pid,
                                            int* s_tok, float* s_gate, int* s_np) {
    if (threadIdx.x >= 64) return;
    const int lane = threadIdx.x;
    if (shared_T > 0) {
        if (lane < shared_T) {
            s_pid[lane] = lane;
            s_tok[lane] = lane;
            if (s_gate) s_gate[lane] = 1.0f;
        }
        if (lane == 0) *s_np = shared_T;
        return;
    }
    const int v = sel.slot[e * kMaxT + lane];  // zero for t >= T
    const float g = s_gate ? sel.gate[e * kMaxT + lane] : 0.0f;
    const unsigned long long m = __ballot(v != 0);
    if (v != 0) {
        const int pos = __popcll(m & ((1ull << lane) - 1ull));
        s_pid[pos] = lane * K + v - 1;
        s_tok[pos] = lane;
        if (s_gate) s_gate[pos] = g;
    }
    if (lane == 0) *s_np = __popcll(m);
}

// Chunk c of a weight row, or zeros when c >= C (address clamped into the
// row, so the load itself is unconditional).
__device__ __forceinline__ int4 row_chunk(const int4* row, int c, int C) {
    const int4 v = ld_stream(row + (c < C ? c : C - 1));
    const int m = c < C ? -1 : 0;
    return make_int4(v.x & m, v.y & m, v.z & m, v.w & m);
}

// Stage int8 token rows into LDS: lds[p * C + c] = row(p)[c] for p < nrows,
// where row(p) is token rows[p] (or p when rows is null). Four chunks per
// thread per round, loads issued before the stores. Indices past the end are
// clamped to the last chunk for the store as well as the load (a conditional
// store lets the compiler sink the load under the condition): those threads
// rewrite the last chunk with the value it already holds.
__device__ __forceinline__ void stage_rows(int4* lds, const int8_t* __restrict__ xq, int H, int C, int nrows,
                                          const int* rows) {
    const int n = nrows * C;
    for (int base = 0; base < n; base += 4 * 256) {
        int4 v[4];
        int at[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int i = base + 256 * k + static_cast<int>(threadIdx.x);
            at[k] = i < n ? i : n - 1;
            const int pp = at[k] / C, c = at[k] - pp * C;
            const int tok = rows ? rows[pp] : pp;
            v[k] = reinterpret_cast<const int4*>(xq + static_cast<size_t>(tok) * H)[c];
        }
#pragma unroll
        for (int k = 0; k < 4; ++k) lds[at[k]] = v[k];
    }
}

typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(1))) const void global_void_t;

// Copy n 16-byte chunks src[0..n) to lds[0..n) with gfx950's direct
// global-to-LDS loads (global_load_lds_dwordx4: lane L of a wave lands at the
// wave's LDS base + 16 L), no VGPRs involved; the next barrier waits for them.
// Whole 64-chunk blocks are written, so lds must hold n rounded up to 64.
__device__ __forceinline__ void stage_lds_dma(int4* lds, const int4* __restrict__ src, int n) {
    const int lane = threadIdx.x & 63;
    for (int base = threadIdx.x & ~63; base < n; base += 256) {
        const int i = base + lane;
        __builtin_amdgcn_global_load_lds((global_void_t*)(src + (i < n ? i : n - 1)), (lds_void_t*)(lds + base), 16,
                                         0, 0);
    }
}

constexpr int kAllTok = 32;  // stage every token row when T <= kAllTok

// ---- gate/up ------------------------------------------------------------------
// Block = 256 threads = (256 / LPR) row groups, one weight row per group held
// in registers (2 * JC 16-byte loads in flight per lane); the block's pairs
// are then taken one at a time against the staged token rows. ALLTOK (T <=
// kAllTok) stages every token row once; its own instantiation, without the
// per-pass staging path, fits 64 VGPRs, i.e. 8 waves per SIMD, so about
// every block of a T = 8 step is resident at once.
// The shared expert folded into the routed launch: grid rows y < nslots are
// its blocks (each covering gridDim.x * G of its I rows), every token a pair
// with gate 1, and y - nslots is the routed slot. Its blocks come first in
// the dispatch order: each takes every token, so dispatched last they would
// be the launch's tail. nslots = 0: none.
struct SharedGU {
    const int8_t *wg, *wu;
    const float *sg, *su;
    float* act;  // [T][I]
    int I, nslots;
    // non-null: block (0, 0) advances the route exchange's counter (the
    // call's route kernel has finished, by stream order)
    unsigned long long* route_counter;
};

template <int LPR, int JC, bool ALLTOK>
__global__ __launch_bounds__(256) void moe_gate_up_kernel(
    const MoeSel sel, int T, int K,
    const int8_t* __restrict__ xq, const float* __restrict__ xs, const int8_t* __restrict__ wg,
    const float* __restrict__ sg, const int8_t* __restrict__ wu, const float* __restrict__ su,
    float* __restrict__ act, int H, int I, int shared_T, const SharedGU sh) {
    extern __shared__ int4 lds_x[];  // [rows staged][H/16]
    __shared__ int s_pid[kMaxT];
    __shared__ int s_tok[kMaxT];
    __shared__ float s_xs[64];  // one per lane of the staging wave
    __shared__ int s_np;
    constexpr int G = 256 / LPR;  // rows per block
    if (sh.route_counter && blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x == 0)
        *sh.route_counter = *sh.route_counter + 1ull;
    const bool shb = static_cast<int>(blockIdx.y) < sh.nslots;  // block-uniform
    if (shb) {
        shared_T = T;
        wg = sh.wg;
        wu = sh.wu;
        sg = sh.sg;
        su = sh.su;
        act = sh.act;
        I = sh.I;
    }
    const int e = shb ? 0 : block_expert(sel, shared_T, T, static_cast<int>(blockIdx.y) - sh.nslots);
    if (e < 0) return;
    const int grp = threadIdx.x / LPR;
    const int lane = threadIdx.x % LPR;
    const int C = H >> 4;
    const int r = (shb ? static_cast<int>(blockIdx.y) * static_cast<int>(gridDim.x) * G : 0) +
                  static_cast<int>(blockIdx.x) * G + grp;
    const bool live = r < I;  // rows past I compute unused values from row 0
    const size_t row = static_cast<size_t>(e) * I + (live ? r : 0);
    int4 wgv[JC], wuv[JC];
    {
        const int4* grow = reinterpret_cast<const int4*>(wg + row * H);
        const int4* urow = reinterpret_cast<const int4*>(wu + row * H);
#pragma unroll
        for (int j = 0; j < JC; ++j) {
            const int c = lane + LPR * j;
            wgv[j] = row_chunk(grow, c, C);
            wuv[j] = row_chunk(urow, c, C);
        }
    }
    const float sgr = sg[row];
    const float sur = su[row];
    constexpr bool all_tok = ALLTOK;
    if (all_tok) stage_lds_dma(lds_x, reinterpret_cast<const int4*>(xq), T * C);  // rows are contiguous
    if (threadIdx.x < 64) {
        const int tt = threadIdx.x < T ? threadIdx.x : T - 1;
        __builtin_amdgcn_global_load_lds((global_void_t*)(xs + tt), (lds_void_t*)s_xs, 4, 0, 0);
    }
    block_pairs(sel, T, K, e, shared_T, s_pid, s_tok, nullptr, &s_np);
    __syncthreads();
    const int P = s_np;

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
    const MoeSel sel, int T, int K, const float* __restrict__ act, const int8_t* __restrict__ wd,
    const float* __restrict__ sd, float* __restrict__ ybuf, int H, int I, int shared_T) {
    extern __shared__ int4 lds_a[];  // [kPairStage][I/16]
    __shared__ float lds_as[kPairStage];
    __shared__ int s_pid[kMaxT];
    __shared__ int s_tok[kMaxT];
    __shared__ float s_gate[kMaxT];
    __shared__ int s_np;
    constexpr int G = 256 / LPR;
    const int e = block_expert(sel, shared_T, T);
    if (e < 0) return;
    const int grp = threadIdx.x / LPR;
    const int lane = threadIdx.x % LPR;
    const int wave = threadIdx.x >> 6;
    const int wl = threadIdx.x & 63;
    const int C = I >> 4;
    const int r = blockIdx.x * G + grp;
    const bool live = r < H;  // rows past H compute unused values from row 0
    const size_t row = static_cast<size_t>(e) * H + (live ? r : 0);
    int4 wv[JC];
    {
        const int4* drow = reinterpret_cast<const int4*>(wd + row * I);
#pragma unroll
        for (int j = 0; j < JC; ++j) wv[j] = row_chunk(drow, lane + LPR * j, C);
    }
    const float sdr = sd[row];
    block_pairs(sel, T, K, e, shared_T, s_pid, s_tok, s_gate, &s_np);
    __syncthreads();
    const int P = s_np;
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
                amax = wave_max_f_full(amax);
                const float a_scale = amax > 0.0f ? amax / 127.0f : 1.0f;
                const float inv = 1.0f / a_scale;
                for (int i = wl; i < I; i += 64) lds_b[pp * I + i] = quant_i8(ar[i], inv, false);
                if (wl == 0) lds_as[pp] = a_scale;
                continue;
            }
            float v[NQ];
#pragma unroll
            for (int q = 0; q < NQ; ++q) {
                const int i = wl + 64 * q;
                v[q] = ar[i < I ? i : I - 1];  // a duplicate of the last value past I: max unchanged
            }
            float amax = 0.0f;
#pragma unroll
            for (int q = 0; q < NQ; ++q) amax = fmaxf(amax, fabsf(v[q]));
            amax = wave_max_f_full(amax);
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
                ybuf[static_cast<size_t>(pid) * H + r] = yv * s_gate[pb + i];
            }
        }
    }
}

// ---- down + combine (one block per token and row block) -----------------------
// Block (t, rb), DC_THREADS threads = (DC_THREADS / LPR) lane groups; group g
// < K * R owns slot j = g % K and row r = rb * R + g / K of token t, R =
// (DC_THREADS / LPR) / K. The expert ids and the token's K act rows are
// requested first, the down rows as soon as the ids arrive, and the block
// re-quantizes the act rows (quantize_row_i8, one wave per row, K <= 8) into
// LDS while the down rows are in flight; each group's dot gives
// y_j[r] = ((f32)acc * as_j) * sd[e_j][r] * gate_j (decoder.rs:2244-2246),
// and the block sums y_0..y_{K-1} in slot order (+ shared) into out[t][r]
// (decoder.rs:2253-2261) — no per-pair buffer, no separate combine launch.
// A weight row used by several of the step's tokens is read once per token;
// such blocks run together (t varies fastest), so the repeats mostly hit the
// caches.
constexpr int DC_THREADS = 512;

template <int LPR, int JC, int RPG>
__global__ __launch_bounds__(DC_THREADS) void moe_down_combine_kernel(
    const uint32_t* __restrict__ idx, const float* __restrict__ gates, const int* __restrict__ flag, int T, int K,
    const float* __restrict__ act, const int8_t* __restrict__ wd, const float* __restrict__ sd,
    const float* __restrict__ shared_y, const float* __restrict__ resid, float* __restrict__ out, int H, int I,
    int E) {
    extern __shared__ int4 lds_q[];  // [K][I/16] quantized act rows of token t
    __shared__ float s_as[kMaxK];
    constexpr int NG = DC_THREADS / LPR;
    __shared__ float s_y[RPG * NG];
    // XCD-aware order: blocks are dispatched to the 8 XCDs round-robin
    // (block b to XCD b % 8, each with its own L2), and block b takes row
    // block rb = b % 8 + 8 * (b / (8 T)) of token t = (b / 8) % T, so every
    // token's block for one row block runs on the same XCD, one after the
    // other: a down row two tokens share (the same expert) comes from HBM
    // once and from that L2 the second time.
    const int b = static_cast<int>(blockIdx.x);
    const int t = (b >> 3) % T;
    const int rb = (b & 7) + 8 * ((b >> 3) / T);
    // lane group g owns the RPG (slot, row) pairs p = g + NG q: slot
    // j = p % K, row rb * R + p / K
    const int R = RPG * NG / K;
    const int g = threadIdx.x / LPR;
    const int ln = threadIdx.x % LPR;
    const int wave = threadIdx.x >> 6;
    const int wl = threadIdx.x & 63;
    const int C = I >> 4;
    int jq[RPG];
    bool liveq[RPG];
    uint32_t eid[RPG];
    float gate[RPG];
    // 1. expert ids and gates of the group's slots, the token's flag, and
    //    (wave w < K) act row t*K + w — all issued before anything waits
#pragma unroll
    for (int q = 0; q < RPG; ++q) {
        const int p = g + NG * q;
        jq[q] = p % K;
        liveq[q] = p < K * R && rb * R + p / K < H;  // dead pairs compute unused values from valid addresses
        const int pid = t * K + (liveq[q] ? jq[q] : 0);
        eid[q] = idx[pid];
        gate[q] = gates[pid];
    }
    const int bad = flag[t];
    const bool qwave = wave < K;  // wave-uniform
    const float* ar = act + static_cast<size_t>(t * K + (qwave ? wave : 0)) * I;
    const bool short_row = I <= 64 * NQ;
    float v[NQ];
    if (short_row) {
#pragma unroll
        for (int q = 0; q < NQ; ++q) {
            const int i = wl + 64 * q;
            v[q] = ar[i < I ? i : I - 1];  // a duplicate of the last value past I: max unchanged
        }
    }
    // 2. the down rows of the group's pairs
    int4 wv[RPG][JC];
    float sdr[RPG];
#pragma unroll
    for (int q = 0; q < RPG; ++q) {
        const uint32_t e = eid[q] < static_cast<uint32_t>(E) ? eid[q] : 0u;
        const size_t row = static_cast<size_t>(e) * H + (liveq[q] ? rb * R + (g + NG * q) / K : 0);
        const int4* drow = reinterpret_cast<const int4*>(wd + row * I);
#pragma unroll
        for (int c = 0; c < JC; ++c) wv[q][c] = row_chunk(drow, ln + LPR * c, C);
        sdr[q] = sd[row];
    }
    // 3. quantize_row_i8 of the act rows into LDS
    if (qwave) {
        int8_t* qrow = reinterpret_cast<int8_t*>(lds_q) + wave * I;
        if (short_row) {
            float amax = 0.0f;
#pragma unroll
            for (int q = 0; q < NQ; ++q) amax = fmaxf(amax, fabsf(v[q]));
            amax = wave_max_f_full(amax);
            const float a_scale = amax > 0.0f ? amax / 127.0f : 1.0f;
            const float inv = 1.0f / a_scale;
#pragma unroll
            for (int q = 0; q < NQ; ++q)
                if (wl + 64 * q < I) qrow[wl + 64 * q] = quant_i8(v[q], inv, false);
            if (wl == 0) s_as[wave] = a_scale;
        } else {  // long rows: two passes over L2
            float amax = 0.0f;
            for (int i = wl; i < I; i += 64) amax = fmaxf(amax, fabsf(ar[i]));
            amax = wave_max_f_full(amax);
            const float a_scale = amax > 0.0f ? amax / 127.0f : 1.0f;
            const float inv = 1.0f / a_scale;
            for (int i = wl; i < I; i += 64) qrow[i] = quant_i8(ar[i], inv, false);
            if (wl == 0) s_as[wave] = a_scale;
        }
    }
    __syncthreads();
#pragma unroll
    for (int q = 0; q < RPG; ++q) {
        int d = 0;
#pragma unroll
        for (int c = 0; c < JC; ++c) {
            const int cc = ln + LPR * c;
            if (cc < C) d = dot16_i8(wv[q][c], lds_q[jq[q] * C + cc], d);
        }
        d = reduce_lanes<LPR>(d);
        if (ln == 0) s_y[g + NG * q] = ((static_cast<float>(d) * s_as[jq[q]]) * sdr[q]) * gate[q];
    }
    __syncthreads();
    // 4. slot-order sum of the token's K results for each row
    if (threadIdx.x < R) {
        const int rr = rb * R + threadIdx.x;
        if (rr < H) {
            float o = 0.0f;
            if (!bad) {
                for (int jj = 0; jj < K; ++jj) o += s_y[threadIdx.x * K + jj];
                if (shared_y) o += shared_y[static_cast<size_t>(t) * H + rr];
            }
            if (resid) o = resid[static_cast<size_t>(t) * H + rr] + o;  // h + mlp_out (decoder.rs:2625)
            out[static_cast<size_t>(t) * H + rr] = o;
        }
    }
}

// ---- combine (after the grouped down kernel) ----------------------------------
// out[t][c] = ((0 + y[t*K + 0][c]) + y[t*K + 1][c]) ... (+ shared[t][c]) in
// slot order (decoder.rs:2253-2261), the same sums in the same order as the
// down + combine kernel; a token whose routing failed (flag) combines to zero.
// Thread = 4 consecutive columns of one token.
__global__ __launch_bounds__(256) void moe_combine_kernel(const float* __restrict__ ybuf, const int* __restrict__ flag,
                                                          const float* __restrict__ shared_y,
                                                          const float* __restrict__ resid, float* __restrict__ out,
                                                          int K, int H) {
    const int t = blockIdx.y;
    const int c4 = blockIdx.x * 256 + static_cast<int>(threadIdx.x);
    if (c4 >= (H >> 2)) return;
    float4 o = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (!flag[t]) {
        for (int j = 0; j < K; ++j) {
            const float4 y = reinterpret_cast<const float4*>(ybuf + static_cast<size_t>(t * K + j) * H)[c4];
            o.x += y.x;
            o.y += y.y;
            o.z += y.z;
            o.w += y.w;
        }
        if (shared_y) {
            const float4 y = reinterpret_cast<const float4*>(shared_y + static_cast<size_t>(t) * H)[c4];
            o.x += y.x;
            o.y += y.y;
            o.z += y.z;
            o.w += y.w;
        }
    }
    if (resid) {  // the layer's residual: h + mlp_out (decoder.rs:2625)
        const float4 r = reinterpret_cast<const float4*>(resid + static_cast<size_t>(t) * H)[c4];
        o = make_float4(r.x + o.x, r.y + o.y, r.z + o.z, r.w + o.w);
    }
    reinterpret_cast<float4*>(out + static_cast<size_t>(t) * H)[c4] = o;
}

struct GemvArgs {
    MoeSel sel;
    int T, K, H, I, shared_T;
};

template <int LPR>
hipError_t launch_gate_up_lpr(hipStream_t s, dim3 grid, size_t lds, int JC, const GemvArgs& a, const int8_t* xq,
                              const float* xs, const int8_t* wg, const float* sg, const int8_t* wu, const float* su,
                              float* act, const SharedGU& sh) {
#define FOCR_GU(J)                                                                                              \
    case J:                                                                                                     \
        if (a.T <= kAllTok)                                                                                     \
            FOCR_LAUNCH((moe_gate_up_kernel<LPR, J, true>), grid, dim3(256), lds, s, a.sel, a.T, a.K, xq, xs, wg, \
                        sg, wu, su, act, a.H, a.I, a.shared_T, sh);                                             \
        else                                                                                                    \
            FOCR_LAUNCH((moe_gate_up_kernel<LPR, J, false>), grid, dim3(256), lds, s, a.sel, a.T, a.K, xq, xs,    \
                        wg, sg, wu, su, act, a.H, a.I, a.shared_T, sh);                                         \
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
hipError_t launch_down_lpr(hipStream_t s, dim3 grid, size_t lds, int JC, const GemvArgs& a, const float* act,
                           const int8_t* wd, const float* sd, float* ybuf) {
#define FOCR_DN(J)                                                                                           \
    case J:                                                                                                  \
        FOCR_LAUNCH((moe_down_kernel<LPR, J>), grid, dim3(256), lds, s, a.sel, a.T, a.K, act, wd, sd, ybuf, \
                    a.H, a.I, a.shared_T);                                                                   \
        break;
    switch (JC) {
        FOCR_DN(1) FOCR_DN(2) FOCR_DN(3) FOCR_DN(4) FOCR_DN(5) FOCR_DN(6) FOCR_DN(7) FOCR_DN(8)
        default:
            return hipErrorInvalidValue;
    }
#undef FOCR_DN
    return hipGetLastError();
}

MoeSel sel_of(void* buf) {
    char* b = static_cast<char*>(buf);
    if (!b) return MoeSel{nullptr, nullptr};
    return MoeSel{reinterpret_cast<uint8_t*>(b), reinterpret_cast<float*>(b + kMaxE * kMaxT)};
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

bool dims_ok(const MoeDims& d) {
    return d.t >= 1 && d.t <= kMaxT && d.n_experts >= 1 && d.n_experts <= kMaxE && d.top_k >= 1 &&
           d.top_k <= kMaxK && d.top_k <= d.n_experts;
}

}  // namespace

size_t moe_sel_bytes() { return kMaxE * kMaxT + kMaxE * kMaxT * 4; }

size_t moe_route_xchg_bytes(size_t t) {
    return sizeof(RouteXchg) + t * kRouteParts * kRouteEPP * sizeof(unsigned long long);
}

hipError_t launch_moe_route(hipStream_t s, const MoeDims& d, const float* hidden, const float* router,
                            int norm_topk, float routed_scale, int8_t* xq, float* xs, uint32_t* idx, float* gates,
                            float* probs, int* flag, void* sel, void* xchg, unsigned wait_ticks,
                            const MoeRouteNorm* norm) {
    // with the selection matrices (the decode kernels' input) t <= kMaxT; a
    // prefill chunk's routing alone, t <= kRouteMaxT
    const int t_max = sel ? kMaxT : kRouteMaxT;
    if (d.t < 1 || d.t > t_max || d.n_experts < 1 || d.n_experts > kMaxE || d.top_k < 1 || d.top_k > kMaxK ||
        d.top_k > d.n_experts || d.hidden % 4 != 0 || d.hidden > 2048 || !xchg)
        return hipErrorInvalidValue;
    static_assert(kRouteRPW == 2, "route_dots results are taken as d[0] / d[1]");
    // token t on XCD t % 8, its kRouteParts blocks at slots (t / 8) * kRouteParts + p
    const dim3 grid(static_cast<unsigned>(8 * ((d.t + 7) / 8) * kRouteParts));
    RouteXchg* x = static_cast<RouteXchg*>(xchg);
    if (norm) {
        // one batch of kRouteNC float4 per lane holds the whole row
        if (d.hidden > 64 * 4 * kRouteNC || !norm->attn || !norm->w || !norm->h_out) return hipErrorInvalidValue;
        const RouteNorm rn{norm->attn, norm->w, norm->eps, norm->h_out};
        FOCR_LAUNCH(moe_route_kernel<true>, grid, dim3(kRouteThreads), 0, s, hidden, router, d.t, d.hidden,
                    d.n_experts, d.top_k, norm_topk, routed_scale, xq, xs, idx, gates, probs, flag, sel_of(sel), rn, x,
                    wait_ticks);
    } else {
        FOCR_LAUNCH(moe_route_kernel<false>, grid, dim3(kRouteThreads), 0, s, hidden, router, d.t, d.hidden,
                    d.n_experts, d.top_k, norm_topk, routed_scale, xq, xs, idx, gates, probs, flag, sel_of(sel),
                    RouteNorm{}, x, wait_ticks);
    }
    return hipGetLastError();
}

bool moe_route_rows_supported(int hidden) { return hidden % 4 == 0 && hidden > 0 && hidden <= 64 * 4 * kRouteNC; }

hipError_t launch_moe_route_rows(hipStream_t s, const MoeDims& d, const float* hidden, const float* router,
                                 int norm_topk, float routed_scale, uint32_t* idx, float* gates, float* probs,
                                 int* flag, float* logits) {
    if (d.t < 1 || d.t > kRouteMaxT || d.n_experts < 1 || d.n_experts > kMaxE || d.top_k < 1 ||
        d.top_k > kMaxK || d.top_k > d.n_experts || !moe_route_rows_supported(d.hidden) || !logits)
        return hipErrorInvalidValue;
    const unsigned parts = static_cast<unsigned>((d.n_experts + kRouteEPP - 1) / kRouteEPP);
    if (d.t <= 512)
        FOCR_LAUNCH(route_logits_kernel<4>, dim3(static_cast<unsigned>((d.t + 3) / 4), parts), dim3(256), 0, s,
                    hidden, router, d.t, d.hidden, d.n_experts, logits);
    else
        FOCR_LAUNCH(route_logits_kernel<8>, dim3(static_cast<unsigned>((d.t + 7) / 8), parts), dim3(256), 0, s,
                    hidden, router, d.t, d.hidden, d.n_experts, logits);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    FOCR_LAUNCH(route_rank_kernel, dim3(static_cast<unsigned>((d.t + 3) / 4)), dim3(256), 0, s, logits, d.t,
                d.n_experts, d.top_k, norm_topk, routed_scale, idx, gates, probs, flag);
    return hipGetLastError();
}

hipError_t launch_route_epoch_bump(hipStream_t s, void* xchg) {
    if (!xchg) return hipErrorInvalidValue;
    FOCR_LAUNCH(route_epoch_bump_kernel, dim3(1), dim3(64), 0, s, static_cast<RouteXchg*>(xchg));
    return hipGetLastError();
}

hipError_t launch_moe_gate_up(hipStream_t s, const MoeDims& d, const void* sel, const int8_t* xq, const float* xs,
                              const int8_t* wg, const float* sg, const int8_t* wu, const float* su, float* act,
                              int inter, bool shared, const MoeSharedGateUp* with_shared, void* route_xchg) {
    int lpr, jc;
    pick_lpr(d.hidden, &lpr, &jc);
    if (!dims_ok(d) || !sel || d.hidden % 16 != 0 || jc > 8) return hipErrorInvalidValue;
    const int rows_per_block = 256 / lpr;
    const int max_active = shared ? 1 : (d.n_experts < d.t * d.top_k ? d.n_experts : d.t * d.top_k);
    const int gx = (inter + rows_per_block - 1) / rows_per_block;
    SharedGU sh{};
    if (with_shared && !shared) {
        const int per = gx * rows_per_block;
        sh = SharedGU{with_shared->wg, with_shared->wu, with_shared->sg, with_shared->su, with_shared->act,
                      with_shared->inter, (with_shared->inter + per - 1) / per, nullptr};
    }
    sh.route_counter = route_xchg ? &static_cast<RouteXchg*>(route_xchg)->counter : nullptr;
    const dim3 grid(gx, max_active + sh.nslots);
    const int staged = d.t <= kAllTok ? d.t : kPairStage;
    const size_t lds = (static_cast<size_t>(staged) * d.hidden + 1023) & ~static_cast<size_t>(1023);
    const GemvArgs a{sel_of(const_cast<void*>(sel)), d.t, d.top_k, d.hidden, inter, shared ? d.t : 0};
    if (lpr == 16) return launch_gate_up_lpr<16>(s, grid, lds, jc, a, xq, xs, wg, sg, wu, su, act, sh);
    return launch_gate_up_lpr<8>(s, grid, lds, jc, a, xq, xs, wg, sg, wu, su, act, sh);
}

hipError_t launch_moe_down(hipStream_t s, const MoeDims& d, const void* sel, const float* act, const int8_t* wd,
                           const float* sd, float* ybuf, int inter, bool shared) {
    int lpr, jc;
    pick_lpr(inter, &lpr, &jc);
    if (!dims_ok(d) || !sel || inter % 16 != 0 || jc > 8) return hipErrorInvalidValue;
    const int rows_per_block = 256 / lpr;
    const int max_active = shared ? 1 : (d.n_experts < d.t * d.top_k ? d.n_experts : d.t * d.top_k);
    const dim3 grid((d.hidden + rows_per_block - 1) / rows_per_block, max_active);
    const size_t lds = static_cast<size_t>(kPairStage) * inter;
    const GemvArgs a{sel_of(const_cast<void*>(sel)), d.t, d.top_k, d.hidden, inter, shared ? d.t : 0};
    if (lpr == 16) return launch_down_lpr<16>(s, grid, lds, jc, a, act, wd, sd, ybuf);
    return launch_down_lpr<8>(s, grid, lds, jc, a, act, wd, sd, ybuf);
}

hipError_t launch_moe_combine(hipStream_t s, const MoeDims& d, const float* ybuf, const int* flag,
                              const float* shared_y, const float* resid, float* out) {
    if (!dims_ok(d) || d.hidden % 4 != 0) return hipErrorInvalidValue;
    const dim3 grid(static_cast<unsigned>((d.hidden / 4 + 255) / 256), static_cast<unsigned>(d.t));
    FOCR_LAUNCH(moe_combine_kernel, grid, dim3(256), 0, s, ybuf, flag, shared_y, resid, out, d.top_k, d.hidden);
    return hipGetLastError();
}

hipError_t launch_moe_down_combine(hipStream_t s, const MoeDims& d, const uint32_t* idx, const float* gates,
                                   const int* flag, const float* act, const int8_t* wd, const float* sd,
                                   const float* shared_y, const float* resid, float* out, int inter) {
    int lpr, jc;
    pick_lpr(inter, &lpr, &jc);
    if (!dims_ok(d) || inter % 16 != 0 || jc > 8) return hipErrorInvalidValue;
    // row blocks per token, a multiple of 8 (the extra ones have no rows)
    auto row_blocks = [&](int rpg) {
        const int R = rpg * (DC_THREADS / lpr) / d.top_k;
        return (((d.hidden + R - 1) / R) + 7) & ~7;
    };
    // two rows per lane group where one row each would need more blocks than
    // fit at once (768: three 8-wave blocks per CU at the one-row kernel's
    // registers; T = 8 needs 1024), so no second round of blocks pays the
    // whole id -> weight -> act latency chain again at the kernel's end
    const bool two_ok = (lpr == 8 && jc == 7) || (lpr == 16 && jc == 5);
    const int rpg = two_ok && d.t * row_blocks(1) > 768 ? 2 : 1;
    const int nrb8 = row_blocks(rpg);
    const dim3 grid(static_cast<unsigned>(d.t * nrb8));
    const size_t lds = static_cast<size_t>(d.top_k) * inter;
#define FOCR_DC(L, J, P)                                                                                          \
    if (lpr == L && jc == J && rpg == P) {                                                                       \
        FOCR_LAUNCH((moe_down_combine_kernel<L, J, P>), grid, dim3(DC_THREADS), lds, s, idx, gates, flag, d.t,   \
                    d.top_k, act, wd, sd, shared_y, resid, out, d.hidden, inter, d.n_experts);                   \
        return hipGetLastError();                                                                                \
    }
    FOCR_DC(8, 1, 1) FOCR_DC(8, 2, 1) FOCR_DC(8, 3, 1) FOCR_DC(8, 4, 1) FOCR_DC(8, 5, 1) FOCR_DC(8, 6, 1)
    FOCR_DC(8, 7, 1) FOCR_DC(8, 8, 1) FOCR_DC(16, 1, 1) FOCR_DC(16, 2, 1) FOCR_DC(16, 3, 1) FOCR_DC(16, 4, 1)
    FOCR_DC(16, 5, 1) FOCR_DC(16, 6, 1) FOCR_DC(16, 7, 1) FOCR_DC(16, 8, 1)
    FOCR_DC(8, 7, 2) FOCR_DC(16, 5, 2)
#undef FOCR_DC
    return hipErrorInvalidValue;
}

}  // namespace focr
