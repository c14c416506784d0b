// k_common.hpp — gfx950 device helpers shared by the kernel files.
//
// Wavefronts are 64 lanes. The int8 GEMV family assigns 16 lanes to one
// weight row: each lane streams 16-byte chunks of the row (global_load
// dwordx4), so one load instruction of a wave covers four 256-byte row
// segments, and the 16 partial i32 sums are reduced with four xor shuffles.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace focr {

__device__ __forceinline__ int dot4_i8(int a, int b, int c) {
    // v_dot4_i32_i8 without clamp: four signed byte products added to c,
    // wrapping in 32 bits exactly like the reference's release-mode i32 adds.
    return __builtin_amdgcn_sdot4(a, b, c, false);
}

__device__ __forceinline__ int dot16_i8(const int4& a, const int4& b, int c) {
    c = dot4_i8(a.x, b.x, c);
    c = dot4_i8(a.y, b.y, c);
    c = dot4_i8(a.z, b.z, c);
    c = dot4_i8(a.w, b.w, c);
    return c;
}

typedef int v4i_t __attribute__((ext_vector_type(4)));

// Streaming (read-once) 16-byte load: non-temporal hint so weight rows do
// not evict reusable lines (activations, scales) from the caches.
__device__ __forceinline__ int4 ld_stream(const int4* p) {
    const v4i_t v = __builtin_nontemporal_load(reinterpret_cast<const v4i_t*>(p));
    return make_int4(v.x, v.y, v.z, v.w);
}

// Sum across the 16 lanes of a row group (all 16 lanes end with the total).


__device__ __forceinline__ float wave_max_f(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

__device__ __forceinline__ double wave_sum_d(double v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// The same reductions through DPP row moves (VALU, a few cycles a step)
// and four v_readlane_b32, for call sites that run with every lane of the
// wave active; the shuffles above go through ds_bpermute at LDS latency, six
// dependent round trips per reduction. The max is exact in any order; the
// f64 sum adds pairs, quads, 8- and 16-lane rows, then the four rows, which
// is another order than the butterfly above (a different last bit at most).
template <int CTRL>
__device__ __forceinline__ int dpp_mov(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}

template <int CTRL>
__device__ __forceinline__ double dpp_mov_d(double v) {
    const unsigned long long u = static_cast<unsigned long long>(__double_as_longlong(v));
    const unsigned lo = static_cast<unsigned>(dpp_mov<CTRL>(static_cast<int>(u & 0xffffffffu)));
    const unsigned hi = static_cast<unsigned>(dpp_mov<CTRL>(static_cast<int>(u >> 32)));
    return __longlong_as_double(static_cast<long long>((static_cast<unsigned long long>(hi) << 32) | lo));
}

__device__ __forceinline__ double readlane_d(double v, int lane) {
    const unsigned long long u = static_cast<unsigned long long>(__double_as_longlong(v));
    const unsigned lo = static_cast<unsigned>(__builtin_amdgcn_readlane(static_cast<int>(u & 0xffffffffu), lane));
    const unsigned hi = static_cast<unsigned>(__builtin_amdgcn_readlane(static_cast<int>(u >> 32), lane));
    return __longlong_as_double(static_cast<long long>((static_cast<unsigned long long>(hi) << 32) | lo));
}

// Sum over aligned groups of LPR lanes (2, 4, 8 or 16), every lane of a
// group getting its sum, as an xor butterfly of width LPR would (integers:
// exact in any order). A disabled source lane reads as 0.
template <int LPR>
__device__ __forceinline__ int reduce_lanes(int v) {
    static_assert(LPR == 2 || LPR == 4 || LPR == 8 || LPR == 16, "groups within one 16-lane DPP row");
    v += dpp_mov<0xB1>(v);
    if constexpr (LPR >= 4) v += dpp_mov<0x4E>(v);
    if constexpr (LPR >= 8) v += dpp_mov<0x141>(v);
    if constexpr (LPR >= 16) v += dpp_mov<0x140>(v);
    return v;
}

__device__ __forceinline__ int reduce16_add(int v) { return reduce_lanes<16>(v); }

// DPP controls: quad_perm [1,0,3,2], quad_perm [2,3,0,1], row_half_mirror, row_mirror
__device__ __forceinline__ float wave_max_f_full(float v) {
    v = fmaxf(v, __int_as_float(dpp_mov<0xB1>(__float_as_int(v))));
    v = fmaxf(v, __int_as_float(dpp_mov<0x4E>(__float_as_int(v))));
    v = fmaxf(v, __int_as_float(dpp_mov<0x141>(__float_as_int(v))));
    v = fmaxf(v, __int_as_float(dpp_mov<0x140>(__float_as_int(v))));  // every lane: its 16-lane row's max
    const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}

// f32 sum over each 16-lane DPP row (every lane gets its row's sum; pairs,
// quads, halves, then the row), for the full-wave reductions below.
__device__ __forceinline__ float row16_sum_f(float v) {
    v += __int_as_float(dpp_mov<0xB1>(__float_as_int(v)));
    v += __int_as_float(dpp_mov<0x4E>(__float_as_int(v)));
    v += __int_as_float(dpp_mov<0x141>(__float_as_int(v)));
    v += __int_as_float(dpp_mov<0x140>(__float_as_int(v)));
    return v;
}

__device__ __forceinline__ float lane_f(float v, int lane) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

__device__ __forceinline__ float wave_sum_f_full(float v) {
    v = row16_sum_f(v);
    return ((lane_f(v, 0) + lane_f(v, 16)) + lane_f(v, 32)) + lane_f(v, 48);
}

__device__ __forceinline__ double wave_sum_d_full(double v) {
    v += dpp_mov_d<0xB1>(v);
    v += dpp_mov_d<0x4E>(v);
    v += dpp_mov_d<0x141>(v);
    v += dpp_mov_d<0x140>(v);  // every lane: its 16-lane row's sum
    return ((readlane_d(v, 0) + readlane_d(v, 16)) + readlane_d(v, 32)) + readlane_d(v, 48);
}

template <int CTRL>
__device__ __forceinline__ uint64_t dpp_mov_u64(uint64_t v) {
    const unsigned lo = static_cast<unsigned>(dpp_mov<CTRL>(static_cast<int>(v & 0xffffffffu)));
    const unsigned hi = static_cast<unsigned>(dpp_mov<CTRL>(static_cast<int>(v >> 32)));
    return (static_cast<uint64_t>(hi) << 32) | lo;
}

__device__ __forceinline__ uint64_t umax64(uint64_t a, uint64_t b) { return a > b ? a : b; }

// max over each 16-lane DPP row, every lane getting its row's max (keys
// ordered as u64, 0 the identity)
__device__ __forceinline__ uint64_t row16_max_u64(uint64_t v) {
    v = umax64(v, dpp_mov_u64<0xB1>(v));
    v = umax64(v, dpp_mov_u64<0x4E>(v));
    v = umax64(v, dpp_mov_u64<0x141>(v));
    return umax64(v, dpp_mov_u64<0x140>(v));
}

__device__ __forceinline__ uint64_t lane_u64(uint64_t v, int lane) {
    const unsigned lo = static_cast<unsigned>(__builtin_amdgcn_readlane(static_cast<int>(v & 0xffffffffu), lane));
    const unsigned hi = static_cast<unsigned>(__builtin_amdgcn_readlane(static_cast<int>(v >> 32), lane));
    return (static_cast<uint64_t>(hi) << 32) | lo;
}

__device__ __forceinline__ uint64_t wave_max_u64_full(uint64_t v) {
    v = row16_max_u64(v);
    return umax64(umax64(lane_u64(v, 0), lane_u64(v, 16)), umax64(lane_u64(v, 32), lane_u64(v, 48)));
}

__device__ __forceinline__ double wave_max_d(double v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmax(v, __shfl_xor(v, o, 64));
    return v;
}

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        uint64_t w = __shfl_xor(v, o, 64);
        v = w > v ? w : v;
    }
    return v;
}

// Argmax key: larger key = larger value, ties -> lower index. NaN -> 0
// ("no candidate"); -0.0 and +0.0 compare equal, as `v <= best` does in
// sampler.rs:180. Every non-NaN value maps to a key > 0.
__device__ __forceinline__ uint64_t argmax_key(float v, uint32_t idx) {
    if (v != v) return 0ull;
    if (v == 0.0f) v = 0.0f;
    uint32_t u = __float_as_uint(v);
    uint32_t ord = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return (static_cast<uint64_t>(ord) << 32) | static_cast<uint64_t>(0xFFFFFFFFu - idx);
}

__device__ __forceinline__ uint32_t argmax_key_index(uint64_t key) {
    return key ? 0xFFFFFFFFu - static_cast<uint32_t>(key & 0xFFFFFFFFull) : 0u;
}

__device__ __forceinline__ float key_value(uint64_t key) {
    uint32_t ord = static_cast<uint32_t>(key >> 32);
    uint32_t u = (ord & 0x80000000u) ? (ord & 0x7FFFFFFFu) : ~ord;
    return __uint_as_float(u);
}

// decoder.rs:1588-1597 (half away from zero) / :1647-1656 (ties even):
// clamp into [-127, 127], NaN -> 0 (Rust's saturating `as i8`).
__device__ __forceinline__ int8_t quant_i8(float v, float inv, bool ties_even) {
    float r = ties_even ? rintf(v * inv) : roundf(v * inv);
    if (r != r) return 0;
    r = fminf(fmaxf(r, -127.0f), 127.0f);
    return static_cast<int8_t>(static_cast<int>(r));
}

// The three row quantization rules, all with a_scale = max|x| / 127 (1.0 for
// an all-zero row) and a clamp into [-127, 127]:
//   kQuantHalfAway  quantize_row_i8 (decoder.rs:1588-1597): x * (1 / a_scale), half away from zero;
//   kQuantTiesEven  quantize_row_i8_te (decoder.rs:1647-1656): x * (1 / a_scale), ties to even;
//   kQuantDynamic   the dynamic activation rule of linear_int8_dynamic
//                   (docs/focrq-format.md:296-320): x / a_scale (true division), ties to even.
enum QuantRule : int { kQuantHalfAway = 0, kQuantTiesEven = 1, kQuantDynamic = 2 };

__device__ __forceinline__ int8_t quant_rule(float v, float a_scale, float inv, int rule) {
    if (rule == kQuantDynamic) {
        float r = v / a_scale;
        if (r != r) return 0;
        r = fminf(fmaxf(r, -127.0f), 127.0f);
        return static_cast<int8_t>(static_cast<int>(rintf(r)));
    }
    return quant_i8(v, inv, rule == kQuantTiesEven);
}

// One row by a whole block of THREADS lanes: amax = max|x|, a_scale, q by
// `rule` (a QuantRule). red holds THREADS / 64 floats of LDS.
template <int THREADS>
__device__ __forceinline__ void block_quantize_row(const float* __restrict__ xr, int K, int8_t* __restrict__ q,
                                                   float* __restrict__ a_scale_out, int rule, float* red) {
    float amax = 0.0f;
    for (int i = threadIdx.x; i < K; i += THREADS) amax = fmaxf(amax, fabsf(xr[i]));
    amax = wave_max_f(amax);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = amax;
    __syncthreads();
    amax = red[0];
#pragma unroll
    for (int w = 1; w < THREADS / 64; ++w) amax = fmaxf(amax, red[w]);
    const float a_scale = amax > 0.0f ? amax / 127.0f : 1.0f;
    const float inv = 1.0f / a_scale;
    for (int i = threadIdx.x; i < K; i += THREADS) q[i] = quant_rule(xr[i], a_scale, inv, rule);
    if (threadIdx.x == 0) *a_scale_out = a_scale;
}

// The same with the row held in registers: thread t takes float4 chunks
// t + THREADS j (j < NC; K % 4 == 0, 4 THREADS NC >= K, xr 16-byte and q
// 4-byte aligned), every load issued before the first use, the amax from
// registers (DPP wave max), the codes stored four to a word. Same quant_rule,
// same amax (order-free), so the same bytes and scale as block_quantize_row,
// whose strided loop waits for each load in turn.
template <int THREADS, int NC>
__device__ __forceinline__ void block_quantize_row_vec(const float* __restrict__ xr, int K, int8_t* __restrict__ q,
                                                       float* __restrict__ a_scale_out, int rule, float* red) {
    const int K4 = K >> 2;
    const float4* x4 = reinterpret_cast<const float4*>(xr);
    float4 v[NC];
    float amax = 0.0f;
#pragma unroll
    for (int j = 0; j < NC; ++j) {
        const int c = static_cast<int>(threadIdx.x) + THREADS * j;
        const float4 t = x4[c < K4 ? c : K4 - 1];  // past the row: its last chunk again (unused)
        v[j] = t;
        if (c < K4) amax = fmaxf(amax, fmaxf(fmaxf(fabsf(t.x), fabsf(t.y)), fmaxf(fabsf(t.z), fabsf(t.w))));
    }
    amax = wave_max_f_full(amax);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = amax;
    __syncthreads();
    amax = red[0];
#pragma unroll
    for (int w = 1; w < THREADS / 64; ++w) amax = fmaxf(amax, red[w]);
    const float a_scale = amax > 0.0f ? amax / 127.0f : 1.0f;
    const float inv = 1.0f / a_scale;
    char4* q4 = reinterpret_cast<char4*>(q);
#pragma unroll
    for (int j = 0; j < NC; ++j) {
        const int c = static_cast<int>(threadIdx.x) + THREADS * j;
        if (c < K4) {
            char4 o;
            o.x = quant_rule(v[j].x, a_scale, inv, rule);
            o.y = quant_rule(v[j].y, a_scale, inv, rule);
            o.z = quant_rule(v[j].z, a_scale, inv, rule);
            o.w = quant_rule(v[j].w, a_scale, inv, rule);
            q4[c] = o;
        }
    }
    if (threadIdx.x == 0) *a_scale_out = a_scale;
}

// This thread's maximum over keys kr[t + THREADS i] (i >= 0, < n): U loads
// in flight at once (a strided loop waits for each in turn); past the end a
// key is read again, which leaves a maximum as it is.
template <int THREADS, int U = 8>
__device__ __forceinline__ uint64_t thread_max_keys(const uint64_t* __restrict__ kr, int n) {
    uint64_t b = 0ull;
    for (int i0 = static_cast<int>(threadIdx.x); i0 < n; i0 += U * THREADS) {
        uint64_t k[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int i = i0 + u * THREADS;
            k[u] = kr[i < n ? i : n - 1];
        }
#pragma unroll
        for (int u = 0; u < U; ++u) b = k[u] > b ? k[u] : b;
    }
    return b;
}

// decoder.rs:1079-1083 silu(x) = x / (1 + e^-x), accurate expf (no fast math).
__device__ __forceinline__ float silu_f(float x) { return x / (1.0f + expf(-x)); }
// SiLU from the hardware exp2 and reciprocal (v_exp_f32, v_rcp_f32, about
// 1 ulp each; the argument's rounding adds |x| * 2^-24 relative): a few
// ulp from silu_f in 5 VALU instead of ~30, for VALU-bound epilogues whose
// output is requantized to int8 (an ulp moves a code only on a rounding
// boundary). -inf / +inf / NaN behave as silu_f's.
__device__ __forceinline__ float silu_fast(float x) {
    return x * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(x * -1.4426950408889634f));
}

// The activation order of the 256 x 128 int8 GEMM (k_i8gemm.hip): rows in
// tiles of 256, each tile stored stage by stage (64 K bytes), each stage as
// 256 rows of 64 bytes with the 16-byte piece p of row r at slot
// p ^ ((r / 4) & 3) (its LDS image). Byte offset of K piece p of row r, nst
// = K / 64 stages. Written by the quantizers that feed that GEMM.
constexpr int kI8TiledRows = 256;
constexpr int kI8TiledStage = 64;
__device__ __forceinline__ int i8_tiled_swz(int r) { return (r >> 2) & 3; }
__device__ __forceinline__ size_t i8_tiled_act_off(int r, int p, int nst) {
    const int t = r / kI8TiledRows, rr = r % kI8TiledRows, st = p >> 2, sl = (p & 3) ^ i8_tiled_swz(rr);
    return ((static_cast<size_t>(t) * nst + st) * kI8TiledRows + rr) * kI8TiledStage + 16 * sl;
}

}  // namespace focr
