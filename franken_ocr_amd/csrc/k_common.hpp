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
__device__ __forceinline__ int reduce16_add(int v) {
    v += __shfl_xor(v, 8, 16);
    v += __shfl_xor(v, 4, 16);
    v += __shfl_xor(v, 2, 16);
    v += __shfl_xor(v, 1, 16);
    return v;
}

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

// decoder.rs:1079-1083 silu(x) = x / (1 + e^-x), accurate expf (no fast math).
__device__ __forceinline__ float silu_f(float x) { return x / (1.0f + expf(-x)); }

}  // namespace focr
