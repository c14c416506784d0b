// k_quant.hip — weight-side conversions run once at load / convert time:
// widening of stored F32/F16/BF16 payloads to f32, the per-output-channel
// int8 weight quantizer, and the per-group int4 packer. They run on the
// device so that a multi-hundred-MB tensor is copied to HBM once, raw, and
// converted there.
//
// Both quantizers use true division w / scale with round-half-to-even
// (src/quant/int8.rs:104-131, src/quant/int4.rs:142-205); the host-side
// activation quantizers elsewhere multiply by a reciprocal and must not be
// used here.
#include <algorithm>

#include "focr_internal.hpp"
#include "k_common.hpp"

namespace focr {
namespace {

// Element i of a stored payload of dtype dt (FOCR_HIP_DT_F32/F16/BF16),
// widened exactly to f32.
__device__ __forceinline__ float load_widened(const void* src, int dt, size_t i) {
    if (dt == FOCR_HIP_DT_F32) return reinterpret_cast<const float*>(src)[i];
    const uint16_t h = reinterpret_cast<const uint16_t*>(src)[i];
    if (dt == FOCR_HIP_DT_BF16) return __uint_as_float(static_cast<uint32_t>(h) << 16);
    return static_cast<float>(__builtin_bit_cast(_Float16, h));
}

// Saturating narrow of an already-rounded value: NaN -> 0, as Rust's
// `r.clamp(lo, hi) as i32 as i8` does.
__device__ __forceinline__ int clamp_round(float r, float lo, float hi) {
    if (r != r) return 0;
    return static_cast<int>(fminf(fmaxf(r, lo), hi));
}

// src/quant/int8.rs:104-131 quantize_row over every row: one wave per row.
// max|w| folds with fmaxf, which skips NaN as f32::max does; an all-zero row
// stores scale 1.0 and zero codes.
__global__ void __launch_bounds__(256) quant_weight_i8_kernel(const void* __restrict__ src, int dt, int n, int k,
                                                              int8_t* __restrict__ q, float* __restrict__ scales) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= n) return;
    const size_t base = static_cast<size_t>(row) * k;
    float mx = 0.0f;
    for (int i = lane; i < k; i += 64) mx = fmaxf(mx, fabsf(load_widened(src, dt, base + i)));
    mx = wave_max_f(mx);
    if (mx == 0.0f) {
        for (int i = lane; i < k; i += 64) q[base + i] = 0;
        if (lane == 0) scales[row] = 1.0f;
        return;
    }
    const float s = mx / 127.0f;
    for (int i = lane; i < k; i += 64)
        q[base + i] = static_cast<int8_t>(clamp_round(rintf(load_widened(src, dt, base + i) / s), -127.0f, 127.0f));
    if (lane == 0) scales[row] = s;
}

// src/quant/int4.rs:142-205 pack_int4_f32: one thread per (row, group).
// scale = max|g| / 7 (all-zero group: 1.0); q = clamp(rne(w / scale), -8, 7);
// byte j of the row = q[2j] & 0xF | (q[2j+1] & 0xF) << 4.
__global__ void __launch_bounds__(256) pack_weight_i4_kernel(const void* __restrict__ src, int dt, int n, int k,
                                                             int group, uint8_t* __restrict__ packed,
                                                             float* __restrict__ scales) {
    const int groups = k / group;
    const long gid = static_cast<long>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (gid >= static_cast<long>(n) * groups) return;
    const int row = static_cast<int>(gid / groups), g = static_cast<int>(gid % groups);
    const size_t base = static_cast<size_t>(row) * k + static_cast<size_t>(g) * group;
    float mx = 0.0f;
    for (int i = 0; i < group; ++i) mx = fmaxf(mx, fabsf(load_widened(src, dt, base + i)));
    const float s = mx == 0.0f ? 1.0f : mx / 7.0f;
    scales[gid] = s;
    uint8_t* out = packed + base / 2;
    for (int i = 0; i < group; i += 2) {
        const int lo = clamp_round(rintf(load_widened(src, dt, base + i) / s), -8.0f, 7.0f);
        const int hi = clamp_round(rintf(load_widened(src, dt, base + i + 1) / s), -8.0f, 7.0f);
        out[i / 2] = static_cast<uint8_t>((lo & 0xF) | ((hi & 0xF) << 4));
    }
}

__global__ void __launch_bounds__(256) widen_kernel(const void* __restrict__ src, int dt, size_t count,
                                                    float* __restrict__ dst) {
    const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
    for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < count; i += stride)
        dst[i] = load_widened(src, dt, i);
}

}  // namespace

hipError_t launch_quant_weight_i8(hipStream_t s, const void* src, int dt, int n, int k, int8_t* q, float* scales) {
    if (n <= 0 || k <= 0) return hipSuccess;
    FOCR_LAUNCH(quant_weight_i8_kernel, dim3((n + 3) / 4), dim3(256), 0, s, src, dt, n, k, q, scales);
    return hipGetLastError();
}

hipError_t launch_pack_weight_i4(hipStream_t s, const void* src, int dt, int n, int k, int group, uint8_t* packed,
                                 float* scales) {
    const long units = static_cast<long>(n) * (k / group);
    if (units <= 0) return hipSuccess;
    FOCR_LAUNCH(pack_weight_i4_kernel, dim3(static_cast<unsigned>((units + 255) / 256)), dim3(256), 0, s, src, dt, n,
                k, group, packed, scales);
    return hipGetLastError();
}

hipError_t launch_widen(hipStream_t s, const void* src, int dt, size_t count, float* dst) {
    if (count == 0) return hipSuccess;
    const size_t blocks = std::min<size_t>((count + 255) / 256, 8192);
    FOCR_LAUNCH(widen_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s, src, dt, count, dst);
    return hipGetLastError();
}

}  // namespace focr
