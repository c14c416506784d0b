// k_int4.hip — int4 x int8 kernels (simd/int4.rs contract):
//   * unpack: [n, k/2] packed -> [n, k] i8 (int4.rs:125-142),
//   * the drop-in packed GEMM (int4.rs:304-343): per (m, n), per group in
//     increasing order, the i32 group dot then acc_f = acc_f + s * f32(acc_i)
//     with a separate multiply and add (the library is built with
//     -ffp-contract=off), so the f32 result is bit-identical to the scalar
//     reference; optional per-group i32 partials for the parity tests.
//
// Nibble unpack in registers: for four packed bytes B, lo = B & 0x0F0F0F0F
// and hi = (B >> 4) & 0x0F0F0F0F; v_perm_b32 interleaves them into
// [lo0 hi0 lo1 hi1] / [lo2 hi2 lo3 hi3]; a nibble n is sign-extended inside
// its byte by OR-ing 0xF0 when bit 3 is set (no carries cross bytes).
#include "focr_internal.hpp"
#include "k_common.hpp"
#include "k_int4.hpp"

namespace focr {
namespace {

__global__ __launch_bounds__(256) void unpack_i4_kernel(const uint8_t* __restrict__ b, size_t nbytes,
                                                        int8_t* __restrict__ out) {
    const size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= nbytes) return;
    const uint8_t v = b[i];
    out[2 * i] = static_cast<int8_t>(static_cast<int8_t>(static_cast<uint8_t>(v << 4)) >> 4);
    out[2 * i + 1] = static_cast<int8_t>(static_cast<int8_t>(v) >> 4);
}

// One wave = 64 activation rows of one output channel n: the weight row and
// its scales are read once per wave (uniform addresses), each lane walks its
// own activation row.
__global__ __launch_bounds__(64) void s4s8_packed_kernel(const int8_t* __restrict__ A,
                                                         const uint8_t* __restrict__ B,
                                                         const float* __restrict__ scales,
                                                         int group, int M, int K, int N,
                                                         float* __restrict__ out,
                                                         int32_t* __restrict__ partials) {
    const int n = blockIdx.x;
    const int m = blockIdx.y * 64 + threadIdx.x;
    if (m >= M) return;
    const int groups = K / group;
    const uint32_t* brow = reinterpret_cast<const uint32_t*>(B + static_cast<size_t>(n) * (K / 2));
    const uint32_t* arow = reinterpret_cast<const uint32_t*>(A + static_cast<size_t>(m) * K);
    const float* srow = scales + static_cast<size_t>(n) * groups;
    float acc_f = 0.0f;
    for (int g = 0; g < groups; ++g) {
        int acc_i = 0;
        // 8 weights (4 packed bytes) and 8 activations per step
        for (int kk = g * group; kk < (g + 1) * group; kk += 8) {
            uint32_t wlo, whi;
            unpack8_i4(brow[kk >> 3], wlo, whi);
            acc_i = dot4_i8(static_cast<int>(arow[kk >> 2]), static_cast<int>(wlo), acc_i);
            acc_i = dot4_i8(static_cast<int>(arow[(kk >> 2) + 1]), static_cast<int>(whi), acc_i);
        }
        if (partials) partials[(static_cast<size_t>(m) * N + n) * groups + g] = acc_i;
        const float prod = srow[g] * static_cast<float>(acc_i);
        acc_f = acc_f + prod;
    }
    out[static_cast<size_t>(m) * N + n] = acc_f;
}

}  // namespace

hipError_t launch_unpack_i4(hipStream_t s, const uint8_t* b, size_t nbytes, int8_t* out) {
    if (nbytes == 0) return hipSuccess;
    const size_t grid = (nbytes + 255) / 256;
    FOCR_LAUNCH(unpack_i4_kernel, dim3(static_cast<unsigned>(grid)), dim3(256), 0, s, b, nbytes, out);
    return hipGetLastError();
}

hipError_t launch_s4s8_packed(hipStream_t s, const int8_t* a, const uint8_t* b,
                              const float* scales, int group, int m, int k, int n, float* out,
                              int32_t* partials) {
    if (m == 0 || n == 0) return hipSuccess;
    if (k % 16 != 0 || (group != 16 && group != 32) || k % group != 0) return hipErrorInvalidValue;
    const dim3 grid(n, (m + 63) / 64);
    FOCR_LAUNCH(s4s8_packed_kernel, grid, dim3(64), 0, s, a, b, scales, group, m, k, n, out,
                       partials);
    return hipGetLastError();
}

}  // namespace focr
