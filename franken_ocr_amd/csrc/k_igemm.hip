// k_igemm.hip — the drop-in int8 tier: out[M,N] += A[M,K] . B[N,K]^T in i32
// (simd::igemm_s8s8 / igemm_u8s8, scalar.rs:78-166).
//
// B is output-channel-major, so each output channel is one contiguous weight
// row. A 256-thread block is 16 row groups of 16 lanes; a group owns one
// output channel, each lane streams 16-byte chunks of the row and multiplies
// them against up to MC activation rows staged in LDS with v_dot4_i32_i8.
// U8S8 runs the signed dot on (a ^ 0x80) = a - 128 and adds 128 * sum(b), an
// identity that holds in wrapping i32 arithmetic, so results equal the
// scalar oracle bit for bit even where the oracle's i32 sum wraps.
#include "focr_internal.hpp"
#include "k_common.hpp"

namespace focr {
namespace {

constexpr int kThreads = 256;
constexpr int kGroups = kThreads / 16;
// s8s8 products of up to this many rows (two 16-row passes) go to the
// matrix-core split-K GEMV (each pass reads the weights once; the sdot4
// kernel below spends one VALU dot per 4 weight bytes per row)
constexpr int kMfmaMaxRows = 32;

// blockIdx.y selects one of a batch of independent instances, A, B and out
// advanced by sa, sb, so elements (0 for a single product).
template <bool kU8, int MC>
__global__ __launch_bounds__(kThreads) void igemm_vec_kernel(const int8_t* __restrict__ A,
                                                             const int8_t* __restrict__ B,
                                                             int32_t* __restrict__ out, int M,
                                                             int K, int N, size_t sa, size_t sb,
                                                             size_t so) {
    extern __shared__ int4 lds_a[];  // [MC][K/16]
    A += blockIdx.y * sa;
    B += blockIdx.y * sb;
    out += blockIdx.y * so;
    const int group = threadIdx.x >> 4;
    const int lane = threadIdx.x & 15;
    const int C = K >> 4;
    for (int m0 = 0; m0 < M; m0 += MC) {
        const int mc = min(MC, M - m0);
        __syncthreads();
        const int4* a4 = reinterpret_cast<const int4*>(A + static_cast<size_t>(m0) * K);
        for (int i = threadIdx.x; i < mc * C; i += kThreads) {
            int4 v = a4[i];
            if (kU8) {
                v.x ^= 0x80808080;
                v.y ^= 0x80808080;
                v.z ^= 0x80808080;
                v.w ^= 0x80808080;
            }
            lds_a[i] = v;
        }
        __syncthreads();
        for (int n0 = blockIdx.x * kGroups; n0 < N; n0 += gridDim.x * kGroups) {
            const int n = n0 + group;
            int acc[MC];
#pragma unroll
            for (int i = 0; i < MC; ++i) acc[i] = 0;
            int bsum = 0;
            if (n < N) {
                const int4* brow = reinterpret_cast<const int4*>(B + static_cast<size_t>(n) * K);
                for (int c = lane; c < C; c += 16) {
                    const int4 w = brow[c];
                    if (kU8) bsum = dot16_i8(w, make_int4(0x01010101, 0x01010101, 0x01010101, 0x01010101), bsum);
#pragma unroll
                    for (int i = 0; i < MC; ++i)
                        if (i < mc) acc[i] = dot16_i8(w, lds_a[i * C + c], acc[i]);
                }
            }
            if (kU8) bsum = reduce16_add(bsum);
#pragma unroll
            for (int i = 0; i < MC; ++i) {
                int v = reduce16_add(acc[i]);
                if (kU8) v = static_cast<int>(static_cast<uint32_t>(v) + 128u * static_cast<uint32_t>(bsum));
                if (n < N && i < mc && lane == (i & 15)) {
                    int32_t* o = out + static_cast<size_t>(m0 + i) * N + n;
                    *o = static_cast<int32_t>(static_cast<uint32_t>(*o) + static_cast<uint32_t>(v));
                }
            }
        }
    }
}

// Any K, any alignment (the self-test's K-tail shapes): lanes stride bytes.
template <bool kU8>
__global__ __launch_bounds__(kThreads) void igemm_byte_kernel(const int8_t* __restrict__ A,
                                                              const int8_t* __restrict__ B,
                                                              int32_t* __restrict__ out, int M,
                                                              int K, int N) {
    const int group = threadIdx.x >> 4;
    const int lane = threadIdx.x & 15;
    for (int n0 = blockIdx.x * kGroups; n0 < N; n0 += gridDim.x * kGroups) {
        const int n = n0 + group;
        for (int m = 0; m < M; ++m) {
            uint32_t acc = 0;
            if (n < N) {
                const int8_t* brow = B + static_cast<size_t>(n) * K;
                const int8_t* arow = A + static_cast<size_t>(m) * K;
                for (int k = lane; k < K; k += 16) {
                    const int a = kU8 ? static_cast<int>(static_cast<uint8_t>(arow[k])) : static_cast<int>(arow[k]);
                    acc += static_cast<uint32_t>(a * static_cast<int>(brow[k]));
                }
            }
            int v = reduce16_add(static_cast<int>(acc));
            if (n < N && lane == 0) {
                int32_t* o = out + static_cast<size_t>(m) * N + n;
                *o = static_cast<int32_t>(static_cast<uint32_t>(*o) + static_cast<uint32_t>(v));
            }
        }
    }
}

template <bool kU8>
hipError_t launch_vec(hipStream_t s, const int8_t* a, const int8_t* b, int32_t* out, int m, int k,
                      int n, int batch = 1) {
    const int tiles = (n + kGroups - 1) / kGroups;
    const int grid = tiles < 4096 ? tiles : 4096;
    // Stage up to 32 rows, keeping LDS at or under 64 KiB.
    int mc = 32;
    while (mc > 1 && static_cast<size_t>(mc) * k > 65536) mc >>= 1;
    if (mc > 1 && m < mc) {
        int p = 1;
        while (p < m) p <<= 1;
        mc = p;
    }
    const size_t lds = static_cast<size_t>(mc) * k;
#define FOCR_IGEMM_CASE(MCV)                                                                   \
    case MCV:                                                                                  \
        FOCR_LAUNCH((igemm_vec_kernel<kU8, MCV>), dim3(grid, batch), dim3(kThreads), lds, s, a, \
                    b, out, m, k, n, static_cast<size_t>(m) * k, static_cast<size_t>(n) * k,      \
                    static_cast<size_t>(m) * n);                                                  \
        break;
    switch (mc) {
        FOCR_IGEMM_CASE(1)
        FOCR_IGEMM_CASE(2)
        FOCR_IGEMM_CASE(4)
        FOCR_IGEMM_CASE(8)
        FOCR_IGEMM_CASE(16)
        FOCR_IGEMM_CASE(32)
        default:
            return hipErrorInvalidValue;
    }
#undef FOCR_IGEMM_CASE
    return hipGetLastError();
}

}  // namespace

hipError_t launch_igemm_i8_batched(hipStream_t s, const int8_t* a, const int8_t* b, int32_t* out, int batch, int m,
                                   int k, int n) {
    if (batch == 0 || m == 0 || n == 0) return hipSuccess;
    if (batch < 0 || batch > 65535 || k <= 0 || k % 16 || k > 65536 ||
        reinterpret_cast<uintptr_t>(a) % 16 || reinterpret_cast<uintptr_t>(b) % 16)
        return hipErrorInvalidValue;
    if (m <= kMfmaMaxRows) {  // 2..32 rows: the matrix-core split-K GEMV
        const hipError_t e = launch_igemm_i8_mfma(s, a, b, out, batch, m, k, n);
        if (e != hipErrorNotSupported) return e;
    }
    return launch_vec<false>(s, a, b, out, m, k, n, batch);
}

hipError_t launch_igemm_i8(hipStream_t s, const void* a, bool a_unsigned, const int8_t* b,
                           int32_t* out, int m, int k, int n) {
    if (m == 0 || n == 0) return hipSuccess;
    const int8_t* a8 = static_cast<const int8_t*>(a);
    const bool aligned = (reinterpret_cast<uintptr_t>(a8) % 16 == 0) &&
                         (reinterpret_cast<uintptr_t>(b) % 16 == 0);
    if (!a_unsigned && aligned && m <= kMfmaMaxRows) {  // 2..32 rows: the matrix-core split-K GEMV
        const hipError_t e = launch_igemm_i8_mfma(s, a8, b, out, 1, m, k, n);
        if (e != hipErrorNotSupported) return e;
    }
    if (k > 0 && k % 16 == 0 && aligned && k <= 65536) {
        return a_unsigned ? launch_vec<true>(s, a8, b, out, m, k, n)
                          : launch_vec<false>(s, a8, b, out, m, k, n);
    }
    const int tiles = (n + kGroups - 1) / kGroups;
    const int grid = tiles < 4096 ? tiles : 4096;
    if (a_unsigned)
        FOCR_LAUNCH(igemm_byte_kernel<true>, dim3(grid), dim3(kThreads), 0, s, a8, b, out, m, k, n);
    else
        FOCR_LAUNCH(igemm_byte_kernel<false>, dim3(grid), dim3(kThreads), 0, s, a8, b, out, m, k, n);
    return hipGetLastError();
}

}  // namespace focr
