// k_gemv.hip — decode GEMV family on uploaded int8 weights:
//   * per-row activation quantization (decoder.rs:1588-1597 / :1647-1656),
//   * the int8 GEMV with the dequant epilogue y = ((f32)acc * a_s) * w_s
//     (decoder.rs:1621-1640, :2703-2747), optionally emitting per-block
//     argmax keys for the LM head (sampler.rs:168-186),
//   * the argmax reductions.
//
// HBM-bound design (ops/byte ~ 2M << the int8 ridge): 16 lanes per weight
// row, 16-byte coalesced loads, all of a lane's row chunks issued before the
// dot products, activations (M <= 32 rows) staged once per block in LDS and
// read as broadcast 16-byte LDS reads. Each block walks a contiguous range of
// 16-row tiles so the per-block prologue (staging xq) is amortised.
#include "focr_internal.hpp"
#include "k_common.hpp"

namespace focr {
namespace {

constexpr int kThreads = 256;
constexpr int kGroups = kThreads / 16;

__global__ __launch_bounds__(kThreads) void quantize_rows_kernel(const float* __restrict__ x, int K,
                                                                 int8_t* __restrict__ xq,
                                                                 float* __restrict__ a_scales,
                                                                 int ties_even) {
    __shared__ float red[kThreads / 64];
    const int row = blockIdx.x;
    block_quantize_row<kThreads>(x + static_cast<size_t>(row) * K, K, xq + static_cast<size_t>(row) * K,
                                 a_scales + row, ties_even != 0, red);
}

// JB = row chunks (16 B) a lane holds in flight per batch. BAN: output
// channel n of row i is written -inf when bit n of ban_bits[i] is set (the
// no-repeat-ngram ban folded into the dequant epilogue, decoder.rs:2319-2357).
template <int MC, int JB, bool BAN>
__global__ __launch_bounds__(kThreads) void gemv_i8_kernel(
    const int8_t* __restrict__ W, const float* __restrict__ ws, int N, int K,
    const int8_t* __restrict__ xq, const float* __restrict__ a_scales, int M,
    float* __restrict__ y, int32_t* __restrict__ acc_out, uint64_t* __restrict__ keys,
    int tiles_per_block, const uint32_t* __restrict__ ban_bits, int ban_words) {
    extern __shared__ int4 lds_x[];  // [MC][K/16]
    __shared__ uint64_t lds_keys[kGroups][MC];
    __shared__ float lds_as[MC];
    const int group = threadIdx.x >> 4;
    const int lane = threadIdx.x & 15;
    const int C = K >> 4;
    const int4* x4 = reinterpret_cast<const int4*>(xq);
    for (int i = threadIdx.x; i < M * C; i += kThreads) lds_x[i] = x4[i];
    if (threadIdx.x < MC) lds_as[threadIdx.x] = threadIdx.x < M ? a_scales[threadIdx.x] : 0.0f;
    __syncthreads();

    uint64_t best[MC];
#pragma unroll
    for (int i = 0; i < MC; ++i) best[i] = 0ull;

    const int tile0 = blockIdx.x * tiles_per_block;
    for (int t = 0; t < tiles_per_block; ++t) {
        const int n = (tile0 + t) * kGroups + group;
        if ((tile0 + t) * kGroups >= N) break;
        int acc[MC];
#pragma unroll
        for (int i = 0; i < MC; ++i) acc[i] = 0;
        if (n < N) {
            const int4* wrow = reinterpret_cast<const int4*>(W + static_cast<size_t>(n) * K);
            for (int cb = 0; cb < C; cb += 16 * JB) {
                int4 w[JB];
#pragma unroll
                for (int j = 0; j < JB; ++j) {
                    const int c = cb + lane + 16 * j;
                    w[j] = c < C ? ld_stream(wrow + c) : make_int4(0, 0, 0, 0);
                }
#pragma unroll
                for (int j = 0; j < JB; ++j) {
                    const int c = cb + lane + 16 * j;
                    if (c < C) {
#pragma unroll
                        for (int i = 0; i < MC; ++i)
                            if (i < M) acc[i] = dot16_i8(w[j], lds_x[i * C + c], acc[i]);
                    }
                }
            }
        }
        const float wscale = n < N ? ws[n] : 0.0f;
#pragma unroll
        for (int i = 0; i < MC; ++i) {
            const int v = reduce16_add(acc[i]);
            if (n < N && i < M && lane == (i & 15)) {
                const float t0 = static_cast<float>(v) * lds_as[i];
                float yv = t0 * wscale;
                if (BAN && ((ban_bits[static_cast<size_t>(i) * ban_words + (n >> 5)] >> (n & 31)) & 1u))
                    yv = -__builtin_inff();
                y[static_cast<size_t>(i) * N + n] = yv;
                if (acc_out) acc_out[static_cast<size_t>(i) * N + n] = v;
                if (keys) {
                    const uint64_t k = argmax_key(yv, static_cast<uint32_t>(n));
                    best[i] = k > best[i] ? k : best[i];
                }
            }
        }
    }
    if (keys) {
        // best[i] lives in lane (i & 15) of each group; fold the 16 groups.
#pragma unroll
        for (int i = 0; i < MC; ++i)
            if (lane == (i & 15)) lds_keys[group][i] = best[i];
        __syncthreads();
        if (threadIdx.x < M) {
            uint64_t b = 0ull;
            for (int g = 0; g < kGroups; ++g) b = lds_keys[g][threadIdx.x] > b ? lds_keys[g][threadIdx.x] : b;
            keys[static_cast<size_t>(threadIdx.x) * gridDim.x + blockIdx.x] = b;
        }
    }
}

// One block per row: fold nparts keys -> the argmax index.
__global__ __launch_bounds__(kThreads) void argmax_reduce_kernel(const uint64_t* __restrict__ keys,
                                                                 int nparts,
                                                                 uint32_t* __restrict__ argmax) {
    __shared__ uint64_t red[kThreads / 64];
    const int row = blockIdx.x;
    uint64_t b = 0ull;
    for (int i = threadIdx.x; i < nparts; i += kThreads) {
        const uint64_t k = keys[static_cast<size_t>(row) * nparts + i];
        b = k > b ? k : b;
    }
    b = wave_max_u64(b);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = b;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint64_t r = red[0];
        for (int i = 1; i < kThreads / 64; ++i) r = red[i] > r ? red[i] : r;
        argmax[row] = argmax_key_index(r);
    }
}

// Partial argmax keys over a logits matrix: grid (nparts, m). With ban_bits,
// a banned entry counts as -inf (sampler.rs:245-257 masked copy, then
// argmax_row) without writing the logits.
__global__ __launch_bounds__(kThreads) void argmax_partial_kernel(const float* __restrict__ logits,
                                                                  int n, uint64_t* __restrict__ keys,
                                                                  const uint32_t* __restrict__ ban_bits,
                                                                  int ban_words) {
    __shared__ uint64_t red[kThreads / 64];
    const int row = blockIdx.y;
    const float* lr = logits + static_cast<size_t>(row) * n;
    const uint32_t* bb = ban_bits ? ban_bits + static_cast<size_t>(row) * ban_words : nullptr;
    uint64_t b = 0ull;
    for (int i = blockIdx.x * kThreads + threadIdx.x; i < n; i += gridDim.x * kThreads) {
        float v = lr[i];
        if (bb && ((bb[i >> 5] >> (i & 31)) & 1u)) v = -__builtin_inff();
        const uint64_t k = argmax_key(v, static_cast<uint32_t>(i));
        b = k > b ? k : b;
    }
    b = wave_max_u64(b);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = b;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint64_t r = red[0];
        for (int i = 1; i < kThreads / 64; ++i) r = red[i] > r ? red[i] : r;
        keys[static_cast<size_t>(row) * gridDim.x + blockIdx.x] = r;
    }
}

int tiles_per_block_for(int n, int cu_count) {
    const int tiles = (n + kGroups - 1) / kGroups;
    // Aim for ~8 blocks per CU; keep at least one tile per block.
    const int target_blocks = (cu_count > 0 ? cu_count : 256) * 8;
    int tpb = (tiles + target_blocks - 1) / target_blocks;
    return tpb < 1 ? 1 : tpb;
}

}  // namespace

int gemv_i8_nparts(int n, int cu_count) {
    const int tiles = (n + kGroups - 1) / kGroups;
    const int tpb = tiles_per_block_for(n, cu_count);
    return (tiles + tpb - 1) / tpb;
}

hipError_t launch_quantize_rows(hipStream_t s, const float* x, int m, int k, int8_t* xq,
                                float* a_scales, bool ties_even) {
    if (m == 0) return hipSuccess;
    FOCR_LAUNCH(quantize_rows_kernel, dim3(m), dim3(kThreads), 0, s, x, k, xq, a_scales,
                       ties_even ? 1 : 0);
    return hipGetLastError();
}

hipError_t launch_gemv_i8(hipStream_t s, const int8_t* w, const float* ws, int n, int k,
                          const int8_t* xq, const float* a_scales, int m, float* y, int32_t* acc,
                          uint64_t* arg_keys, int* nparts_out, int cu_count) {
    return launch_gemv_i8_banned(s, w, ws, n, k, xq, a_scales, m, y, acc, arg_keys, nparts_out, cu_count, nullptr,
                                 0);
}

hipError_t launch_gemv_i8_banned(hipStream_t s, const int8_t* w, const float* ws, int n, int k,
                                 const int8_t* xq, const float* a_scales, int m, float* y, int32_t* acc,
                                 uint64_t* arg_keys, int* nparts_out, int cu_count, const uint32_t* ban_bits,
                                 int ban_words) {
    if (m < 1 || m > 32 || k % 16 != 0 || k <= 0) return hipErrorInvalidValue;
    if (ban_bits && ban_words * 32 < n) return hipErrorInvalidValue;
    const int tiles = (n + kGroups - 1) / kGroups;
    const int tpb = tiles_per_block_for(n, cu_count);
    const int grid = (tiles + tpb - 1) / tpb;
    if (nparts_out) *nparts_out = grid;
    const size_t lds = static_cast<size_t>(m) * k;
    if (lds > 57344) return hipErrorInvalidValue;
    int mc = 1;
    while (mc < m) mc <<= 1;
#define FOCR_GEMV_CASE(MCV)                                                                              \
    case MCV:                                                                                            \
        if (ban_bits)                                                                                    \
            FOCR_LAUNCH((gemv_i8_kernel<MCV, 8, true>), dim3(grid), dim3(kThreads), lds, s, w, ws, n, k, \
                        xq, a_scales, m, y, acc, arg_keys, tpb, ban_bits, ban_words);                    \
        else                                                                                             \
            FOCR_LAUNCH((gemv_i8_kernel<MCV, 8, false>), dim3(grid), dim3(kThreads), lds, s, w, ws, n,   \
                        k, xq, a_scales, m, y, acc, arg_keys, tpb, nullptr, 0);                          \
        break;
    switch (mc) {
        FOCR_GEMV_CASE(1)
        FOCR_GEMV_CASE(2)
        FOCR_GEMV_CASE(4)
        FOCR_GEMV_CASE(8)
        FOCR_GEMV_CASE(16)
        FOCR_GEMV_CASE(32)
        default:
            return hipErrorInvalidValue;
    }
#undef FOCR_GEMV_CASE
    return hipGetLastError();
}

hipError_t launch_argmax_reduce(hipStream_t s, const uint64_t* keys, int m, int nparts,
                                uint32_t* argmax) {
    if (m == 0) return hipSuccess;
    FOCR_LAUNCH(argmax_reduce_kernel, dim3(m), dim3(kThreads), 0, s, keys, nparts, argmax);
    return hipGetLastError();
}

hipError_t launch_argmax_rows(hipStream_t s, const float* logits, int m, int n, uint64_t* keys,
                              int nparts, uint32_t* argmax) {
    if (m == 0) return hipSuccess;
    hipError_t e = launch_argmax_partial(s, logits, m, n, keys, nparts, nullptr, 0);
    if (e != hipSuccess) return e;
    return launch_argmax_reduce(s, keys, m, nparts, argmax);
}

hipError_t launch_argmax_partial(hipStream_t s, const float* logits, int m, int n, uint64_t* keys, int nparts,
                                 const uint32_t* ban_bits, int ban_words) {
    if (m == 0) return hipSuccess;
    FOCR_LAUNCH(argmax_partial_kernel, dim3(nparts, m), dim3(kThreads), 0, s, logits, n, keys, ban_bits, ban_words);
    return hipGetLastError();
}

}  // namespace focr
