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
#include <atomic>

#include "focr_internal.hpp"
#include "k_common.hpp"

namespace focr {
namespace {

constexpr int kThreads = 256;
constexpr int kGroups = kThreads / 16;

__global__ __launch_bounds__(kThreads) void quantize_rows_kernel(const float* __restrict__ x, int K,
                                                                 int8_t* __restrict__ xq,
                                                                 float* __restrict__ a_scales,
                                                                 int rule) {
    __shared__ float red[kThreads / 64];
    const int row = blockIdx.x;
    block_quantize_row<kThreads>(x + static_cast<size_t>(row) * K, K, xq + static_cast<size_t>(row) * K,
                                 a_scales + row, rule, red);
}

// The same per row with the row held in registers: thread t takes float4
// chunks t + 256 j (j < NC, 1024 NC >= K), all loads issued at once, the amax
// from registers (DPP wave max), the codes stored four to a word. Same
// quant_rule, same amax (order-free), so the same bytes and scale; the
// strided one-float loop above made a 6848-wide row take ~15 us.
template <int NC>
__global__ __launch_bounds__(kThreads) void quantize_rows_vec_kernel(const float* __restrict__ x, int K,
                                                                     int8_t* __restrict__ xq,
                                                                     float* __restrict__ a_scales, int rule) {
    __shared__ float red[kThreads / 64];
    const int row = blockIdx.x;
    block_quantize_row_vec<kThreads, NC>(x + static_cast<size_t>(row) * K, K, xq + static_cast<size_t>(row) * K,
                                         a_scales + row, rule, red);
}

// Two row sets in one launch (blocks [0, r1.m) the first, the rest the
// second), each row exactly as quantize_rows_vec_kernel does it: the MoE
// block's routed and shared act rows, whose widths differ.
template <int NC>
__global__ __launch_bounds__(kThreads) void quantize_rows2_vec_kernel(QuantRows r1, QuantRows r2, int rule) {
    __shared__ float red[kThreads / 64];
    const bool first = static_cast<int>(blockIdx.x) < r1.m;  // block-uniform
    const QuantRows r = first ? r1 : r2;
    const int row = first ? static_cast<int>(blockIdx.x) : static_cast<int>(blockIdx.x) - r1.m;
    block_quantize_row_vec<kThreads, NC>(r.x + static_cast<size_t>(row) * r.K, r.K,
                                         r.xq + static_cast<size_t>(row) * r.K, r.scales + row, rule, red);
}

// JB = row chunks (16 B) a lane holds in flight per batch; R = weight rows a
// 16-lane group computes per activation chunk it reads from LDS (LDS bytes
// per weight byte = M / R: at M = 8 the one-row form is LDS-bound). A tile
// is 16 * R rows: row base + r * 16 + group, so every load instruction of a
// wave covers four adjacent rows, 256 contiguous bytes each. BAN: output
// channel n of row i is written -inf when bit n of ban_bits[i] is set (the
// no-repeat-ngram ban folded into the dequant epilogue, decoder.rs:2319-2357).
// FQ (MC = 1): the row comes as f32 (xf, K % 4 == 0, K <= 2048) and each
// block quantizes it itself (quantize_row_i8, half away: the bytes and scale
// of quantize_rows_vec_kernel) — the separate quantize launch goes away.
template <int MC, int JB, int R, bool BAN, bool FQ = false>
__global__ __launch_bounds__(kThreads) void gemv_i8_kernel(
    const int8_t* __restrict__ W, const float* __restrict__ ws, int N, int K,
    const int8_t* __restrict__ xq, const float* __restrict__ a_scales, int M,
    float* __restrict__ y, int32_t* __restrict__ acc_out, uint64_t* __restrict__ keys,
    int tiles_per_block, const uint32_t* __restrict__ ban_bits, int ban_words, const float* __restrict__ xf) {
    static_assert(!FQ || MC == 1, "f32 input: one row");
    extern __shared__ int4 lds_x[];  // [MC][K/16]
    __shared__ uint64_t lds_keys[kGroups][MC];
    __shared__ float lds_as[MC];
    constexpr int MB = MC > 16 ? MC / 16 : 1;  // rows i a lane writes: lane == (i & 15)
    const int group = threadIdx.x >> 4;
    const int lane = threadIdx.x & 15;
    const int C = K >> 4;
    if constexpr (FQ) {
        __shared__ float red[kThreads / 64];
        const int K4 = K >> 2;
        const float4* xr4 = reinterpret_cast<const float4*>(xf);
        float4 v[2];
        float amax = 0.0f;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int c = static_cast<int>(threadIdx.x) + kThreads * j;
            v[j] = xr4[c < K4 ? c : K4 - 1];
            if (c < K4) amax = fmaxf(amax, fmaxf(fmaxf(fabsf(v[j].x), fabsf(v[j].y)), fmaxf(fabsf(v[j].z), fabsf(v[j].w))));
        }
        amax = wave_max_f_full(amax);
        if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = amax;
        __syncthreads();
        amax = red[0];
#pragma unroll
        for (int wv = 1; wv < kThreads / 64; ++wv) amax = fmaxf(amax, red[wv]);
        const float a_scale = amax > 0.0f ? amax / 127.0f : 1.0f;
        const float inv = 1.0f / a_scale;
        char4* q4 = reinterpret_cast<char4*>(lds_x);
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int c = static_cast<int>(threadIdx.x) + kThreads * j;
            if (c < K4) {
                char4 o;
                o.x = quant_i8(v[j].x, inv, false);
                o.y = quant_i8(v[j].y, inv, false);
                o.z = quant_i8(v[j].z, inv, false);
                o.w = quant_i8(v[j].w, inv, false);
                q4[c] = o;
            }
        }
        if (threadIdx.x == 0) lds_as[0] = a_scale;
    } else {
        const int4* x4 = reinterpret_cast<const int4*>(xq);
        for (int i = threadIdx.x; i < M * C; i += kThreads) lds_x[i] = x4[i];
        if (threadIdx.x < MC) lds_as[threadIdx.x] = threadIdx.x < M ? a_scales[threadIdx.x] : 0.0f;
    }
    __syncthreads();

    // the argmax key of row i is kept by lane i & 15 only: best[i >> 4]
    uint64_t best[MB];
#pragma unroll
    for (int q = 0; q < MB; ++q) best[q] = 0ull;

    const int tile0 = blockIdx.x * tiles_per_block;
    for (int t = 0; t < tiles_per_block; ++t) {
        const int base = (tile0 + t) * kGroups * R;
        if (base >= N) break;
        // ban words of this lane's outputs, fetched ahead of the weights
        uint32_t banw[R][MB];
        if (BAN) {
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const int n = base + r * kGroups + group;
#pragma unroll
                for (int q = 0; q < MB; ++q) {
                    const int i = lane + 16 * q;
                    banw[r][q] = (n < N && i < M) ? ban_bits[static_cast<size_t>(i) * ban_words + (n >> 5)] : 0u;
                }
            }
        }
        int acc[R][MC];
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int i = 0; i < MC; ++i) acc[r][i] = 0;
        for (int cb = 0; cb < C; cb += 16 * JB) {
            int4 w[R][JB];
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const int n = base + r * kGroups + group;
                const int4* wrow = reinterpret_cast<const int4*>(W + static_cast<size_t>(n < N ? n : 0) * K);
#pragma unroll
                for (int j = 0; j < JB; ++j) {
                    const int c = cb + lane + 16 * j;
                    w[r][j] = (n < N && c < C) ? ld_stream(wrow + c) : make_int4(0, 0, 0, 0);
                }
            }
#pragma unroll
            for (int j = 0; j < JB; ++j) {
                const int c = cb + lane + 16 * j;
                if (c < C) {
#pragma unroll
                    for (int i = 0; i < MC; ++i)
                        if (i < M) {
                            const int4 xv = lds_x[i * C + c];
#pragma unroll
                            for (int r = 0; r < R; ++r) acc[r][i] = dot16_i8(w[r][j], xv, acc[r][i]);
                        }
                }
            }
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int n = base + r * kGroups + group;
            const float wscale = n < N ? ws[n] : 0.0f;
#pragma unroll
            for (int i = 0; i < MC; ++i) {
                const int v = reduce16_add(acc[r][i]);
                if (n < N && i < M && lane == (i & 15)) {
                    const float t0 = static_cast<float>(v) * lds_as[i];
                    float yv = t0 * wscale;
                    if (BAN && ((banw[r][i >> 4] >> (n & 31)) & 1u)) yv = -__builtin_inff();
                    y[static_cast<size_t>(i) * N + n] = yv;
                    if (acc_out) acc_out[static_cast<size_t>(i) * N + n] = v;
                    if (keys) {
                        const uint64_t k = argmax_key(yv, static_cast<uint32_t>(n));
                        best[i >> 4] = k > best[i >> 4] ? k : best[i >> 4];
                    }
                }
            }
        }
    }
    if (keys) {
        // best[i >> 4] of row i lives in lane (i & 15) of each group; fold the 16 groups.
#pragma unroll
        for (int i = 0; i < MC; ++i)
            if (lane == (i & 15)) lds_keys[group][i] = best[i >> 4];
        __syncthreads();
        if (threadIdx.x < M) {
            uint64_t b = 0ull;
            for (int g = 0; g < kGroups; ++g) b = lds_keys[g][threadIdx.x] > b ? lds_keys[g][threadIdx.x] : b;
            keys[static_cast<size_t>(threadIdx.x) * gridDim.x + blockIdx.x] = b;
        }
    }
}

// The GEMV on the matrix cores (K % 256 == 0, M <= 32). A wave owns tiles
// of 16 weight rows and walks each in 256-byte column chunks:
//   * global -> VGPRs: 4 coalesced 16-byte loads per lane per chunk (each
//     load instruction covers 4 rows x 256 contiguous bytes), issued two
//     chunks ahead of the math;
//   * VGPRs -> LDS (a wave-private buffer [16][256]) with the
//     16-byte piece p of row r stored at slot p ^ r, so both the writes and
//     the 16-row B-fragment reads are bank-conflict free;
//   * v_mfma_i32_16x16x64_i8 with the activations as A (16 rows staged
//     once per block, rows >= M zero; M > 16 runs a second pass) and the
//     weights as B.
// The VALU does no dot products (the sdot4 form is VALU-bound from M = 4
// up); output element v of lane l is row 4*(l/16) + v of channel
// n0 + l%16, dequantized as ((f32)acc * a_s) * w_s like the sdot4 kernel.
typedef int v4i_m __attribute__((ext_vector_type(4)));
constexpr int kMfmaMinRows = 2;  // below this the sdot4 kernel is already HBM-bound
constexpr int kMfmaTileBytes = 16 * 256;  // one chunk of one tile

template <int NF>
__device__ __forceinline__ void fq_rows2_to_lds(const float4 (&v0)[NF], const float4 (&v1)[NF],
                                                const float4 (&wv)[NF], bool norm, float eps, int K, int K4,
                                                int lane, int8_t* dst0, int8_t* dst1, bool has1, float& s0,
                                                float& s1) {
    float rstd0 = 1.0f, rstd1 = 1.0f;
    if (norm) {
        double ss0 = 0.0, ss1 = 0.0;
#pragma unroll
        for (int j = 0; j < NF; ++j) {
            const double a0 = v0[j].x, b0 = v0[j].y, c0 = v0[j].z, d0 = v0[j].w;
            const double a1 = v1[j].x, b1 = v1[j].y, c1 = v1[j].z, d1 = v1[j].w;
            ss0 = fma(a0, a0, ss0);
            ss1 = fma(a1, a1, ss1);
            ss0 = fma(b0, b0, ss0);
            ss1 = fma(b1, b1, ss1);
            ss0 = fma(c0, c0, ss0);
            ss1 = fma(c1, c1, ss1);
            ss0 = fma(d0, d0, ss0);
            ss1 = fma(d1, d1, ss1);
        }
        ss0 = wave_sum_d_full(ss0);
        ss1 = wave_sum_d_full(ss1);
        rstd0 = static_cast<float>(1.0 / sqrt(ss0 / static_cast<double>(K) + static_cast<double>(eps)));
        rstd1 = static_cast<float>(1.0 / sqrt(ss1 / static_cast<double>(K) + static_cast<double>(eps)));
    }
    float4 u0[NF], u1[NF];
    float amax0 = 0.0f, amax1 = 0.0f;
#pragma unroll
    for (int j = 0; j < NF; ++j) {
        u0[j] = norm ? make_float4((v0[j].x * rstd0) * wv[j].x, (v0[j].y * rstd0) * wv[j].y,
                                   (v0[j].z * rstd0) * wv[j].z, (v0[j].w * rstd0) * wv[j].w)
                     : v0[j];
        u1[j] = norm ? make_float4((v1[j].x * rstd1) * wv[j].x, (v1[j].y * rstd1) * wv[j].y,
                                   (v1[j].z * rstd1) * wv[j].z, (v1[j].w * rstd1) * wv[j].w)
                     : v1[j];
        amax0 = fmaxf(amax0, fmaxf(fmaxf(fabsf(u0[j].x), fabsf(u0[j].y)), fmaxf(fabsf(u0[j].z), fabsf(u0[j].w))));
        amax1 = fmaxf(amax1, fmaxf(fmaxf(fabsf(u1[j].x), fabsf(u1[j].y)), fmaxf(fabsf(u1[j].z), fabsf(u1[j].w))));
    }
    amax0 = wave_max_f_full(amax0);
    amax1 = wave_max_f_full(amax1);
    const float a_scale0 = amax0 > 0.0f ? amax0 / 127.0f : 1.0f;
    const float a_scale1 = amax1 > 0.0f ? amax1 / 127.0f : 1.0f;
    const float inv0 = 1.0f / a_scale0, inv1 = 1.0f / a_scale1;
#pragma unroll
    for (int j = 0; j < NF; ++j) {
        const int c = lane + 64 * j;
        if (c < K4) {
            char4 q0, q1;
            q0.x = quant_i8(u0[j].x, inv0, false);
            q0.y = quant_i8(u0[j].y, inv0, false);
            q0.z = quant_i8(u0[j].z, inv0, false);
            q0.w = quant_i8(u0[j].w, inv0, false);
            q1.x = quant_i8(u1[j].x, inv1, false);
            q1.y = quant_i8(u1[j].y, inv1, false);
            q1.z = quant_i8(u1[j].z, inv1, false);
            q1.w = quant_i8(u1[j].w, inv1, false);
            reinterpret_cast<char4*>(dst0)[c] = q0;
            if (has1) reinterpret_cast<char4*>(dst1)[c] = q1;
        }
    }
    s0 = a_scale0;
    s1 = a_scale1;
}

// The igemm form (simd::igemm_s8s8 on device buffers): y and the scales
// unused, acc_out += the i32 sums (wrapping, as the reference's i32 adds);
// grid row y advances W, xq and acc_out by sw, sx, so elements (a batch of
// independent products in one launch).
struct IgemmMode {
    int accumulate;
    size_t sw, sx, so;
    // row groups (the split-K kernel, rows > 0): blockIdx.y takes activation
    // rows [16 y, 16 y + 16) of `rows`; y and a_scales advance by sy / sa
    size_t sy, sa;
    int rows;
};

// FQ: the <= 16 activation rows come as f32 (xf [M][K], K % 64 == 0,
// K <= 1280) and every block quantizes them (quantize_row_i8, two rows per
// wave in lockstep, while the first weight chunks are in flight) — the same
// bytes and scales as the quantize kernel, whose launch goes away.
template <bool BAN, bool FQ = false>
__global__ __launch_bounds__(kThreads) void gemv_i8_mfma_kernel(
    const int8_t* __restrict__ W, const float* __restrict__ ws, int N, int K,
    const int8_t* __restrict__ xq, const float* __restrict__ a_scales, int M,
    float* __restrict__ y, int32_t* __restrict__ acc_out, uint64_t* __restrict__ keys,
    int tiles_per_block, const uint32_t* __restrict__ ban_bits, int ban_words, const float* __restrict__ xf,
    const IgemmMode im) {
    extern __shared__ int4 lds_dyn[];  // x [16][K/16 + 1] then per-wave [16][16] chunks
    __shared__ uint64_t lds_keys[kThreads / 64][16];
    if (gridDim.y > 1) {  // the igemm form's batch: instance blockIdx.y
        W += blockIdx.y * im.sw;
        xq += blockIdx.y * im.sx;
        acc_out += blockIdx.y * im.so;
    }
    __shared__ float lds_as[16];
    const int C = K >> 4;
    const int xs = C + 1;  // x row stride in 16-byte chunks (one chunk of padding)
    const int wave = threadIdx.x >> 6;
    const int l = threadIdx.x & 63;
    const int g = l >> 4, col = l & 15;
    int4* lds_xv = lds_dyn;
    int4* wbuf = lds_dyn + 16 * xs + wave * (kMfmaTileBytes / 16);

    const int nch = K >> 8;  // 256-byte chunks per row
    const int tile0 = blockIdx.x * tiles_per_block;
    int my_tiles = 0;  // tiles tile0 + wave + 4j of this block that hold rows
    for (int tt = wave; tt < tiles_per_block && (tile0 + tt) * 16 < N; tt += kThreads / 64) ++my_tiles;
    const int nq = my_tiles * nch;
    // chunk q of this wave: tile tile0 + wave + 4 * (q / nch), column chunk q % nch
    auto load = [&](int q, int4 (&rg)[4]) {
        const int n0 = (tile0 + wave + (kThreads / 64) * (q / nch)) * 16;
        const int kc = q % nch;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int n = n0 + 4 * j + g;  // this lane's row for load j
            rg[j] = n < N ? ld_stream(reinterpret_cast<const int4*>(W + static_cast<size_t>(n) * K + kc * 256) + col)
                          : make_int4(0, 0, 0, 0);
        }
    };
    // One chunk buffer per wave: the chunk q + 1 store follows the chunk q
    // reads in the same wave, and a wave's LDS operations execute in order.
    auto store = [&](const int4 (&rg)[4]) {
        int4* b = wbuf;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int r = 4 * j + g;
            b[r * 16 + (col ^ r)] = rg[j];
        }
    };
    // the first two chunks are in flight while the activations are staged
    int4 rg0[4], rg1[4];
    if (nq > 0) load(0, rg0);
    if (nq > 1) load(1, rg1);
    if constexpr (FQ) {
        constexpr int NF = 5;  // float4 chunks of a row per lane: K <= 1280
        const int K4 = K >> 2;
        const float4 wv[NF] = {};  // no norm weight
        // rows r and r + 4 per wave and pass; rows >= M are zero
        for (int r = wave; r < 16; r += 8) {
            const int r2 = r + 4;
            if (r >= M) {  // wave-uniform
                for (int c = l; c < C; c += 64) {
                    lds_xv[r * xs + c] = make_int4(0, 0, 0, 0);
                    lds_xv[r2 * xs + c] = make_int4(0, 0, 0, 0);
                }
                if (l == 0) lds_as[r] = lds_as[r2] = 0.0f;
                continue;
            }
            const bool has1 = r2 < M;  // wave-uniform
            const float4* x0 = reinterpret_cast<const float4*>(xf + static_cast<size_t>(r) * K);
            const float4* x1 = reinterpret_cast<const float4*>(xf + static_cast<size_t>(has1 ? r2 : r) * K);
            float4 v0[NF], v1[NF];
#pragma unroll
            for (int j = 0; j < NF; ++j) {
                const int c = l + 64 * j;
                const int cc = c < K4 ? c : K4 - 1;
                const unsigned mk = c < K4 ? 0xFFFFFFFFu : 0u;
                const float4 a = x0[cc], b = x1[cc];
                v0[j] = make_float4(__uint_as_float(__float_as_uint(a.x) & mk), __uint_as_float(__float_as_uint(a.y) & mk),
                                    __uint_as_float(__float_as_uint(a.z) & mk), __uint_as_float(__float_as_uint(a.w) & mk));
                v1[j] = make_float4(__uint_as_float(__float_as_uint(b.x) & mk), __uint_as_float(__float_as_uint(b.y) & mk),
                                    __uint_as_float(__float_as_uint(b.z) & mk), __uint_as_float(__float_as_uint(b.w) & mk));
            }
            float s0, s1;
            fq_rows2_to_lds<NF>(v0, v1, wv, false, 0.0f, K, K4, l, reinterpret_cast<int8_t*>(lds_xv + r * xs),
                                reinterpret_cast<int8_t*>(lds_xv + r2 * xs), has1, s0, s1);
            if (!has1)
                for (int c = l; c < C; c += 64) lds_xv[r2 * xs + c] = make_int4(0, 0, 0, 0);
            if (l == 0) {
                lds_as[r] = s0;
                lds_as[r2] = has1 ? s1 : 0.0f;
            }
        }
    } else {
        const int4* x4 = reinterpret_cast<const int4*>(xq);
        // wave w stages rows w, w + 4, ... (rows >= M zero), lane l its chunks
        // l + 64 j, all of a row's loads issued before its stores; past the
        // row's end: its padding chunk, never read
        constexpr int J = 4;  // C <= 256 (the launch's LDS bound keeps K below 3840)
        for (int r = wave; r < 16; r += kThreads / 64) {
            int4 v[J];
            if (r < M) {  // wave-uniform
                const int4* xr = x4 + static_cast<size_t>(r) * C;
#pragma unroll
                for (int j = 0; j < J; ++j) {
                    const int c = l + 64 * j;
                    v[j] = xr[c < C ? c : C - 1];
                }
            } else {
#pragma unroll
                for (int j = 0; j < J; ++j) v[j] = make_int4(0, 0, 0, 0);
            }
#pragma unroll
            for (int j = 0; j < J; ++j) {
                const int c = l + 64 * j;
                lds_xv[r * xs + (c < C ? c : C)] = v[j];
            }
        }
        if (threadIdx.x < 16) lds_as[threadIdx.x] = threadIdx.x < M && a_scales ? a_scales[threadIdx.x] : 0.0f;
    }
    __syncthreads();
    if (nq > 0) store(rg0);

    uint64_t best[4];
#pragma unroll
    for (int v = 0; v < 4; ++v) best[v] = 0ull;
    v4i_m acc = {0, 0, 0, 0};
    // Chunk q is read from LDS while q + 1 (in rg_next) and q + 2 (issued
    // into rg_free, whose chunk q is already in LDS) are in flight.
    auto iter = [&](int q, int4 (&rg_next)[4], int4 (&rg_free)[4]) {
        const int kc = q % nch;
        if (kc == 0) acc = v4i_m{0, 0, 0, 0};
        if (q + 2 < nq) load(q + 2, rg_free);
        const int4* b = wbuf;
#pragma unroll
        for (int st = 0; st < 4; ++st) {
            const int piece = 4 * st + g;
            const int4 bw = b[col * 16 + (piece ^ col)];
            const int4 a = lds_xv[col * xs + kc * 16 + piece];
            const v4i_m bv = {bw.x, bw.y, bw.z, bw.w};
            const v4i_m av = {a.x, a.y, a.z, a.w};
            acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, bv, acc, 0, 0, 0);
        }
        if (kc == nch - 1) {
            const int n = (tile0 + wave + (kThreads / 64) * (q / nch)) * 16 + col;
            const bool valid = n < N;
            const float wscale = valid && ws ? ws[n] : 0.0f;
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int i = 4 * g + v;
                if (valid && i < M) {
                    const int av = acc[v];
                    const float t0 = static_cast<float>(av) * lds_as[i];
                    float yv = t0 * wscale;
                    if (BAN && ((ban_bits[static_cast<size_t>(i) * ban_words + (n >> 5)] >> (n & 31)) & 1u))
                        yv = -__builtin_inff();
                    if (y) y[static_cast<size_t>(i) * N + n] = yv;
                    if (acc_out) {
                        int32_t* o = acc_out + static_cast<size_t>(i) * N + n;
                        *o = im.accumulate ? static_cast<int32_t>(static_cast<uint32_t>(*o) + static_cast<uint32_t>(av))
                                           : av;
                    }
                    if (keys) {
                        const uint64_t k = argmax_key(yv, static_cast<uint32_t>(n));
                        best[v] = k > best[v] ? k : best[v];
                    }
                }
            }
        }
        if (q + 1 < nq) store(rg_next);
    };
    for (int q = 0; q < nq; q += 2) {
        iter(q, rg1, rg0);
        if (q + 1 < nq) iter(q + 1, rg0, rg1);
    }
    if (keys) {
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const uint64_t bk = row16_max_u64(best[v]);
            if (col == 0) lds_keys[wave][4 * g + v] = bk;
        }
        __syncthreads();
        if (threadIdx.x < M) {
            uint64_t bk = 0ull;
            for (int w2 = 0; w2 < kThreads / 64; ++w2)
                bk = lds_keys[w2][threadIdx.x] > bk ? lds_keys[w2][threadIdx.x] : bk;
            keys[static_cast<size_t>(threadIdx.x) * gridDim.x + blockIdx.x] = bk;
        }
    }
}

// The same GEMV for small N (a few thousand rows: a layer's qkv, o_proj,
// a shared expert's down projection), split along K: one block per 16-row
// tile, wave w takes the 256-byte column chunks w, w + 4, ... (all of them
// loaded before the first is used), and the four waves' i32 accumulators are
// added through LDS before wave 0's epilogue. With one tile per wave instead,
// N = 1280 gives only 20 blocks for the 256 CUs. Integer sums, so the
// result is bit-identical to the kernel above. K need only be a multiple of
// 64: the pieces of a last, partial chunk past K are zeroed on both sides
// (the weight pieces by a mask on the loaded data, the activation pieces
// likewise), so they add nothing.
constexpr int kSplitKMaxChunks = 8;  // per wave: K <= 32 * 256
constexpr int kFqMaxK = 2048;  // f32-input form: a row's float4s held by one wave's lanes (8 per lane)

// quantize_row_i8 (half away, reciprocal) of two f32 rows held as float4
// chunks c = lane + 64 j (zero past K4), after an RMSNorm when norm is set
// (y = (x * rstd) * w, the sum of squares in f64), written as int8 into the
// LDS stage rows dst0 / dst1 (row 1 stored only when has1); s0 / s1 get the
// activation scales. The two rows run in lockstep, their dependent
// chains (f64 sum and reduction, sqrt, amax, division) interleaved, which one
// wave per SIMD cannot hide otherwise (one row took ~1.6 us of a block's
// time), and the reductions through DPP (the call is wave-uniform: every lane
// of the wave takes part).

// FQ: the activation rows come as f32 (xf [M][K], K <= kFqMaxK) and each
// block quantizes them itself (after the RMSNorm with weight nw when nw is
// set) while its weight loads are in flight — the separate norm / quantize
// kernel and its kernel boundary go away. Every block computes the same bytes
// and scales (the same operations in the same order), and they equal what
// the quantize kernels give up to the f64 sum order of the norm.
// ROPE (with FQ): W is the qkv weight in RoPE pair order; the epilogue
// rotates each (i, i + half) pair — lanes col and col ^ 1 hold the two halves
// of the same rows — with the RoPE kernel's expressions, and writes q to its
// row and k / v to the streams' ring slots instead of y.
// ADD (with FQ): the activation row is xf + xf2 (add_residual, decoder.rs:
// 529-546, ahead of the post-attention norm); block 0 writes that sum to
// h_out for the layer's final residual. resid (no ROPE): the epilogue returns
// y + resid[i][n] (the residual folded into the projection's store; f32 adds
// commute, so it equals the separate add bit for bit).
struct RowAdd {
    const float* xf2;
    float* h_out;
    const float* resid;
};

// NF (FQ): float4 chunks of a row per lane, 64 NF >= K / 4 (5 for K = 1280,
// so the norm / quantize work covers no dead chunks)
// SWIGLU: W is [gate rows; up rows] (2N rows) and ws their 2N scales; a block
// computes the same 16 columns of both and its epilogue returns
// y = silu(g) * u (decoder.rs:1711-1752: the dense MLP's gate and up GEMVs and
// silu_mul_kernel, the same expressions in the same order).
template <int CPW, bool FQ, bool ROPE = false, int NF = kFqMaxK / 256, bool ADD = false, bool SWIGLU = false>  // chunks per wave: 4 * CPW >= the row's 256-byte chunks
__global__ __launch_bounds__(kThreads) void gemv_i8_mfma_splitk_kernel(
    const int8_t* __restrict__ W, const float* __restrict__ ws, int N, int K, const int8_t* __restrict__ xq,
    const float* __restrict__ a_scales, int M, float* __restrict__ y, int32_t* __restrict__ acc_out,
    const float* __restrict__ xf, const float* __restrict__ nw, float eps, RopeEpi re, const IgemmMode im,
    const RowAdd radd) {
    static_assert(!ADD || (FQ && !ROPE), "ADD is an f32-input form");
    static_assert(!SWIGLU || !ROPE, "one epilogue");
    extern __shared__ int4 lds_dyn[];  // x [M][K/16 + 1], then per-wave [16][16] chunks
    if (gridDim.y > 1) {
        W += blockIdx.y * im.sw;
        xq += blockIdx.y * im.sx;
        acc_out += blockIdx.y * im.so;
        if (y) y += blockIdx.y * im.sy;
        if (a_scales) a_scales += blockIdx.y * im.sa;
        if (im.rows > 0) M = min(16, im.rows - 16 * static_cast<int>(blockIdx.y));  // block-uniform
    }
    __shared__ v4i_m red[kThreads / 64][64];
    __shared__ v4i_m red_u[SWIGLU ? kThreads / 64 : 1][64];  // SWIGLU: the up tile's partials
    __shared__ float lds_as[16];
    const int C = K >> 4;
    const int xs = C + 1;
    const int wave = threadIdx.x >> 6;
    const int l = threadIdx.x & 63;
    const int g = l >> 4, col = l & 15;
    int4* lds_xv = lds_dyn;
    int4* wbuf = lds_dyn + M * xs + wave * (kMfmaTileBytes / 16);
    const int nch = (K + 255) >> 8;
    const int n0 = blockIdx.x * 16;
    int4 rg[CPW][4];
    int4 rgu[SWIGLU ? CPW : 1][4];  // SWIGLU: the up rows n + N
    auto issue_weights = [&]() {
#pragma unroll
        for (int c = 0; c < CPW; ++c) {
            const int kc = wave + 4 * c;
            const int kcl = kc < nch ? kc : nch - 1;  // loads past this wave's chunks re-read its last one (unused)
            const int pc = kcl * 16 + col;            // this lane's 16-byte piece of the row
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int n = n0 + 4 * j + g;
                const size_t row = static_cast<size_t>(n < N ? n : N - 1);
                const int4 v = ld_stream(reinterpret_cast<const int4*>(W + row * K) + (pc < C ? pc : C - 1));
                const int mm = (n < N && pc < C) ? -1 : 0;  // past N or past K: zero
                rg[c][j] = make_int4(v.x & mm, v.y & mm, v.z & mm, v.w & mm);
                if constexpr (SWIGLU) {
                    const int4 u = ld_stream(reinterpret_cast<const int4*>(W + (row + N) * K) + (pc < C ? pc : C - 1));
                    rgu[c][j] = make_int4(u.x & mm, u.y & mm, u.z & mm, u.w & mm);
                }
            }
        }
    };
    if constexpr (FQ) {
        static_assert(64 * NF <= kFqMaxK / 4, "a row's chunks fit the lanes");
        const int K4 = K >> 2;
        const float4* w4 = reinterpret_cast<const float4*>(nw);
        float4 wv[NF];
#pragma unroll
        for (int j = 0; j < NF; ++j) {
            const int c = l + 64 * j;
            wv[j] = nw ? w4[c < K4 ? c : K4 - 1] : make_float4(0.f, 0.f, 0.f, 0.f);
        }
        // rows wave, wave + 4, ...: two rows' loads in flight at once. The
        // first pair's rows are requested before the weights (loads complete
        // in issue order, so rows issued after the weights would wait for
        // them); a wave past the last row loads row M - 1 and drops it.
        auto load_pair = [&](int r, float4 (&v0)[NF], float4 (&v1)[NF]) {
            const int ra = r < M ? r : M - 1;
            const int r2 = r + kThreads / 64;
            const float4* x0 = reinterpret_cast<const float4*>(xf + static_cast<size_t>(ra) * K);
            const float4* x1 = reinterpret_cast<const float4*>(xf + static_cast<size_t>(r2 < M ? r2 : ra) * K);
            const float4* y0 = ADD ? reinterpret_cast<const float4*>(radd.xf2 + static_cast<size_t>(ra) * K) : nullptr;
            const float4* y1 =
                ADD ? reinterpret_cast<const float4*>(radd.xf2 + static_cast<size_t>(r2 < M ? r2 : ra) * K) : nullptr;
#pragma unroll
            for (int j = 0; j < NF; ++j) {
                const int c = l + 64 * j;
                const int cc = c < K4 ? c : K4 - 1;
                const unsigned mk = c < K4 ? 0xFFFFFFFFu : 0u;
                float4 a = x0[cc], b = x1[cc];
                if constexpr (ADD) {
                    const float4 a2 = y0[cc], b2 = y1[cc];
                    a = make_float4(a.x + a2.x, a.y + a2.y, a.z + a2.z, a.w + a2.w);
                    b = make_float4(b.x + b2.x, b.y + b2.y, b.z + b2.z, b.w + b2.w);
                }
                v0[j] = make_float4(__uint_as_float(__float_as_uint(a.x) & mk), __uint_as_float(__float_as_uint(a.y) & mk),
                                    __uint_as_float(__float_as_uint(a.z) & mk), __uint_as_float(__float_as_uint(a.w) & mk));
                v1[j] = make_float4(__uint_as_float(__float_as_uint(b.x) & mk), __uint_as_float(__float_as_uint(b.y) & mk),
                                    __uint_as_float(__float_as_uint(b.z) & mk), __uint_as_float(__float_as_uint(b.w) & mk));
            }
        };
        auto quant_pair = [&](int r, const float4 (&v0)[NF], const float4 (&v1)[NF]) {
            const int r2 = r + kThreads / 64;
            if (r >= M) return;  // wave-uniform
            const bool has1 = r2 < M;  // wave-uniform; without it row 1 repeats row 0 and is dropped
            if constexpr (ADD) {
                if (blockIdx.x == 0) {  // h = x + xf2 for the residual, once
                    float4* h0 = reinterpret_cast<float4*>(radd.h_out + static_cast<size_t>(r) * K);
                    float4* h1 = reinterpret_cast<float4*>(radd.h_out + static_cast<size_t>(r2) * K);
#pragma unroll
                    for (int j = 0; j < NF; ++j) {
                        const int c = l + 64 * j;
                        if (c < K4) {
                            h0[c] = v0[j];
                            if (has1) h1[c] = v1[j];
                        }
                    }
                }
            }
            float s0, s1;
            fq_rows2_to_lds<NF>(v0, v1, wv, nw != nullptr, eps, K, K4, l, reinterpret_cast<int8_t*>(lds_xv + r * xs),
                                reinterpret_cast<int8_t*>(lds_xv + (has1 ? r2 : r) * xs), has1, s0, s1);
            if (l == 0) {
                lds_as[r] = s0;
                if (has1) lds_as[r2] = s1;
            }
        };
        {
            float4 v0[NF], v1[NF];
            load_pair(wave, v0, v1);
            issue_weights();
            quant_pair(wave, v0, v1);
        }
        for (int r = wave + 2 * (kThreads / 64); r < M; r += 2 * (kThreads / 64)) {
            float4 v0[NF], v1[NF];
            load_pair(r, v0, v1);
            quant_pair(r, v0, v1);
        }
        if (threadIdx.x < 16 && threadIdx.x >= M) lds_as[threadIdx.x] = 0.0f;
    } else {
        issue_weights();
        const int4* x4 = reinterpret_cast<const int4*>(xq);
        // only the M live rows (the rest read as zero): wave w stages rows
        // w, w + 4, ..., lane l its 16-byte chunks l + 64 j, all of a row's
        // loads issued before its stores (a loop of single loads waits for
        // each in turn); past the row's end: its padding chunk, never read
        constexpr int J = CPW;  // C <= 64 CPW: the kernel's K <= 256 * 4 * CPW
        for (int r = wave; r < M; r += kThreads / 64) {
            const int4* xr = x4 + static_cast<size_t>(r) * C;
            int4 v[J];
#pragma unroll
            for (int j = 0; j < J; ++j) {
                const int c = l + 64 * j;
                v[j] = xr[c < C ? c : C - 1];
            }
#pragma unroll
            for (int j = 0; j < J; ++j) {
                const int c = l + 64 * j;
                lds_xv[r * xs + (c < C ? c : C)] = v[j];
            }
        }
        if (threadIdx.x < 16) lds_as[threadIdx.x] = threadIdx.x < M && a_scales ? a_scales[threadIdx.x] : 0.0f;
    }
    // the epilogue's residual values, requested now so they arrive under the
    // MFMAs (wave 0 writes the outputs)
    float rsd[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (!ROPE && !SWIGLU && radd.resid && wave == 0) {
        const int nn = n0 + col < N ? n0 + col : N - 1;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int i = 4 * g + v;
            rsd[v] = radd.resid[static_cast<size_t>(i < M ? i : 0) * N + nn];
        }
    }
    __syncthreads();
    v4i_m acc = {0, 0, 0, 0}, accu = {0, 0, 0, 0};
    // one 16-row tile of chunk kc: the rows through the wave's LDS tile (one
    // wave writes and reads it, in order), 4 MFMA steps into a
    auto tile_mfma = [&](const int4 (&rgc)[4], int kc, v4i_m& a_acc) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int r = 4 * j + g;
            wbuf[r * 16 + (col ^ r)] = rgc[j];
        }
#pragma unroll
        for (int st = 0; st < 4; ++st) {
            const int piece = 4 * st + g;
            const int4 bw = wbuf[col * 16 + (piece ^ col)];
            const int pa = kc * 16 + piece;
            const int4 a = lds_xv[(col < M ? col : 0) * xs + (pa < C ? pa : C - 1)];
            const int ma = (pa < C && col < M) ? -1 : 0;
            const v4i_m bv = {bw.x, bw.y, bw.z, bw.w};
            const v4i_m av = {a.x & ma, a.y & ma, a.z & ma, a.w & ma};
            a_acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, bv, a_acc, 0, 0, 0);
        }
    };
#pragma unroll
    for (int c = 0; c < CPW; ++c) {
        const int kc = wave + 4 * c;
        if (kc >= nch) break;  // wave-uniform
        tile_mfma(rg[c], kc, acc);
        if constexpr (SWIGLU) tile_mfma(rgu[c], kc, accu);
    }
    red[wave][l] = acc;
    if constexpr (SWIGLU) red_u[wave][l] = accu;
    __syncthreads();
    if (wave != 0) return;
#pragma unroll
    for (int w2 = 1; w2 < kThreads / 64; ++w2) {
        const v4i_m o = red[w2][l];
        acc = v4i_m{acc[0] + o[0], acc[1] + o[1], acc[2] + o[2], acc[3] + o[3]};
        if constexpr (SWIGLU) {
            const v4i_m ou = red_u[w2][l];
            accu = v4i_m{accu[0] + ou[0], accu[1] + ou[1], accu[2] + ou[2], accu[3] + ou[3]};
        }
    }
    const int n = n0 + col;
    if constexpr (SWIGLU) {
        if (n >= N) return;
        const float sg = ws[n], su = ws[N + n];
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int i = 4 * g + v;
            if (i < M) {
                const float gv = (static_cast<float>(acc[v]) * lds_as[i]) * sg;
                const float uv = (static_cast<float>(accu[v]) * lds_as[i]) * su;
                y[static_cast<size_t>(i) * N + n] = silu_f(gv) * uv;
            }
        }
        return;
    }
    if constexpr (ROPE) {
        const float wscale = ws[n < N ? n : N - 1];
        const int D = re.d_model, hdim = re.head_dim, half = hdim >> 1;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int i = 4 * g + v;
            const float yv = (static_cast<float>(acc[v]) * lds_as[i]) * wscale;
            const float pv = __int_as_float(dpp_mov<0xB1>(__float_as_int(yv)));  // lane col ^ 1: the pair partner
            if (i >= M || n >= N) continue;
            const int s = re.r0 + i;
            if (n < 2 * D) {
                const int part = n / D, pl = n - part * D;
                const int hd = pl / hdim, pr = pl - hd * hdim;
                const int ii = pr >> 1, b = pr & 1;
                const float angle = static_cast<float>(re.pos.p[s]) * re.inv_freq[ii];
                float sn, cs;
                sincosf(angle, &sn, &cs);
                // b = 0: a * cs - b * sn (a = mine); b = 1: b * cs + a * sn (b = mine)
                const float o = b == 0 ? yv * cs - pv * sn : yv * cs + pv * sn;
                const int j = ii + b * half;
                if (part == 0)
                    re.q[static_cast<size_t>(s) * D + hd * hdim + j] = o;
                else
                    re.ring.k[s][static_cast<size_t>(hd) * re.ring.head_stride + j] = o;
            } else {
                const int pl = n - 2 * D, hd = pl / hdim;
                re.ring.v[s][static_cast<size_t>(hd) * re.ring.head_stride + (pl - hd * hdim)] = yv;
            }
        }
        return;
    }
    if (n >= N) return;
    const float wscale = ws ? ws[n] : 0.0f;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
        const int i = 4 * g + v;
        if (i < M) {
            const int av = acc[v];
            const float t0 = static_cast<float>(av) * lds_as[i];
            if (y) {
                const float o = t0 * wscale;
                y[static_cast<size_t>(i) * N + n] = radd.resid ? o + rsd[v] : o;
            }
            if (acc_out) {
                int32_t* o = acc_out + static_cast<size_t>(i) * N + n;
                *o = im.accumulate ? static_cast<int32_t>(static_cast<uint32_t>(*o) + static_cast<uint32_t>(av)) : av;
            }
        }
    }
}

// Row p of the output = row qkv_rope_row(p) of w (and its scale): the qkv
// weights in RoPE pair order, made once per decoder layer.
__global__ __launch_bounds__(kThreads) void permute_rows_i8_kernel(const int8_t* __restrict__ w,
                                                                  const float* __restrict__ ws, int k, int D,
                                                                  int head_dim, int8_t* __restrict__ w_out,
                                                                  float* __restrict__ ws_out) {
    const int p = blockIdx.x;
    const int src = qkv_rope_row(p, D, head_dim);
    const int8_t* in = w + static_cast<size_t>(src) * k;
    int8_t* out = w_out + static_cast<size_t>(p) * k;
    for (int c = threadIdx.x; c < k; c += kThreads) out[c] = in[c];
    if (threadIdx.x == 0) ws_out[p] = ws[src];
}

// One block per row: fold nparts keys -> the argmax index.
__global__ __launch_bounds__(kThreads) void argmax_reduce_kernel(const uint64_t* __restrict__ keys,
                                                                 int nparts,
                                                                 uint32_t* __restrict__ argmax) {
    __shared__ uint64_t red[kThreads / 64];
    const int row = blockIdx.x;
    uint64_t b = thread_max_keys<kThreads>(keys + static_cast<size_t>(row) * nparts, nparts);
    b = wave_max_u64_full(b);
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
    b = wave_max_u64_full(b);
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

// The current device's LDS limit per block (160 KB on gfx950, where a
// kernel may take more than 64 KB of dynamic LDS), queried once per device.
size_t max_lds_per_block() {
    static std::atomic<int> cached[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 65536;
    int v = cached[dev].load(std::memory_order_relaxed);
    if (v == 0) {
        if (hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess || v <= 0)
            v = 65536;
        cached[dev].store(v, std::memory_order_relaxed);
    }
    return static_cast<size_t>(v);
}

hipError_t launch_quantize_rows(hipStream_t s, const float* x, int m, int k, int8_t* xq,
                                float* a_scales, int rule) {
    if (m == 0) return hipSuccess;
    // rows in registers where they fit (K a multiple of 4 up to 8192, 16-byte
    // aligned rows and outputs)
    const bool vec = k > 0 && k % 4 == 0 && k <= 8 * 4 * kThreads && reinterpret_cast<uintptr_t>(x) % 16 == 0 &&
                     reinterpret_cast<uintptr_t>(xq) % 4 == 0;
    if (vec && k <= 1 * 4 * kThreads)
        FOCR_LAUNCH(quantize_rows_vec_kernel<1>, dim3(m), dim3(kThreads), 0, s, x, k, xq, a_scales, rule);
    else if (vec && k <= 2 * 4 * kThreads)
        FOCR_LAUNCH(quantize_rows_vec_kernel<2>, dim3(m), dim3(kThreads), 0, s, x, k, xq, a_scales, rule);
    else if (vec && k <= 4 * 4 * kThreads)
        FOCR_LAUNCH(quantize_rows_vec_kernel<4>, dim3(m), dim3(kThreads), 0, s, x, k, xq, a_scales, rule);
    else if (vec)
        FOCR_LAUNCH(quantize_rows_vec_kernel<8>, dim3(m), dim3(kThreads), 0, s, x, k, xq, a_scales, rule);
    else
        FOCR_LAUNCH(quantize_rows_kernel, dim3(m), dim3(kThreads), 0, s, x, k, xq, a_scales, rule);
    return hipGetLastError();
}

hipError_t launch_quantize_rows2(hipStream_t s, const QuantRows& r1, const QuantRows& r2, int rule) {
    auto vec_ok = [](const QuantRows& r) {
        return r.K > 0 && r.K % 4 == 0 && r.K <= 2 * 4 * kThreads && reinterpret_cast<uintptr_t>(r.x) % 16 == 0 &&
               reinterpret_cast<uintptr_t>(r.xq) % 4 == 0;
    };
    if (r1.m <= 0 || r2.m <= 0 || !vec_ok(r1) || !vec_ok(r2)) {  // one launch per set
        hipError_t e = launch_quantize_rows(s, r1.x, r1.m, r1.K, r1.xq, r1.scales, rule);
        return e != hipSuccess ? e : launch_quantize_rows(s, r2.x, r2.m, r2.K, r2.xq, r2.scales, rule);
    }
    const int kmax = r1.K > r2.K ? r1.K : r2.K;
    if (kmax <= 1 * 4 * kThreads)
        FOCR_LAUNCH(quantize_rows2_vec_kernel<1>, dim3(r1.m + r2.m), dim3(kThreads), 0, s, r1, r2, rule);
    else
        FOCR_LAUNCH(quantize_rows2_vec_kernel<2>, dim3(r1.m + r2.m), dim3(kThreads), 0, s, r1, r2, rule);
    return hipGetLastError();
}

hipError_t launch_gemv_i8_f32(hipStream_t s, const int8_t* w, const float* ws, int n, int k, const float* x,
                              const float* norm_w, float eps, int m, float* y, int8_t* xq_tmp, float* xs_tmp,
                              int cu_count) {
    if (m < 1 || k <= 0) return hipErrorInvalidValue;
    const size_t lds_splitk =
        (static_cast<size_t>(m < 16 ? m : 16) * (k / 16 + 1) + (kThreads / 64) * kMfmaTileBytes / 16) * sizeof(int4);
    const size_t lds_splitk_static = (kThreads / 64) * 64 * sizeof(int4) + 16 * sizeof(float);
    if (m >= kMfmaMinRows && k % 64 == 0 && k <= kFqMaxK && lds_splitk + lds_splitk_static <= max_lds_per_block() &&
        (n + 15) / 16 < 4 * (cu_count > 0 ? cu_count : 256)) {
        const int grid = (n + 15) / 16;
        for (int r0 = 0; r0 < m; r0 += 16) {
            const int mr = m - r0 < 16 ? m - r0 : 16;
            if (k <= 64 * 4 * 5)  // rows of <= 5 float4 per lane
                FOCR_LAUNCH((gemv_i8_mfma_splitk_kernel<2, true, false, 5>), dim3(grid), dim3(kThreads), lds_splitk,
                            s, w, ws, n, k, nullptr, nullptr, mr, y + static_cast<size_t>(r0) * n, nullptr,
                            x + static_cast<size_t>(r0) * k, norm_w, eps, RopeEpi{}, IgemmMode{}, RowAdd{});
            else if (k <= 64 * 4 * 7)  // <= 7 (the shared expert's 1792-wide act rows)
                FOCR_LAUNCH((gemv_i8_mfma_splitk_kernel<2, true, false, 7>), dim3(grid), dim3(kThreads), lds_splitk,
                            s, w, ws, n, k, nullptr, nullptr, mr, y + static_cast<size_t>(r0) * n, nullptr,
                            x + static_cast<size_t>(r0) * k, norm_w, eps, RopeEpi{}, IgemmMode{}, RowAdd{});
            else
                FOCR_LAUNCH((gemv_i8_mfma_splitk_kernel<2, true>), dim3(grid), dim3(kThreads), lds_splitk, s, w, ws,
                            n, k, nullptr, nullptr, mr, y + static_cast<size_t>(r0) * n, nullptr,
                            x + static_cast<size_t>(r0) * k, norm_w, eps, RopeEpi{}, IgemmMode{}, RowAdd{});
        }
        return hipGetLastError();
    }
    // otherwise: the norm / quantize kernel, then the GEMV on the int8 rows
    hipError_t e = norm_w ? launch_rms_norm_quant(s, x, norm_w, m, k, eps, xq_tmp, xs_tmp)
                          : launch_quantize_rows(s, x, m, k, xq_tmp, xs_tmp, 0);
    if (e != hipSuccess) return e;
    for (int r0 = 0; r0 < m && e == hipSuccess; r0 += 32) {
        const int mr = m - r0 < 32 ? m - r0 : 32;
        e = launch_gemv_i8(s, w, ws, n, k, xq_tmp + static_cast<size_t>(r0) * k, xs_tmp + r0, mr,
                           y + static_cast<size_t>(r0) * n, nullptr, nullptr, nullptr, cu_count);
    }
    return e;
}

hipError_t launch_swiglu_i8_f32_add(hipStream_t s, const int8_t* w_gu, const float* ws_gu, int n, int k,
                                    const float* x, const float* x2, float* h_out, const float* norm_w, float eps,
                                    int m, float* act, int cu_count) {
    if (m < 1 || !x2 || !h_out) return hipErrorInvalidValue;
    const size_t lds_splitk =
        (static_cast<size_t>(m < 16 ? m : 16) * (k / 16 + 1) + (kThreads / 64) * kMfmaTileBytes / 16) * sizeof(int4);
    const size_t lds_splitk_static = (kThreads / 64) * 64 * sizeof(int4) + 16 * sizeof(float);
    if (m < kMfmaMinRows || k < 64 || k % 64 != 0 || k > 64 * 4 * 5 ||
        lds_splitk + lds_splitk_static > max_lds_per_block() || (n + 15) / 16 >= 4 * (cu_count > 0 ? cu_count : 256))
        return hipErrorNotSupported;
    const int grid = (n + 15) / 16;
    for (int r0 = 0; r0 < m; r0 += 16) {
        const int mr = m - r0 < 16 ? m - r0 : 16;
        const size_t off = static_cast<size_t>(r0) * k;
        FOCR_LAUNCH((gemv_i8_mfma_splitk_kernel<2, true, false, 5, true, true>), dim3(grid), dim3(kThreads),
                    lds_splitk, s, w_gu, ws_gu, n, k, nullptr, nullptr, mr, act + static_cast<size_t>(r0) * n, nullptr,
                    x + off, norm_w, eps, RopeEpi{}, IgemmMode{}, RowAdd{x2 + off, h_out + off, nullptr});
    }
    return hipGetLastError();
}

hipError_t launch_gemv_i8_resid(hipStream_t s, const int8_t* w, const float* ws, int n, int k, const int8_t* xq,
                                const float* a_scales, int m, const float* resid, float* y, int cu_count) {
    if (m < 1 || !resid) return hipErrorInvalidValue;
    const size_t lds_splitk =
        (static_cast<size_t>(m < 16 ? m : 16) * (k / 16 + 1) + (kThreads / 64) * kMfmaTileBytes / 16) * sizeof(int4);
    const size_t lds_splitk_static = (kThreads / 64) * 64 * sizeof(int4) + 16 * sizeof(float);
    if (m < kMfmaMinRows || k < 64 || k % 64 != 0 || k > 256 * 4 * kSplitKMaxChunks ||
        lds_splitk + lds_splitk_static > max_lds_per_block() || (n + 15) / 16 >= 4 * (cu_count > 0 ? cu_count : 256))
        return hipErrorNotSupported;
    const int grid = (n + 15) / 16;
    const int cpw = ((k + 255) / 256 + 3) / 4;
    for (int r0 = 0; r0 < m; r0 += 16) {
        const int mr = m - r0 < 16 ? m - r0 : 16;
        const int8_t* xq_r = xq + static_cast<size_t>(r0) * k;
        float* y_r = y + static_cast<size_t>(r0) * n;
        const RowAdd ra{nullptr, nullptr, resid + static_cast<size_t>(r0) * n};
        if (cpw <= 2)
            FOCR_LAUNCH((gemv_i8_mfma_splitk_kernel<2, false>), dim3(grid), dim3(kThreads), lds_splitk, s, w, ws, n,
                        k, xq_r, a_scales + r0, mr, y_r, nullptr, nullptr, nullptr, 0.0f, RopeEpi{}, IgemmMode{}, ra);
        else if (cpw <= 4)
            FOCR_LAUNCH((gemv_i8_mfma_splitk_kernel<4, false>), dim3(grid), dim3(kThreads), lds_splitk, s, w, ws, n,
                        k, xq_r, a_scales + r0, mr, y_r, nullptr, nullptr, nullptr, 0.0f, RopeEpi{}, IgemmMode{}, ra);
        else
            FOCR_LAUNCH((gemv_i8_mfma_splitk_kernel<8, false>), dim3(grid), dim3(kThreads), lds_splitk, s, w, ws, n,
                        k, xq_r, a_scales + r0, mr, y_r, nullptr, nullptr, nullptr, 0.0f, RopeEpi{}, IgemmMode{}, ra);
    }
    return hipGetLastError();
}

// Prefill-sized products on the split-K kernel: m <= kRowsMaxM prequantized
// rows xq [m][k] with scales xs [m], in groups of 16 on grid.y (each block
// stages its group's rows and takes 16 output columns, the four waves on
// interleaved 256-byte K chunks); the weight rows come from L2 for every
// group after the first. y = ((f32)acc * xs) * ws, the linear's epilogue
// (SWIGLU: w_gu holds the gate rows then the up rows, act = silu(g) * u).
bool gemv_rows_supported(int n, int k, int m) {
    if (m < 1 || m > kRowsMaxM || n < 1 || k < 64 || k % 64 != 0 || k > 256 * 4 * kSplitKMaxChunks) return false;
    const size_t lds = (static_cast<size_t>(16) * (k / 16 + 1) + (kThreads / 64) * kMfmaTileBytes / 16) * sizeof(int4);
    const size_t lds_static = (kThreads / 64) * 64 * sizeof(int4) * 2 + 16 * sizeof(float);
    return lds + lds_static <= max_lds_per_block();
}

// Every block re-reads its 16 activation rows and its 16 (SwiGLU: 32) weight
// rows through L2, so past about 2048 blocks of that traffic the tiled GEMMs
// are faster despite their few blocks (measured at m = 256, k = 1280: n =
// 1280 9.7 us here against 15.7; n = 3840 21.4 against 15.7).
bool gemv_rows_preferred(int n, int k, int m, bool swiglu) {
    if (!gemv_rows_supported(n, k, m)) return false;
    const long blocks = static_cast<long>((n + 15) / 16) * ((m + 15) / 16) * (swiglu ? 2 : 1);
    return blocks <= 2048;
}

template <bool SWIGLU>
static hipError_t launch_rows(hipStream_t s, const int8_t* w, const float* ws, int n, int k, const int8_t* xq,
                              const float* xs, int m, float* y) {
    if (!gemv_rows_supported(n, k, m)) return hipErrorInvalidValue;
    const size_t lds = (static_cast<size_t>(m < 16 ? m : 16) * (k / 16 + 1) + (kThreads / 64) * kMfmaTileBytes / 16) *
                       sizeof(int4);
    const dim3 grid((n + 15) / 16, (m + 15) / 16);
    IgemmMode im{};
    im.sx = static_cast<size_t>(16) * k;
    im.sy = static_cast<size_t>(16) * n;
    im.sa = 16;
    im.rows = m;
    const int mr = m < 16 ? m : 16;
    const int cpw = ((k + 255) / 256 + 3) / 4;
    if (cpw <= 2)
        FOCR_LAUNCH((gemv_i8_mfma_splitk_kernel<2, false, false, kFqMaxK / 256, false, SWIGLU>), grid, dim3(kThreads),
                    lds, s, w, ws, n, k, xq, xs, mr, y, nullptr, nullptr, nullptr, 0.0f, RopeEpi{}, im, RowAdd{});
    else if (cpw <= 4)
        FOCR_LAUNCH((gemv_i8_mfma_splitk_kernel<4, false, false, kFqMaxK / 256, false, SWIGLU>), grid, dim3(kThreads),
                    lds, s, w, ws, n, k, xq, xs, mr, y, nullptr, nullptr, nullptr, 0.0f, RopeEpi{}, im, RowAdd{});
    else
        FOCR_LAUNCH((gemv_i8_mfma_splitk_kernel<8, false, false, kFqMaxK / 256, false, SWIGLU>), grid, dim3(kThreads),
                    lds, s, w, ws, n, k, xq, xs, mr, y, nullptr, nullptr, nullptr, 0.0f, RopeEpi{}, im, RowAdd{});
    return hipGetLastError();
}

hipError_t launch_gemv_i8_rows(hipStream_t s, const int8_t* w, const float* ws, int n, int k, const int8_t* xq,
                               const float* xs, int m, float* y) {
    return launch_rows<false>(s, w, ws, n, k, xq, xs, m, y);
}

hipError_t launch_permute_rows_i8(hipStream_t s, const int8_t* w, const float* ws, int n, int k, int D, int head_dim,
                                  int8_t* w_out, float* ws_out) {
    if (n != 3 * D || head_dim % 2 || D % head_dim) return hipErrorInvalidValue;
    FOCR_LAUNCH(permute_rows_i8_kernel, dim3(n), dim3(kThreads), 0, s, w, ws, k, D, head_dim, w_out, ws_out);
    return hipGetLastError();
}

hipError_t launch_qkv_rope_f32(hipStream_t s, const int8_t* w_perm, const float* ws_perm, int n, int k,
                               const float* x, const float* norm_w, float eps, int m, RopeEpi epi, int cu_count) {
    const size_t lds_splitk =
        (static_cast<size_t>(m < 16 ? m : 16) * (k / 16 + 1) + (kThreads / 64) * kMfmaTileBytes / 16) * sizeof(int4);
    const size_t lds_splitk_static = (kThreads / 64) * 64 * sizeof(int4) + 16 * sizeof(float);
    const int D = epi.d_model;
    if (m < kMfmaMinRows || m > RopePositions::kMax || k < 64 || k % 64 != 0 || k > kFqMaxK || n != 3 * D ||
        epi.head_dim % 16 != 0 || D % epi.head_dim != 0 || !epi.q || !epi.inv_freq ||
        lds_splitk + lds_splitk_static > max_lds_per_block() || (n + 15) / 16 >= 4 * (cu_count > 0 ? cu_count : 256))
        return hipErrorNotSupported;
    for (int i = 0; i < m; ++i)
        if (!epi.ring.k[i] || !epi.ring.v[i]) return hipErrorInvalidValue;
    const int grid = (n + 15) / 16;
    for (int r0 = 0; r0 < m; r0 += 16) {
        const int mr = m - r0 < 16 ? m - r0 : 16;
        RopeEpi e = epi;
        e.r0 = r0;
        if (k <= 64 * 4 * 5)  // rows of <= 5 float4 per lane
            FOCR_LAUNCH((gemv_i8_mfma_splitk_kernel<2, true, true, 5>), dim3(grid), dim3(kThreads), lds_splitk, s,
                        w_perm, ws_perm, n, k, nullptr, nullptr, mr, nullptr, nullptr,
                        x + static_cast<size_t>(r0) * k, norm_w, eps, e, IgemmMode{}, RowAdd{});
        else
            FOCR_LAUNCH((gemv_i8_mfma_splitk_kernel<2, true, true>), dim3(grid), dim3(kThreads), lds_splitk, s,
                        w_perm, ws_perm, n, k, nullptr, nullptr, mr, nullptr, nullptr,
                        x + static_cast<size_t>(r0) * k, norm_w, eps, e, IgemmMode{}, RowAdd{});
    }
    return hipGetLastError();
}

hipError_t launch_gemv_i8(hipStream_t s, const int8_t* w, const float* ws, int n, int k,
                          const int8_t* xq, const float* a_scales, int m, float* y, int32_t* acc,
                          uint64_t* arg_keys, int* nparts_out, int cu_count) {
    return launch_gemv_i8_banned(s, w, ws, n, k, xq, a_scales, m, y, acc, arg_keys, nparts_out, cu_count, nullptr,
                                 0);
}

hipError_t launch_gemv_i8_f32_keys(hipStream_t s, const int8_t* w, const float* ws, int n, int k, const float* x,
                                   int m, float* y, uint64_t* arg_keys, int* nparts_out, int cu_count) {
    if (reinterpret_cast<uintptr_t>(x) % 16 != 0) return hipErrorNotSupported;
    if (m == 1) {
        // one f32 row, quantized by every block: the sdot4 kernel's one-row form
        if (k <= 0 || k % 16 != 0 || k > 2 * 4 * kThreads) return hipErrorNotSupported;
        const int tiles = (n + kGroups - 1) / kGroups;  // R = 1
        const int target_blocks = (cu_count > 0 ? cu_count : 256) * 8;
        int tpb = (tiles + target_blocks - 1) / target_blocks;
        tpb = tpb < 1 ? 1 : tpb;
        const int grid = (tiles + tpb - 1) / tpb;
        if (nparts_out) *nparts_out = grid;
        FOCR_LAUNCH((gemv_i8_kernel<1, 8, 1, false, true>), dim3(grid), dim3(kThreads), static_cast<size_t>(k), s, w,
                    ws, n, k, nullptr, nullptr, 1, y, nullptr, arg_keys, tpb, nullptr, 0, x);
        return hipGetLastError();
    }
    // 2..16 f32 rows on the matrix-core kernel, quantized by every block
    const size_t lds_mfma = (static_cast<size_t>(16) * (k / 16 + 1) + (kThreads / 64) * kMfmaTileBytes / 16) *
                            sizeof(int4);
    if (m < kMfmaMinRows || m > 16 || k < 256 || k % 256 != 0 || k > 64 * 4 * 5 || lds_mfma > 65536)
        return hipErrorNotSupported;
    const int tiles = (n + 15) / 16;
    const int target_blocks = (cu_count > 0 ? cu_count : 256) * 4;  // as launch_gemv_i8's matrix-core form
    int tpb = (tiles + target_blocks - 1) / target_blocks;
    tpb = (tpb + 3) & ~3;
    const int grid = (tiles + tpb - 1) / tpb;
    if (nparts_out) *nparts_out = grid;
    FOCR_LAUNCH((gemv_i8_mfma_kernel<false, true>), dim3(grid), dim3(kThreads), lds_mfma, s, w, ws, n, k, nullptr,
                nullptr, m, y, nullptr, arg_keys, tpb, nullptr, 0, x, IgemmMode{});
    return hipGetLastError();
}

hipError_t launch_gemv_i8_banned(hipStream_t s, const int8_t* w, const float* ws, int n, int k,
                                 const int8_t* xq, const float* a_scales, int m, float* y, int32_t* acc,
                                 uint64_t* arg_keys, int* nparts_out, int cu_count, const uint32_t* ban_bits,
                                 int ban_words) {
    if (m < 1 || m > 32 || k % 16 != 0 || k <= 0) return hipErrorInvalidValue;
    if (ban_bits && ban_words * 32 < n) return hipErrorInvalidValue;
    const size_t lds = static_cast<size_t>(m) * k;
    if (lds > 57344) return hipErrorInvalidValue;
    int mc = 1;
    while (mc < m) mc <<= 1;
    const size_t lds_mfma = (static_cast<size_t>(16) * (k / 16 + 1) + (kThreads / 64) * kMfmaTileBytes / 16) *
                            sizeof(int4);
    // x rows of one pass (<= 16) + the waves' transpose tiles; + the static
    // reduction buffer and scales
    const size_t lds_splitk =
        (static_cast<size_t>(m < 16 ? m : 16) * (k / 16 + 1) + (kThreads / 64) * kMfmaTileBytes / 16) * sizeof(int4);
    const size_t lds_splitk_static = (kThreads / 64) * 64 * sizeof(int4) + 16 * sizeof(float);
    if (m >= kMfmaMinRows && k % 64 == 0 && lds_splitk + lds_splitk_static <= max_lds_per_block() && !arg_keys &&
        !ban_bits &&
        k <= 256 * 4 * kSplitKMaxChunks && (n + 15) / 16 < 4 * (cu_count > 0 ? cu_count : 256)) {
        // small N: one 16-row tile per block, K split over the four waves
        const int grid = (n + 15) / 16;
        if (nparts_out) *nparts_out = grid;
        const int cpw = ((k + 255) / 256 + 3) / 4;
        for (int r0 = 0; r0 < m; r0 += 16) {
            const int mr = m - r0 < 16 ? m - r0 : 16;
            const int8_t* xq_r = xq + static_cast<size_t>(r0) * k;
            float* y_r = y + static_cast<size_t>(r0) * n;
            int32_t* acc_r = acc ? acc + static_cast<size_t>(r0) * n : nullptr;
            if (cpw <= 2)
                FOCR_LAUNCH((gemv_i8_mfma_splitk_kernel<2, false>), dim3(grid), dim3(kThreads), lds_splitk, s, w, ws,
                            n, k, xq_r, a_scales + r0, mr, y_r, acc_r, nullptr, nullptr, 0.0f, RopeEpi{}, IgemmMode{}, RowAdd{});
            else if (cpw <= 4)
                FOCR_LAUNCH((gemv_i8_mfma_splitk_kernel<4, false>), dim3(grid), dim3(kThreads), lds_splitk, s, w, ws,
                            n, k, xq_r, a_scales + r0, mr, y_r, acc_r, nullptr, nullptr, 0.0f, RopeEpi{}, IgemmMode{}, RowAdd{});
            else
                FOCR_LAUNCH((gemv_i8_mfma_splitk_kernel<8, false>), dim3(grid), dim3(kThreads), lds_splitk, s, w, ws,
                            n, k, xq_r, a_scales + r0, mr, y_r, acc_r, nullptr, nullptr, 0.0f, RopeEpi{}, IgemmMode{}, RowAdd{});
        }
        return hipGetLastError();
    }
    if (m >= kMfmaMinRows && k % 256 == 0 && lds_mfma <= 65536) {
        const int tiles = (n + 15) / 16;
        // four blocks per CU (16 waves, 37 KB of LDS each at K = 1280): the
        // measured optimum between 2 and 8 at M = 8 and M = 16
        const int target_blocks = (cu_count > 0 ? cu_count : 256) * 4;
        int tpb = (tiles + target_blocks - 1) / target_blocks;
        tpb = (tpb + 3) & ~3;  // whole rounds of the block's four waves
        const int grid = (tiles + tpb - 1) / tpb;
        if (nparts_out) *nparts_out = grid;
        // up to 16 activation rows per pass; rows 16..31 take a second pass
        // over the weights with every row-indexed pointer advanced
        for (int r0 = 0; r0 < m; r0 += 16) {
            const int mr = m - r0 < 16 ? m - r0 : 16;
            const int8_t* xq_r = xq + static_cast<size_t>(r0) * k;
            float* y_r = y + static_cast<size_t>(r0) * n;
            int32_t* acc_r = acc ? acc + static_cast<size_t>(r0) * n : nullptr;
            uint64_t* keys_r = arg_keys ? arg_keys + static_cast<size_t>(r0) * grid : nullptr;
            if (ban_bits)
                FOCR_LAUNCH((gemv_i8_mfma_kernel<true>), dim3(grid), dim3(kThreads), lds_mfma, s, w, ws, n, k, xq_r,
                            a_scales + r0, mr, y_r, acc_r, keys_r, tpb, ban_bits + static_cast<size_t>(r0) * ban_words,
                            ban_words, nullptr, IgemmMode{});
            else
                FOCR_LAUNCH((gemv_i8_mfma_kernel<false>), dim3(grid), dim3(kThreads), lds_mfma, s, w, ws, n, k,
                            xq_r, a_scales + r0, mr, y_r, acc_r, keys_r, tpb, nullptr, 0, nullptr, IgemmMode{});
        }
        return hipGetLastError();
    }
    // rows per group: one for M <= 2 (HBM-bound already), four up to M = 8,
    // two beyond (accumulator registers grow as R * M)
    const int R = mc <= 2 ? 1 : (mc <= 8 ? 4 : 2);
    const int rows_per_tile = kGroups * R;
    const int tiles = (n + rows_per_tile - 1) / rows_per_tile;
    const int target_blocks = (cu_count > 0 ? cu_count : 256) * 8;
    int tpb = (tiles + target_blocks - 1) / target_blocks;
    tpb = tpb < 1 ? 1 : tpb;
    const int grid = (tiles + tpb - 1) / tpb;
    if (nparts_out) *nparts_out = grid;
#define FOCR_GEMV_CASE(MCV, JBV, RV)                                                                      \
    case MCV:                                                                                             \
        if (ban_bits)                                                                                     \
            FOCR_LAUNCH((gemv_i8_kernel<MCV, JBV, RV, true>), dim3(grid), dim3(kThreads), lds, s, w, ws, n, \
                        k, xq, a_scales, m, y, acc, arg_keys, tpb, ban_bits, ban_words, nullptr);         \
        else                                                                                              \
            FOCR_LAUNCH((gemv_i8_kernel<MCV, JBV, RV, false>), dim3(grid), dim3(kThreads), lds, s, w, ws, n,\
                        k, xq, a_scales, m, y, acc, arg_keys, tpb, nullptr, 0, nullptr);                  \
        break;
    switch (mc) {
        FOCR_GEMV_CASE(1, 8, 1)
        FOCR_GEMV_CASE(2, 8, 1)
        FOCR_GEMV_CASE(4, 5, 4)
        FOCR_GEMV_CASE(8, 5, 4)
        FOCR_GEMV_CASE(16, 4, 2)
        FOCR_GEMV_CASE(32, 4, 2)
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

// simd::igemm_s8s8 on device buffers through the matrix-core split-K GEMV:
// out (+)= a . b^T for batch instances (a [batch][m][k], b [batch][n][k],
// out [batch][m][n]), 16 rows per pass. hipErrorNotSupported where the shape
// does not fit it (k below 64, not a multiple of 64 or above 8192, m < 2, or
// the rows' LDS stage too large).
hipError_t launch_igemm_i8_mfma(hipStream_t s, const int8_t* a, const int8_t* b, int32_t* out, int batch, int m,
                                int k, int n) {
    // k >= 64: the kernel clamps its loads to the row's last 16-byte piece,
    // which k = 0 does not have
    if (batch < 1 || batch > 65535 || m < kMfmaMinRows || n < 1 || k < 64 || k % 64 || k > 256 * 4 * kSplitKMaxChunks)
        return hipErrorNotSupported;
    if (reinterpret_cast<uintptr_t>(a) % 16 || reinterpret_cast<uintptr_t>(b) % 16) return hipErrorNotSupported;
    const size_t lds_splitk =
        (static_cast<size_t>(m < 16 ? m : 16) * (k / 16 + 1) + (kThreads / 64) * kMfmaTileBytes / 16) * sizeof(int4);
    const size_t lds_splitk_static = (kThreads / 64) * 64 * sizeof(int4) + 16 * sizeof(float);
    if (lds_splitk + lds_splitk_static > max_lds_per_block()) return hipErrorNotSupported;
    const int cpw = ((k + 255) / 256 + 3) / 4;
    const dim3 grid(static_cast<unsigned>((n + 15) / 16), static_cast<unsigned>(batch));
    const IgemmMode im{1, static_cast<size_t>(n) * k, static_cast<size_t>(m) * k, static_cast<size_t>(m) * n};
    // Many products (a batch of experts' projections): one 16-row tile per
    // wave over the whole K, the four waves of a block sharing one staged
    // copy of the instance's activation rows, the weight chunks pipelined two
    // deep, about four blocks per CU. (The split-K form below suits a few
    // products: each block stages the activations for a single 16-row tile,
    // and its LDS admits three blocks per CU, so 64 instances' 3584 tiles took
    // five rounds of blocks.)
    const int tiles = (n + 15) / 16;
    const size_t lds_tile = (16 * static_cast<size_t>(k / 16 + 1) + (kThreads / 64) * kMfmaTileBytes / 16) * sizeof(int4);
    const int cus = 256;
    if (k % 256 == 0 && static_cast<long>(batch) * tiles >= 4L * cus && lds_tile <= 65536) {
        const long target_blocks = 4L * cus;
        int tpb = static_cast<int>((static_cast<long>(batch) * tiles + target_blocks - 1) / target_blocks);
        tpb = (tpb + 3) & ~3;  // whole rounds of the block's four waves
        const dim3 tgrid(static_cast<unsigned>((tiles + tpb - 1) / tpb), static_cast<unsigned>(batch));
        for (int r0 = 0; r0 < m; r0 += 16) {
            const int mr = m - r0 < 16 ? m - r0 : 16;
            FOCR_LAUNCH((gemv_i8_mfma_kernel<false>), tgrid, dim3(kThreads), lds_tile, s, b, nullptr, n, k,
                        a + static_cast<size_t>(r0) * k, nullptr, mr, nullptr, out + static_cast<size_t>(r0) * n,
                        nullptr, tpb, nullptr, 0, nullptr, im);
        }
        return hipGetLastError();
    }
    for (int r0 = 0; r0 < m; r0 += 16) {
        const int mr = m - r0 < 16 ? m - r0 : 16;
        const int8_t* ar = a + static_cast<size_t>(r0) * k;
        int32_t* orow = out + static_cast<size_t>(r0) * n;
        if (cpw <= 2)
            FOCR_LAUNCH((gemv_i8_mfma_splitk_kernel<2, false>), grid, dim3(kThreads), lds_splitk, s, b, nullptr, n, k,
                        ar, nullptr, mr, nullptr, orow, nullptr, nullptr, 0.0f, RopeEpi{}, im, RowAdd{});
        else if (cpw <= 4)
            FOCR_LAUNCH((gemv_i8_mfma_splitk_kernel<4, false>), grid, dim3(kThreads), lds_splitk, s, b, nullptr, n, k,
                        ar, nullptr, mr, nullptr, orow, nullptr, nullptr, 0.0f, RopeEpi{}, im, RowAdd{});
        else
            FOCR_LAUNCH((gemv_i8_mfma_splitk_kernel<8, false>), grid, dim3(kThreads), lds_splitk, s, b, nullptr, n, k,
                        ar, nullptr, mr, nullptr, orow, nullptr, nullptr, 0.0f, RopeEpi{}, im, RowAdd{});
    }
    return hipGetLastError();
}

}  // namespace focr
