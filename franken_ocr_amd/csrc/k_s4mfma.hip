// k_s4mfma.hip — int4 x int8 GEMMs on gfx950 matrix cores, and the int4 MoE
// prefill built on them (moe_block_i8's grouped structure, decoder.rs:2142-2181,
// over int4 experts; the kernel contract is s4s8_packed_kernel_scalar,
// int4.rs:304-343).
//
// The contraction. For output (m, n): for each K group g in increasing order,
// acc_i = sum over the group of a[m,k] * w[n,k] (i32), then
// acc_f = acc_f + s[n,g] * (f32)acc_i with a separate multiply and add. One
// v_mfma_i32_32x32x32_i8 covers exactly one group of 32 for a 32x32 tile, so
// it produces each group's i32 partials directly (C operand 0, no running
// accumulator); group 16 takes two MFMAs per 32 K with the other half of the
// A operand zeroed. The f32 group epilogue is then identical to the reference
// and the result is bit-exact — at a price: three VALU ops (cvt, mul, add)
// per output element per group against 32 MACs, so these kernels are bound by
// VALU issue at roughly a sixth of the int8 MFMA peak, not by the MFMA.
//
// Operand layout of v_mfma_i32_32x32x32_i8 (checked on the device): lane l
// holds A row l%32 and B column l%32, bytes k = 16*(l/32) + [0, 16) of the
// 32-wide K step; C element v of lane l is row 8*(v/4) + 4*(l/32) + v%4,
// column l%32. A B fragment is 8 packed bytes (16 nibbles, low nibble = even
// k) unpacked in registers.
//
// Block = 4 waves = a 32-row x 128-column output tile; the 32 activation rows
// (gathered through a row map) are staged once in LDS with a padded stride,
// each wave streams the packed weight rows of its 32 columns.
//
// Prefill pipeline (focr_hip_moe_prefill_i4): quantize x rows (ties-even,
// decoder.rs:1647-1656) -> plan (stable counting sort of the (token, slot)
// pairs by expert, 32-row tiles per expert) -> gate/up GEMM with the SwiGLU
// epilogue -> requantize act rows (ties-even) -> down GEMM with the
// gate-weighted epilogue -> combine each token's pairs in ascending expert
// order (the order moe_block_i8 scatters in).
#include "focr_internal.hpp"
#include "k_common.hpp"
#include "k_int4.hpp"

namespace focr {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

constexpr int BM = 32;   // rows per block
constexpr int BN = 128;  // columns per block (4 waves x 32)
constexpr int kMaxE = 64;
constexpr int kMaxK = 8;

enum Epi { kEpiPlain = 0, kEpiSwiglu = 1, kEpiDown = 2 };

// 8 packed bytes -> 16 int8 weights in k order.
__device__ __forceinline__ v4i unpack16_i4(uint2 p) {
    uint32_t w0, w1, w2, w3;
    unpack8_i4(p.x, w0, w1);
    unpack8_i4(p.y, w2, w3);
    v4i r;
    r.x = static_cast<int>(w0);
    r.y = static_cast<int>(w1);
    r.z = static_cast<int>(w2);
    r.w = static_cast<int>(w3);
    return r;
}

struct TileList {
    const int* n_tiles;  // null: implicit tiles over M rows of one expert
    const int* tile_e;
    const int* tile_r0;
    const int* tile_nr;
};

struct Operand {
    const uint8_t* b;  // [E][N][K/2]
    const float* s;    // [E][N][K/group]
};

struct EpiArgs {
    float* out;               // plain [M][N]; swiglu act [rows][N]; down ybuf [pairs][N]
    const int* perm;          // swiglu/down: permuted row -> pair id (t*top_k + j)
    const float* row_scale;   // swiglu: x scales [token]; down: act scales [row]
    const float* pair_gate;   // down: gates [pair]
    int top_k;
};

template <int NMAT, int EPI, bool G16>
__global__ __launch_bounds__(256) void s4_mfma_kernel(const int8_t* __restrict__ A, TileList tl, int M, int K, int N,
                                                      Operand op0, Operand op1, EpiArgs ep) {
    extern __shared__ int4 lds_raw[];
    int8_t* lds_a = reinterpret_cast<int8_t*>(lds_raw);  // [BM][KS]
    __shared__ int s_arow[BM];
    __shared__ int s_dst[BM];
    __shared__ float s_rs[BM];
    __shared__ float s_gate[BM];

    int e = 0, r0 = blockIdx.x * BM, nr = min(BM, M - r0);
    if (tl.n_tiles) {
        if (static_cast<int>(blockIdx.x) >= *tl.n_tiles) return;
        e = tl.tile_e[blockIdx.x];
        r0 = tl.tile_r0[blockIdx.x];
        nr = tl.tile_nr[blockIdx.x];
    }
    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int l = tid & 63;
    const int h = l >> 5;
    const int n = blockIdx.y * BN + wave * 32 + (l & 31);
    const bool col_ok = n < N;
    const int nc = col_ok ? n : N - 1;
    const int KS = K + 16;          // padded LDS row stride (bank spread)
    const int Q = K >> 5;           // 32-wide K steps
    const int G = G16 ? 2 * Q : Q;  // scale groups per row

    // weight rows of this lane's column (per matrix) and their scale rows
    const size_t wrow = static_cast<size_t>(e) * N + nc;
    const uint8_t* b0 = op0.b + wrow * (K / 2) + h * 8;
    const float* s0 = op0.s + wrow * G;
    const uint8_t* b1 = NMAT > 1 ? op1.b + wrow * (K / 2) + h * 8 : nullptr;
    const float* s1 = NMAT > 1 ? op1.s + wrow * G : nullptr;

    // first weight step (and its scales) in flight before the row map / A
    // staging round trips; each step prefetches the next
    constexpr int GPS = G16 ? 2 : 1;  // scale groups per 32-wide step
    uint2 bn0 = *reinterpret_cast<const uint2*>(b0);
    uint2 bn1 = NMAT > 1 ? *reinterpret_cast<const uint2*>(b1) : make_uint2(0u, 0u);
    float sn0[GPS], sn1[GPS];
#pragma unroll
    for (int i = 0; i < GPS; ++i) {
        sn0[i] = s0[i];
        sn1[i] = NMAT > 1 ? s1[i] : 0.0f;
    }

    // row map and epilogue row data
    if (tid < BM) {
        const int m = tid < nr ? tid : nr - 1;  // rows past the tile repeat its last row
        const int r = r0 + m;
        int arow = r, dst = r;
        float rs = 0.0f, gate = 0.0f;
        if (EPI == kEpiSwiglu) {
            arow = ep.perm[r] / ep.top_k;
            rs = ep.row_scale[arow];
        } else if (EPI == kEpiDown) {
            dst = ep.perm[r];
            rs = ep.row_scale[r];
            gate = ep.pair_gate[dst];
        }
        s_arow[tid] = arow;
        s_dst[tid] = dst;
        s_rs[tid] = rs;
        s_gate[tid] = gate;
    }
    __syncthreads();
    // stage the 32 activation rows: 16-byte chunks, four per thread per round,
    // loads issued before the stores
    {
        const int cpr = K >> 4;  // chunks per row
        const int nch = BM * cpr;
        for (int base = 0; base < nch; base += 4 * 256) {
            int4 v[4];
            int at[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int i = base + q * 256 + tid;
                const int ic = i < nch ? i : nch - 1;
                const int m = ic / cpr, c = ic - m * cpr;
                at[q] = m * KS + 16 * c;
                v[q] = reinterpret_cast<const int4*>(A + static_cast<size_t>(s_arow[m]) * K)[c];
            }
#pragma unroll
            for (int q = 0; q < 4; ++q) *reinterpret_cast<int4*>(lds_a + at[q]) = v[q];  // clamped: same value
        }
    }
    __syncthreads();

    float acc0[16], acc1[16];
#pragma unroll
    for (int v = 0; v < 16; ++v) acc0[v] = acc1[v] = 0.0f;
    const v16i zero = {};
    const int8_t* arow_lds = lds_a + (l & 31) * KS + h * 16;

    for (int q = 0; q < Q; ++q) {
        const uint2 bc0 = bn0, bc1 = bn1;
        float sc0[GPS], sc1[GPS];
#pragma unroll
        for (int i = 0; i < GPS; ++i) {
            sc0[i] = sn0[i];
            sc1[i] = sn1[i];
        }
        {  // next step's weights and scales (the last step re-reads its own: in bounds, unused)
            const int qn = q + 1 < Q ? q + 1 : q;
            bn0 = *reinterpret_cast<const uint2*>(b0 + qn * 16);
            if (NMAT > 1) bn1 = *reinterpret_cast<const uint2*>(b1 + qn * 16);
#pragma unroll
            for (int i = 0; i < GPS; ++i) {
                sn0[i] = s0[GPS * qn + i];
                if (NMAT > 1) sn1[i] = s1[GPS * qn + i];
            }
        }
        const v4i a = *reinterpret_cast<const v4i*>(arow_lds + q * 32);
        if (!G16) {
            const v16i c0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, unpack16_i4(bc0), zero, 0, 0, 0);
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const float prod = sc0[0] * static_cast<float>(c0[v]);
                acc0[v] = acc0[v] + prod;
            }
            if (NMAT > 1) {
                const v16i c1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, unpack16_i4(bc1), zero, 0, 0, 0);
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    const float prod = sc1[0] * static_cast<float>(c1[v]);
                    acc1[v] = acc1[v] + prod;
                }
            }
        } else {
            // groups 2q (k 0..15, lanes h = 0) and 2q + 1 (k 16..31, lanes h = 1)
            const v4i z4 = {0, 0, 0, 0};
            const v4i a_lo = h == 0 ? a : z4;
            const v4i a_hi = h == 1 ? a : z4;
            const v4i w0 = unpack16_i4(bc0);
            const float sa0 = sc0[0], sb0 = sc0[GPS - 1];
            const v16i c0a = __builtin_amdgcn_mfma_i32_32x32x32_i8(a_lo, w0, zero, 0, 0, 0);
            const v16i c0b = __builtin_amdgcn_mfma_i32_32x32x32_i8(a_hi, w0, zero, 0, 0, 0);
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const float pa = sa0 * static_cast<float>(c0a[v]);
                acc0[v] = acc0[v] + pa;
                const float pb = sb0 * static_cast<float>(c0b[v]);
                acc0[v] = acc0[v] + pb;
            }
            if (NMAT > 1) {
                const v4i w1 = unpack16_i4(bc1);
                const float sa1 = sc1[0], sb1 = sc1[GPS - 1];
                const v16i c1a = __builtin_amdgcn_mfma_i32_32x32x32_i8(a_lo, w1, zero, 0, 0, 0);
                const v16i c1b = __builtin_amdgcn_mfma_i32_32x32x32_i8(a_hi, w1, zero, 0, 0, 0);
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    const float pa = sa1 * static_cast<float>(c1a[v]);
                    acc1[v] = acc1[v] + pa;
                    const float pb = sb1 * static_cast<float>(c1b[v]);
                    acc1[v] = acc1[v] + pb;
                }
            }
        }
    }

    // epilogue: element v of this lane = row 8*(v/4) + 4*h + v%4, column n
#pragma unroll
    for (int v = 0; v < 16; ++v) {
        const int m = 8 * (v >> 2) + 4 * h + (v & 3);
        if (m >= nr || !col_ok) continue;
        if (EPI == kEpiPlain) {
            ep.out[static_cast<size_t>(r0 + m) * N + n] = acc0[v];
        } else if (EPI == kEpiSwiglu) {
            const float xs = s_rs[m];
            const float g = acc0[v] * xs;
            const float u = acc1[v] * xs;
            ep.out[static_cast<size_t>(r0 + m) * N + n] = silu_f(g) * u;
        } else {
            const float yv = acc0[v] * s_rs[m];
            ep.out[static_cast<size_t>(s_dst[m]) * N + n] = s_gate[m] * yv;
        }
    }
}

// ---- plan: stable counting sort of the (token, slot) pairs by expert ---------
// One block. Pairs whose expert is out of range set *err (the oracle's shape
// error). Output: perm[row] = pair id, experts' rows contiguous in increasing
// expert order, pair order kept inside an expert (= token order, then slot);
// 32-row tiles (expert, first row, row count) and their number.
constexpr int kPlanThreads = 1024;
constexpr int kPlanWaves = kPlanThreads / 64;

__global__ __launch_bounds__(kPlanThreads) void i4_plan_kernel(const uint32_t* __restrict__ idx, int TK, int E,
                                                               int* __restrict__ perm, int* __restrict__ n_tiles,
                                                               int* __restrict__ tile_e, int* __restrict__ tile_r0,
                                                               int* __restrict__ tile_nr, int* __restrict__ err) {
    __shared__ int s_cnt[kMaxE];
    __shared__ int s_base[kMaxE];
    __shared__ int s_wc[kPlanWaves][kMaxE];
    __shared__ int s_err;
    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int lane = tid & 63;
    if (tid < kMaxE) s_cnt[tid] = 0;
    for (int i = tid; i < kPlanWaves * kMaxE; i += kPlanThreads) (&s_wc[0][0])[i] = 0;
    if (tid == 0) s_err = 0;
    __syncthreads();
    for (int p = tid; p < TK; p += kPlanThreads) {
        const uint32_t e = idx[p];
        if (e >= static_cast<uint32_t>(E)) s_err = 1;
        else atomicAdd(&s_cnt[e], 1);
    }
    __syncthreads();
    if (tid == 0) {
        int run = 0;
        for (int e = 0; e < kMaxE; ++e) {
            s_base[e] = run;
            run += e < E ? s_cnt[e] : 0;
        }
    }
    __syncthreads();
    // tiles (from the counts) — thread e < 64 writes expert e's tiles
    if (tid < kMaxE) {
        const int c = tid < E ? s_cnt[tid] : 0;
        const int nt = (c + BM - 1) / BM;
        int t0 = 0;
        for (int e = 0; e < tid; ++e) t0 += (e < E ? (s_cnt[e] + BM - 1) / BM : 0);
        for (int i = 0; i < nt; ++i) {
            tile_e[t0 + i] = tid;
            tile_r0[t0 + i] = s_base[tid] + BM * i;
            tile_nr[t0 + i] = min(BM, c - BM * i);
        }
        if (tid == kMaxE - 1) *n_tiles = t0 + nt;
        if (tid == 0) *err = s_err;
    }
    // stable scatter, 1024 pairs per round: rank inside the wave by matching
    // expert ids with ballots, wave offsets from per-wave counts
    for (int c0 = 0; c0 < TK; c0 += kPlanThreads) {
        const int p = c0 + tid;
        uint32_t e = p < TK ? idx[p] : 127u;
        if (e >= static_cast<uint32_t>(E)) e = 127u;  // invalid: never placed
        unsigned long long same = ~0ull;
#pragma unroll
        for (int b = 0; b < 7; ++b) {
            const unsigned long long bm = __ballot((e >> b) & 1u);
            same &= ((e >> b) & 1u) ? bm : ~bm;
        }
        const unsigned long long lt = (1ull << lane) - 1ull;
        const int rank = __popcll(same & lt);
        if (e < 127u && (same & lt) == 0ull) s_wc[wave][e] = __popcll(same);
        __syncthreads();
        if (e < 127u) {
            int pos = s_base[e] + rank;
            for (int w = 0; w < wave; ++w) pos += s_wc[w][e];
            perm[pos] = p;
        }
        __syncthreads();
        if (tid < kMaxE) {
            int add = 0;
            for (int w = 0; w < kPlanWaves; ++w) {
                add += s_wc[w][tid];
                s_wc[w][tid] = 0;
            }
            s_base[tid] += add;
        }
        __syncthreads();
    }
}

// ---- combine: out[t] = sum of the token's pair rows in ascending expert order --
__global__ __launch_bounds__(256) void i4_combine_kernel(const float* __restrict__ ybuf,
                                                         const uint32_t* __restrict__ idx, int H, int K,
                                                         float* __restrict__ out) {
    const int t = blockIdx.y;
    const int c = blockIdx.x * 256 + threadIdx.x;
    // the token's slots sorted by (expert, slot): K <= 8, insertion order
    int order[kMaxK];
    uint32_t key[kMaxK];
    for (int j = 0; j < K; ++j) {
        const uint32_t e = idx[t * K + j];
        int at = j;
        while (at > 0 && key[at - 1] > e) {
            key[at] = key[at - 1];
            order[at] = order[at - 1];
            --at;
        }
        key[at] = e;
        order[at] = j;
    }
    if (c >= H) return;
    float o = 0.0f;
    for (int j = 0; j < K; ++j) o = o + ybuf[(static_cast<size_t>(t) * K + order[j]) * H + c];
    out[static_cast<size_t>(t) * H + c] = o;
}

template <int NMAT, int EPI, bool G16>
hipError_t launch_gemm(hipStream_t s, const int8_t* A, const TileList& tl, int grid_x, int M, int K, int N,
                       const Operand& op0, const Operand& op1, const EpiArgs& ep) {
    const size_t lds = static_cast<size_t>(BM) * (K + 16);  // <= 132 KB at K = 4096
    if (lds > 64 * 1024) {
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&s4_mfma_kernel<NMAT, EPI, G16>),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
        if (e != hipSuccess) return e;
    }
    const dim3 grid(grid_x, (N + BN - 1) / BN);
    FOCR_LAUNCH((s4_mfma_kernel<NMAT, EPI, G16>), grid, dim3(256), lds, s, A, tl, M, K, N, op0, op1, ep);
    return hipGetLastError();
}

template <int NMAT, int EPI>
hipError_t launch_gemm_g(hipStream_t s, int group, const int8_t* A, const TileList& tl, int grid_x, int M, int K,
                         int N, const Operand& op0, const Operand& op1, const EpiArgs& ep) {
    if (group == 32) return launch_gemm<NMAT, EPI, false>(s, A, tl, grid_x, M, K, N, op0, op1, ep);
    return launch_gemm<NMAT, EPI, true>(s, A, tl, grid_x, M, K, N, op0, op1, ep);
}

}  // namespace

bool s4_mfma_supported(int group, int k) {
    // 32-wide K steps with scale loads per step, LDS A tile of 32 rows of k bytes
    return (group == 16 || group == 32) && k % 32 == 0 && k > 0 && k <= 4096;
}

hipError_t launch_s4s8_mfma(hipStream_t s, const int8_t* a, const uint8_t* b, const float* scales, int group, int m,
                            int k, int n, float* out) {
    if (!s4_mfma_supported(group, k) || m <= 0 || n <= 0) return hipErrorInvalidValue;
    const TileList tl{nullptr, nullptr, nullptr, nullptr};
    const Operand op0{b, scales};
    const EpiArgs ep{out, nullptr, nullptr, nullptr, 0};
    return launch_gemm_g<1, kEpiPlain>(s, group, a, tl, (m + BM - 1) / BM, m, k, n, op0, Operand{nullptr, nullptr},
                                       ep);
}

size_t moe_i4_plan_ints(int tk, int n_experts) {
    const int max_tiles = (tk + BM - 1) / BM + n_experts;
    return static_cast<size_t>(tk) + 3 * static_cast<size_t>(max_tiles) + 2;
}

hipError_t launch_moe_prefill_i4(hipStream_t s, const focr_hip_moe_layer_i4* L, const float* x, int t, int top_k,
                                 const uint32_t* idx, const float* gates, float* out, MoeI4Scratch& w,
                                 focr_hip_ctx* ctx) {
    const int H = static_cast<int>(L->hidden), I = static_cast<int>(L->inter), E = static_cast<int>(L->n_experts);
    const int group = static_cast<int>(L->group);
    const int TK = t * top_k;
    const int max_tiles = (TK + BM - 1) / BM + E;
    int* perm = w.plan;
    int* tile_e = perm + TK;
    int* tile_r0 = tile_e + max_tiles;
    int* tile_nr = tile_r0 + max_tiles;
    int* n_tiles = tile_nr + max_tiles;
    hipError_t e;
    {
        ProfScope ps(ctx, "i4_quantize_x");
        if ((e = launch_quantize_rows(s, x, t, H, w.xq, w.xs, true)) != hipSuccess) return e;
    }
    {
        ProfScope ps(ctx, "i4_plan");
        FOCR_LAUNCH(i4_plan_kernel, dim3(1), dim3(kPlanThreads), 0, s, idx, TK, E, perm, n_tiles, tile_e, tile_r0,
                    tile_nr, w.err);
        if ((e = hipGetLastError()) != hipSuccess) return e;
    }
    const TileList tl{n_tiles, tile_e, tile_r0, tile_nr};
    {
        ProfScope ps(ctx, "i4_gate_up");
        const EpiArgs ep{w.act, perm, w.xs, nullptr, top_k};
        if ((e = launch_gemm_g<2, kEpiSwiglu>(s, group, w.xq, tl, max_tiles, TK, H, I, Operand{L->wg, L->sg},
                                              Operand{L->wu, L->su}, ep)) != hipSuccess)
            return e;
    }
    {
        ProfScope ps(ctx, "i4_quantize_act");
        if ((e = launch_quantize_rows(s, w.act, TK, I, w.aq, w.as, true)) != hipSuccess) return e;
    }
    {
        ProfScope ps(ctx, "i4_down");
        const EpiArgs ep{w.ybuf, perm, w.as, gates, top_k};
        if ((e = launch_gemm_g<1, kEpiDown>(s, group, w.aq, tl, max_tiles, TK, I, H, Operand{L->wd, L->sd},
                                           Operand{nullptr, nullptr}, ep)) != hipSuccess)
            return e;
    }
    {
        ProfScope ps(ctx, "i4_combine");
        FOCR_LAUNCH(i4_combine_kernel, dim3((H + 255) / 256, t), dim3(256), 0, s, w.ybuf, idx, H, top_k, out);
        if ((e = hipGetLastError()) != hipSuccess) return e;
    }
    return hipSuccess;
}

}  // namespace focr
