// k_s4mfma.hip — int4 x int8 GEMMs on gfx950 matrix cores, and the int4 MoE
// prefill built on them (moe_block_i8's grouped structure, decoder.rs:2142-2181,
// over int4 experts; the kernel contract is s4s8_packed_kernel_scalar,
// int4.rs:304-343).
//
// The contraction. For output (m, n): for each K group g in increasing order,
// acc_i = sum over the group of a[m,k] * w[n,k] (i32), then
// acc_f = acc_f + s[n,g] * (f32)acc_i with a separate multiply and add. One
// v_mfma_i32_32x32x32_i8 covers exactly one group of 32 for a 32x32 tile, so
// it produces each group's i32 partials directly (no running accumulator;
// the weights enter as offset nibbles with the offset folded into the
// accumulator's start, see unpack16_u4); group 16 takes two MFMAs per 32 K
// with the other half of the A operand zeroed. The f32 group epilogue is then identical to the reference
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
// Block = 4 waves over 32 rows; each wave streams the packed weight rows of
// 32 columns of one matrix; the 32 activation rows (gathered through a row
// map) are staged in LDS one K chunk at a time.
//
// Prefill pipeline (focr_hip_moe_prefill_i4): quantize x rows (ties-even,
// decoder.rs:1647-1656) -> plan (stable counting sort of the (token, slot)
// pairs by expert, 32-row tiles per expert) -> gate/up GEMM with the SwiGLU
// epilogue -> requantize act rows (ties-even) -> down GEMM with the
// gate-weighted epilogue -> combine each token's pairs in ascending expert
// order (the order moe_block_i8 scatters in).
#include "focr_internal.hpp"
#include "k_common.hpp"

namespace focr {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

constexpr int BM = 32;  // rows per block
constexpr int kMaxE = 64;
constexpr int kMaxK = 8;

enum Epi { kEpiPlain = 0, kEpiSwiglu = 1, kEpiDown = 2 };

// Offset nibbles. A two's-complement nibble n (value n - 16 [n >= 8]) XOR 8
// is u = value + 8 in [0, 15], so sum_k a_k * w_k = sum_k a_k * u_k - 8 sum_k a_k:
// the kernels feed u_k straight to the signed MFMA (no per-byte sign
// extension) and start its accumulator at -8 sum_k a_k, which one more MFMA
// against a constant -8 operand gives. The i32 result is the exact group dot.
// 8 packed bytes already XOR-ed with 0x88 -> 16 bytes u_k in k order
// (v_perm_b32 selector bytes 0-3 pick from the second operand, 4-7 from the
// first; low nibble = even k).
__device__ __forceinline__ v4i unpack16_u4(uint2 p) {
    const uint32_t lo0 = p.x & 0x0F0F0F0Fu, hi0 = (p.x >> 4) & 0x0F0F0F0Fu;
    const uint32_t lo1 = p.y & 0x0F0F0F0Fu, hi1 = (p.y >> 4) & 0x0F0F0F0Fu;
    v4i r;
    r.x = static_cast<int>(__builtin_amdgcn_perm(hi0, lo0, 0x05010400u));
    r.y = static_cast<int>(__builtin_amdgcn_perm(hi0, lo0, 0x07030602u));
    r.z = static_cast<int>(__builtin_amdgcn_perm(hi1, lo1, 0x05010400u));
    r.w = static_cast<int>(__builtin_amdgcn_perm(hi1, lo1, 0x07030602u));
    return r;
}

constexpr uint32_t kNibbleFlip = 0x88888888u;

struct TileList {
    const int* n_tiles;  // null: implicit tiles over M rows of one expert
    const int* tile_e;
    const int* tile_r0;
    const int* tile_nr;
};

// One weight operand: packed nibbles and group scales, either in the
// reference layout ([E][N][K/2], [E][N][K/group]) or in the MFMA-tiled
// layout the int4 layer keeps on the device (see retile_* below): for
// column tile nt = n/32, step q, half h = k-half, column c = n%32, the
// fragment of lane (h, c) is 8 bytes at (((e*NT + nt)*Q + q)*2 + h)*32 + c
// (in 8-byte units, nibbles stored XOR 8 — see unpack16_u4) and its scale at
// ((e*NT + nt)*G + g)*32 + c — so a wave's per-step loads are 512 and 128
// contiguous bytes.
struct Operand {
    const uint8_t* b;
    const float* s;
};

struct EpiArgs {
    float* out;               // plain [M][N]; swiglu act [rows][N]; down ybuf [pairs][N]
    const int* perm;          // swiglu/down: permuted row -> pair id (t*top_k + j)
    const float* row_scale;   // swiglu: x scales [token]; down: act scales [row]
    const float* pair_gate;   // down: gates [pair]
    int top_k;
};

constexpr int PF = 4;   // 32-wide K steps per prefetch block (two blocks in flight)
constexpr int QC = 16;  // K steps of A staged in LDS at a time (a multiple of 2 * PF)
// Bytes / floats the tiled weight and scale arrays carry past their end, so
// the prefetch of steps beyond a row's last one stays in bounds unclamped.
constexpr size_t kTilePadBytes = 16384;

template <bool G16>
struct StepFrag {
    static constexpr int GPS = G16 ? 2 : 1;  // scale groups per step
    uint2 b;
    float s[GPS];
};

// EXACT: acc = acc + s * (f32)acc_i with two roundings (the reference's
// order, bit-exact); otherwise one FMA per group (the prefill path, whose
// output is compared within a tolerance anyway).
template <bool EXACT>
__device__ __forceinline__ float group_acc(float acc, float s, int c) {
    if (EXACT) {
        const float prod = s * static_cast<float>(c);
        return acc + prod;
    }
    return __builtin_fmaf(s, static_cast<float>(c), acc);
}

// Columns per block: plain/down — 4 waves x 32 columns of one matrix; SwiGLU —
// 2 x 32 columns, waves 0-1 on the gate matrix and 2-3 on the up matrix for
// the same columns, the up waves handing their tile to the gate waves
// through LDS for the epilogue (one matrix stream per wave keeps the
// registers, and so the occupancy, of the single-matrix kernel).
template <int EPI>
constexpr int block_cols() {
    return EPI == kEpiSwiglu ? 64 : 128;
}

template <int EPI, bool G16, bool TILED, bool EXACT>
__global__ __launch_bounds__(256) void s4_mfma_kernel(const int8_t* __restrict__ A, TileList tl, int M, int K, int N,
                                                      Operand op0, Operand op1, EpiArgs ep) {
    extern __shared__ int4 lds_raw[];
    int8_t* lds_a = reinterpret_cast<int8_t*>(lds_raw);  // [BM][KS]; after the K loop: SwiGLU exchange
    __shared__ int s_arow[BM];
    __shared__ int s_dst[BM];
    __shared__ float s_rs[BM];
    __shared__ float s_gate[BM];
    constexpr int GPS = G16 ? 2 : 1;
    constexpr int BNB = block_cols<EPI>();

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
    const bool up_wave = EPI == kEpiSwiglu && wave >= 2;
    const int wcol = EPI == kEpiSwiglu ? (wave & 1) : wave;  // this wave's 32-column slice in the block
    const int n = blockIdx.y * BNB + wcol * 32 + (l & 31);
    const bool col_ok = n < N;
    const int nc = col_ok ? n : N - 1;
    const int KS = QC * 32 + 16;  // LDS row stride: one K chunk plus bank-spreading pad
    const int Q = K >> 5;         // 32-wide K steps
    const int G = GPS * Q;        // scale groups per row

    // this wave's fragment stream (one matrix)
    const Operand op = up_wave ? op1 : op0;
    const uint8_t* bp;
    const float* sp;
    if (TILED) {
        const size_t tile = static_cast<size_t>(e) * (N >> 5) + (nc >> 5);
        bp = op.b + (tile * Q * 2 + h) * 256 + (nc & 31) * 8;
        sp = op.s + tile * G * 32 + (nc & 31);
    } else {
        const size_t wrow = static_cast<size_t>(e) * N + nc;
        bp = op.b + wrow * (K / 2) + h * 8;
        sp = op.s + wrow * G;
    }
    constexpr int bstep = TILED ? 512 : 16;  // bytes between consecutive steps
    constexpr int sstep = TILED ? 32 : 1;    // floats between consecutive groups
    auto load_block = [&](int q0, StepFrag<G16> (&f)[PF]) {
#pragma unroll
        for (int i = 0; i < PF; ++i) {
            // past the end: the tiled arrays are padded (unclamped addresses fold
            // into immediate offsets); the reference layout re-reads its last step
            const int q = TILED ? q0 + i : min(q0 + i, Q - 1);
            uint2 b = *reinterpret_cast<const uint2*>(bp + static_cast<size_t>(q) * bstep);
            if (!TILED) {  // the tiled layout stores the nibbles already flipped
                b.x ^= kNibbleFlip;
                b.y ^= kNibbleFlip;
            }
            f[i].b = b;
#pragma unroll
            for (int g = 0; g < GPS; ++g) f[i].s[g] = sp[static_cast<size_t>(GPS * q + g) * sstep];
        }
    };

    StepFrag<G16> fa[PF], fb[PF];
    load_block(0, fa);  // in flight across the row map / A staging round trips

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

    float acc[16];
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[v] = 0.0f;
    const v16i zero = {};
    const int8_t* arow_lds = lds_a + (l & 31) * KS + h * 16;
    const v4i neg8 = {static_cast<int>(0xF8F8F8F8u), static_cast<int>(0xF8F8F8F8u), static_cast<int>(0xF8F8F8F8u),
                      static_cast<int>(0xF8F8F8F8u)};
    // qa: the step's offset inside the staged K chunk
    auto step = [&](int qa, const StepFrag<G16>& f) {
        const v4i a = *reinterpret_cast<const v4i*>(arow_lds + qa * 32);
        const v4i w = unpack16_u4(f.b);
        if (!G16) {
            const v16i corr = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, neg8, zero, 0, 0, 0);  // -8 sum a
            const v16i c = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, w, corr, 0, 0, 0);
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[v] = group_acc<EXACT>(acc[v], f.s[0], c[v]);
        } else {
            // groups 2q (k 0..15, lanes h = 0) and 2q + 1 (k 16..31, lanes h = 1)
            const v4i z4 = {0, 0, 0, 0};
            const v4i a_lo = h == 0 ? a : z4;
            const v4i a_hi = h == 1 ? a : z4;
            const v16i corr_lo = __builtin_amdgcn_mfma_i32_32x32x32_i8(a_lo, neg8, zero, 0, 0, 0);
            const v16i ca = __builtin_amdgcn_mfma_i32_32x32x32_i8(a_lo, w, corr_lo, 0, 0, 0);
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[v] = group_acc<EXACT>(acc[v], f.s[0], ca[v]);
            const v16i corr_hi = __builtin_amdgcn_mfma_i32_32x32x32_i8(a_hi, neg8, zero, 0, 0, 0);
            const v16i cb = __builtin_amdgcn_mfma_i32_32x32x32_i8(a_hi, w, corr_hi, 0, 0, 0);
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[v] = group_acc<EXACT>(acc[v], f.s[GPS - 1], cb[v]);
        }
    };

    // K in chunks of QC steps: stage the 32 activation rows' chunk in LDS
    // (16-byte pieces, loads issued before the stores), then run its steps
    // with two blocks of PF steps of weights in flight.
    for (int c0 = 0; c0 < Q; c0 += QC) {
        const int qn = min(QC, Q - c0);
        if (c0) __syncthreads();  // every wave is done with the previous chunk
        {
            const int cpr = qn * 2;  // 16-byte pieces per row in this chunk
            const int nch = BM * cpr;
            for (int base = 0; base < nch; base += 4 * 256) {
                int4 v[4];
                int at[4];
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const int i = base + u * 256 + tid;
                    const int ic = i < nch ? i : nch - 1;
                    const int m = ic / cpr, c = ic - m * cpr;
                    at[u] = m * KS + 16 * c;
                    v[u] = reinterpret_cast<const int4*>(A + static_cast<size_t>(s_arow[m]) * K + c0 * 32)[c];
                }
#pragma unroll
                for (int u = 0; u < 4; ++u) *reinterpret_cast<int4*>(lds_a + at[u]) = v[u];  // clamped: same value
            }
        }
        __syncthreads();
        for (int q0 = c0; q0 < c0 + qn; q0 += 2 * PF) {
            load_block(q0 + PF, fb);
#pragma unroll
            for (int i = 0; i < PF; ++i)
                if (q0 + i < c0 + qn) step(q0 + i - c0, fa[i]);
            load_block(q0 + 2 * PF, fa);
#pragma unroll
            for (int i = 0; i < PF; ++i)
                if (q0 + PF + i < c0 + qn) step(q0 + PF + i - c0, fb[i]);
        }
    }

    // epilogue: element v of this lane = row 8*(v/4) + 4*h + v%4, column n
    if (EPI == kEpiSwiglu) {
        float* xu = reinterpret_cast<float*>(lds_a);  // [BM][64] up tile
        __syncthreads();                              // A chunk no longer read
        if (up_wave) {
#pragma unroll
            for (int v = 0; v < 16; ++v) xu[(8 * (v >> 2) + 4 * h + (v & 3)) * 64 + wcol * 32 + (l & 31)] = acc[v];
        }
        __syncthreads();
        if (up_wave) return;
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const int m = 8 * (v >> 2) + 4 * h + (v & 3);
            if (m >= nr || !col_ok) continue;
            const float xs = s_rs[m];
            const float g = acc[v] * xs;
            const float u = xu[m * 64 + wcol * 32 + (l & 31)] * xs;
            ep.out[static_cast<size_t>(r0 + m) * N + n] = silu_f(g) * u;
        }
        return;
    }
#pragma unroll
    for (int v = 0; v < 16; ++v) {
        const int m = 8 * (v >> 2) + 4 * h + (v & 3);
        if (m >= nr || !col_ok) continue;
        if (EPI == kEpiPlain) {
            ep.out[static_cast<size_t>(r0 + m) * N + n] = acc[v];
        } else {
            const float yv = acc[v] * s_rs[m];
            ep.out[static_cast<size_t>(s_dst[m]) * N + n] = s_gate[m] * yv;
        }
    }
}

// ---- the int4 layer's MFMA-tiled weight layout -------------------------------
// Destination-ordered copies (8-byte units for the nibbles, stored as offset
// nibbles; floats for the scales), one thread per unit.
__global__ __launch_bounds__(256) void retile_b_kernel(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst,
                                                       size_t units, int N, int K) {
    const size_t d = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x;
    if (d >= units) return;
    const int Q = K >> 5, NT = N >> 5;
    const int c = static_cast<int>(d & 31);
    size_t r = d >> 5;
    const int h = static_cast<int>(r & 1);
    r >>= 1;
    const int q = static_cast<int>(r % Q);
    r /= Q;
    const int nt = static_cast<int>(r % NT);
    const size_t e = r / NT;
    const size_t row = e * N + static_cast<size_t>(nt) * 32 + c;
    uint2 v = *reinterpret_cast<const uint2*>(src + row * (K / 2) + q * 16 + h * 8);
    v.x ^= kNibbleFlip;  // stored as offset nibbles u = n ^ 8
    v.y ^= kNibbleFlip;
    reinterpret_cast<uint2*>(dst)[d] = v;
}

__global__ __launch_bounds__(256) void retile_s_kernel(const float* __restrict__ src, float* __restrict__ dst,
                                                       size_t units, int N, int G) {
    const size_t d = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x;
    if (d >= units) return;
    const int NT = N >> 5;
    const int c = static_cast<int>(d & 31);
    size_t r = d >> 5;
    const int g = static_cast<int>(r % G);
    r /= G;
    const int nt = static_cast<int>(r % NT);
    const size_t e = r / NT;
    dst[d] = src[(e * N + static_cast<size_t>(nt) * 32 + c) * G + g];
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
// The token's slots sorted by (expert, slot): slot j's rank counts the slots
// ahead of it, the first K threads publish order[rank] = j.
__global__ __launch_bounds__(256) void i4_combine_kernel(const float* __restrict__ ybuf,
                                                         const uint32_t* __restrict__ idx, int H, int K,
                                                         float* __restrict__ out) {
    __shared__ int s_order[kMaxK];
    const int t = blockIdx.y;
    const int c = blockIdx.x * 256 + threadIdx.x;
    if (threadIdx.x < K) {
        const int j = threadIdx.x;
        const uint32_t ej = idx[t * K + j];
        int rank = 0;
        for (int i = 0; i < K; ++i) {
            const uint32_t ei = idx[t * K + i];
            rank += (ei < ej || (ei == ej && i < j)) ? 1 : 0;
        }
        s_order[rank] = j;
    }
    __syncthreads();
    if (c >= H) return;
    float v[kMaxK];
#pragma unroll
    for (int j = 0; j < kMaxK; ++j)  // unconditional loads (slot clamped), summed below only for j < K
        v[j] = ybuf[(static_cast<size_t>(t) * K + s_order[j < K ? j : K - 1]) * H + c];
    float o = 0.0f;
#pragma unroll
    for (int j = 0; j < kMaxK; ++j)
        if (j < K) o = o + v[j];
    out[static_cast<size_t>(t) * H + c] = o;
}

template <int EPI, bool G16, bool TILED, bool EXACT>
hipError_t launch_gemm(hipStream_t s, const int8_t* A, const TileList& tl, int grid_x, int M, int K, int N,
                       const Operand& op0, const Operand& op1, const EpiArgs& ep) {
    const size_t lds = static_cast<size_t>(BM) * (QC * 32 + 16);  // one staged K chunk: 16.5 KB
    constexpr int BNB = block_cols<EPI>();
    const dim3 grid(grid_x, (N + BNB - 1) / BNB);
    FOCR_LAUNCH((s4_mfma_kernel<EPI, G16, TILED, EXACT>), grid, dim3(256), lds, s, A, tl, M, K, N, op0, op1, ep);
    return hipGetLastError();
}

template <int EPI, bool TILED, bool EXACT>
hipError_t launch_gemm_g(hipStream_t s, int group, const int8_t* A, const TileList& tl, int grid_x, int M, int K,
                         int N, const Operand& op0, const Operand& op1, const EpiArgs& ep) {
    if (group == 32) return launch_gemm<EPI, false, TILED, EXACT>(s, A, tl, grid_x, M, K, N, op0, op1, ep);
    return launch_gemm<EPI, true, TILED, EXACT>(s, A, tl, grid_x, M, K, N, op0, op1, ep);
}

}  // namespace

bool s4_mfma_supported(int group, int k) {
    return (group == 16 || group == 32) && k % 32 == 0 && k > 0 && k <= 16384;
}

size_t s4_tile_pad_bytes() { return kTilePadBytes; }

hipError_t launch_s4s8_mfma(hipStream_t s, const int8_t* a, const uint8_t* b, const float* scales, int group, int m,
                            int k, int n, float* out) {
    if (!s4_mfma_supported(group, k) || m <= 0 || n <= 0) return hipErrorInvalidValue;
    const TileList tl{nullptr, nullptr, nullptr, nullptr};
    const Operand op0{b, scales};
    const EpiArgs ep{out, nullptr, nullptr, nullptr, 0};
    return launch_gemm_g<kEpiPlain, false, true>(s, group, a, tl, (m + BM - 1) / BM, m, k, n, op0,
                                                    Operand{nullptr, nullptr}, ep);
}

hipError_t launch_retile_i4(hipStream_t s, const uint8_t* b, const float* sc, int n_experts, int n, int k, int group,
                            uint8_t* b_tiled, float* s_tiled) {
    if (n % 32 || k % 32) return hipErrorInvalidValue;
    const size_t bu = static_cast<size_t>(n_experts) * n * k / 16;
    FOCR_LAUNCH(retile_b_kernel, dim3(static_cast<unsigned>((bu + 255) / 256)), dim3(256), 0, s, b, b_tiled, bu, n, k);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const int G = k / group;
    const size_t su = static_cast<size_t>(n_experts) * n * G;
    FOCR_LAUNCH(retile_s_kernel, dim3(static_cast<unsigned>((su + 255) / 256)), dim3(256), 0, s, sc, s_tiled, su, n, G);
    return hipGetLastError();
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
        if ((e = launch_gemm_g<kEpiSwiglu, true, false>(s, group, w.xq, tl, max_tiles, TK, H, I,
                                                           Operand{L->wg, L->sg}, Operand{L->wu, L->su}, ep)) !=
            hipSuccess)
            return e;
    }
    {
        ProfScope ps(ctx, "i4_quantize_act");
        if ((e = launch_quantize_rows(s, w.act, TK, I, w.aq, w.as, true)) != hipSuccess) return e;
    }
    {
        ProfScope ps(ctx, "i4_down");
        const EpiArgs ep{w.ybuf, perm, w.as, gates, top_k};
        if ((e = launch_gemm_g<kEpiDown, true, false>(s, group, w.aq, tl, max_tiles, TK, I, H,
                                                         Operand{L->wd, L->sd}, Operand{nullptr, nullptr}, ep)) !=
            hipSuccess)
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
