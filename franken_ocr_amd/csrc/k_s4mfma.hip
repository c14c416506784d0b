// k_s4mfma.hip — int4 x int8 GEMMs on gfx950 matrix cores, and the int4 MoE
// prefill built on them (moe_block_i8's grouped structure, decoder.rs:2142-2181,
// over int4 experts; the kernel contract is s4s8_packed_kernel_scalar,
// int4.rs:304-343).
//
// The contraction. For output (m, n): for each K group g in increasing order,
// acc_i = sum over the group of a[m,k] * w[n,k] (i32), then
// acc_f = acc_f + s[n,g] * (f32)acc_i with a separate multiply and add. One
// v_mfma_i32_32x32x32_i8 covers exactly one group of 32 for a 32x32 tile, so
// it produces each group's i32 partials directly (no running accumulator);
// group 16 takes two MFMAs per 32 K with the other half of the A operand
// zeroed.
//
// Weights enter the MFMA as 16 * w: a packed byte holds w[2j] in its low
// nibble and w[2j+1] in its high one, and (byte & 0xF0) is the signed byte
// 16 * w[2j+1], ((byte << 4) & 0xF0) the signed byte 16 * w[2j] — one AND, or
// a shift and an AND, per four weights, no sign extension. The k order this
// leaves in a 16-byte fragment, [0 2 4 6 1 3 5 7 8 10 12 14 9 11 13 15], is
// applied to the activations when they are staged in LDS, so the MFMA's i32
// result is exactly 16 * (the group's dot product). The reference-exact
// epilogue shifts it back (>> 4, exact) and does the reference's
// (f32)acc_i, multiply, add; the prefill path folds the 16 into the final
// scale instead (one FMA per element and group, f32 output within
// tolerance). The per-group f32 epilogue is VALU work (two or three ops per
// output element per 32 MACs), which is what bounds these kernels, not the
// MFMA: each weight fragment is loaded and unpacked once per wave and feeds
// two 32-row MFMA tiles.
//
// Operand layout of v_mfma_i32_32x32x32_i8 (checked on the device): lane l
// holds A row l%32 and B column l%32, bytes k = 16*(l/32) + [0, 16) of the
// 32-wide K step; C element v of lane l is row 8*(v/4) + 4*(l/32) + v%4,
// column l%32.
//
// Block = 4 waves over a 64-row tile (two 32-row MFMA tiles per wave); each
// wave streams the packed weights of 32 columns of one matrix; the 64
// activation rows (gathered through a row map) are staged in LDS one K chunk
// at a time.
//
// Prefill pipeline (focr_hip_moe_prefill_i4): quantize x rows (ties-even,
// decoder.rs:1647-1656) and plan (stable counting sort of the (token, slot)
// pairs by expert, 64-row tiles per expert) in one launch -> gate/up GEMM
// with the SwiGLU epilogue -> requantize act rows (ties-even) -> down GEMM
// with the gate-weighted epilogue -> combine each token's pairs in ascending
// expert order (the order moe_block_i8 scatters in).
#include "focr_internal.hpp"
#include "k_common.hpp"

namespace focr {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

constexpr int BM = 64;  // rows per block tile (two 32-row MFMA tiles per wave)
constexpr int kMaxE = 64;
constexpr int kMaxK = 8;

enum Epi { kEpiPlain = 0, kEpiSwiglu = 1, kEpiDown = 2 };

// 8 packed bytes (16 nibbles, low nibble = even k) -> 16 signed bytes 16 * w
// in the k order [0 2 4 6 1 3 5 7 | 8 10 12 14 9 11 13 15].
__device__ __forceinline__ v4i unpack16_x16(uint2 p) {
    v4i r;
    r.x = static_cast<int>((p.x << 4) & 0xF0F0F0F0u);
    r.y = static_cast<int>(p.x & 0xF0F0F0F0u);
    r.z = static_cast<int>((p.y << 4) & 0xF0F0F0F0u);
    r.w = static_cast<int>(p.y & 0xF0F0F0F0u);
    return r;
}

// 16 activation bytes in k order -> the order unpack16_x16 leaves the
// weights in (v_perm_b32: selector bytes 0-3 pick the second operand's
// bytes, 4-7 the first's).
__device__ __forceinline__ int4 perm16_a(int4 a) {
    int4 r;
    r.x = static_cast<int>(__builtin_amdgcn_perm(static_cast<uint32_t>(a.y), static_cast<uint32_t>(a.x), 0x06040200u));
    r.y = static_cast<int>(__builtin_amdgcn_perm(static_cast<uint32_t>(a.y), static_cast<uint32_t>(a.x), 0x07050301u));
    r.z = static_cast<int>(__builtin_amdgcn_perm(static_cast<uint32_t>(a.w), static_cast<uint32_t>(a.z), 0x06040200u));
    r.w = static_cast<int>(__builtin_amdgcn_perm(static_cast<uint32_t>(a.w), static_cast<uint32_t>(a.z), 0x07050301u));
    return r;
}

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
// (in 8-byte units) and its scale at ((e*NT + nt)*G + g)*32 + c — so a
// wave's per-step loads are 512 and 128 contiguous bytes.
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

constexpr int PF = 3;   // 32-wide K steps per prefetch block (two blocks in flight)
constexpr int QC = 6;   // K steps of A staged in LDS at a time (a multiple of 2 * PF)
constexpr int KS = QC * 32 + 16;  // LDS row stride: one K chunk plus a bank-spreading pad
constexpr int kChunkBytes = BM * KS;  // one staged chunk; two are kept
// Bytes / floats the tiled weight and scale arrays carry past their end, so
// the prefetch of steps beyond a row's last one stays in bounds unclamped.
constexpr size_t kTilePadBytes = 16384;

template <bool G16>
struct StepFrag {
    static constexpr int GPS = G16 ? 2 : 1;  // scale groups per step
    uint2 b;
    float s[GPS];
};

// EXACT: the reference's acc = acc + s * (f32)acc_i (c = 16 * acc_i, shifted
// back exactly; two roundings, bit-exact); otherwise one FMA on 16 * acc_i,
// the 16 divided out of the final value (exact: a power of two).
template <bool EXACT>
__device__ __forceinline__ float group_acc(float acc, float s, int c) {
    if (EXACT) {
        const float prod = s * static_cast<float>(c >> 4);
        return acc + prod;
    }
    return __builtin_fmaf(s, static_cast<float>(c), acc);
}

// Columns per block: plain/down — 4 waves x 32 columns of one matrix;
// SwiGLU — 2 x 32 columns, waves 0 and 2 on the gate matrix, 1 and 3 on the
// up matrix for the same columns, the up waves handing their tile to the
// gate waves through LDS for the epilogue.
template <int EPI>
constexpr int block_cols() {
    return EPI == kEpiSwiglu ? 64 : 128;
}

// One block tile: rows [r0, r0 + nr) of expert e's tile (nr <= 64) against
// column block cb. Every thread of the block calls it (it synchronises).
template <int EPI, bool G16, bool TILED, bool EXACT>
__device__ __forceinline__ void s4_tile(const int8_t* __restrict__ A, int K, int N, const Operand& op0,
                                        const Operand& op1, const EpiArgs& ep, int e, int r0, int nr, int cb) {
    extern __shared__ int4 lds_raw[];
    int8_t* lds_a = reinterpret_cast<int8_t*>(lds_raw);  // 2 x [BM][KS]; after the K loop: SwiGLU exchange
    __shared__ int s_arow[BM];
    __shared__ int s_dst[BM];
    __shared__ float s_rs[BM];
    __shared__ float s_gate[BM];
    constexpr int GPS = G16 ? 2 : 1;
    constexpr int BNB = block_cols<EPI>();
    constexpr float kOut = EXACT ? 1.0f : 0.0625f;  // divides out the 16 of the weight operand

    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int l = tid & 63;
    const int h = l >> 5;
    const bool up_wave = EPI == kEpiSwiglu && (wave & 1);
    const int wcol = EPI == kEpiSwiglu ? (wave >> 1) : wave;  // this wave's 32-column slice in the block
    const int n = cb * BNB + wcol * 32 + (l & 31);
    const bool col_ok = n < N;
    const int nc = col_ok ? n : N - 1;
    const bool two = nr > 32;  // the second 32-row tile has rows
    const int Q = K >> 5;      // 32-wide K steps
    const int G = GPS * Q;     // scale groups per row

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
            f[i].b = *reinterpret_cast<const uint2*>(bp + static_cast<size_t>(q) * bstep);
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

    float acc0[16], acc1[16];
#pragma unroll
    for (int v = 0; v < 16; ++v) acc0[v] = acc1[v] = 0.0f;
    const v16i zero = {};
    int boff = 0;  // the staged chunk's LDS buffer
    const int8_t* arow0 = lds_a + (l & 31) * KS + h * 16;
    const int8_t* arow1 = arow0 + 32 * KS;
    // qa: the step's offset inside the staged K chunk
    auto step = [&](int qa, const StepFrag<G16>& f) {
        const v4i w = unpack16_x16(f.b);
        const v4i a0 = *reinterpret_cast<const v4i*>(arow0 + boff + qa * 32);
        if (!G16) {
            const v16i c0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a0, w, zero, 0, 0, 0);
#pragma unroll
            for (int v = 0; v < 16; ++v) acc0[v] = group_acc<EXACT>(acc0[v], f.s[0], c0[v]);
            if (two) {
                const v4i a1 = *reinterpret_cast<const v4i*>(arow1 + boff + qa * 32);
                const v16i c1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a1, w, zero, 0, 0, 0);
#pragma unroll
                for (int v = 0; v < 16; ++v) acc1[v] = group_acc<EXACT>(acc1[v], f.s[0], c1[v]);
            }
        } else {
            // groups 2q (k 0..15, lanes h = 0) and 2q + 1 (k 16..31, lanes h = 1)
            const v4i z4 = {0, 0, 0, 0};
            {
                const v16i ca = __builtin_amdgcn_mfma_i32_32x32x32_i8(h == 0 ? a0 : z4, w, zero, 0, 0, 0);
                const v16i cb = __builtin_amdgcn_mfma_i32_32x32x32_i8(h == 1 ? a0 : z4, w, zero, 0, 0, 0);
#pragma unroll
                for (int v = 0; v < 16; ++v) acc0[v] = group_acc<EXACT>(acc0[v], f.s[0], ca[v]);
#pragma unroll
                for (int v = 0; v < 16; ++v) acc0[v] = group_acc<EXACT>(acc0[v], f.s[GPS - 1], cb[v]);
            }
            if (two) {
                const v4i a1 = *reinterpret_cast<const v4i*>(arow1 + boff + qa * 32);
                const v16i ca = __builtin_amdgcn_mfma_i32_32x32x32_i8(h == 0 ? a1 : z4, w, zero, 0, 0, 0);
                const v16i cb = __builtin_amdgcn_mfma_i32_32x32x32_i8(h == 1 ? a1 : z4, w, zero, 0, 0, 0);
#pragma unroll
                for (int v = 0; v < 16; ++v) acc1[v] = group_acc<EXACT>(acc1[v], f.s[0], ca[v]);
#pragma unroll
                for (int v = 0; v < 16; ++v) acc1[v] = group_acc<EXACT>(acc1[v], f.s[GPS - 1], cb[v]);
            }
        }
    };

    // K in chunks of QC steps, the tile's activation rows for each chunk
    // staged in LDS (16-byte pieces in the weights' k order) in two buffers:
    // the next chunk's loads are issued before the current chunk's steps and
    // stored after them. Issued any later, they would queue behind the
    // weight prefetches (memory counters retire in order) and every chunk
    // would drain the weight stream.
    const int rows_staged = two ? BM : 32;
    constexpr int APT = (BM * QC * 2 + 255) / 256;  // pieces per thread and chunk
    int4 va[APT];
    int vat[APT];
    // a full chunk's pieces of this thread: the same rows, columns and LDS
    // offsets in every full chunk, so they are worked out once per tile (the
    // division by the pieces per row is a software division)
    const int8_t* fsrc[APT];
    int fvat[APT];
#pragma unroll
    for (int u = 0; u < APT; ++u) {
        constexpr int cpr = 2 * QC;
        const int i = u * 256 + tid, nch = rows_staged * cpr;
        const int ic = i < nch ? i : nch - 1;  // past the end: a duplicate of the last piece
        const int m = ic / cpr, c = ic - m * cpr;
        fvat[u] = m * KS + 16 * c;
        fsrc[u] = A + static_cast<size_t>(s_arow[m]) * K + 16 * c;
    }
    auto load_a = [&](int c0) {
        const int cpr = min(QC, Q - c0) * 2;  // 16-byte pieces per row in the chunk
        if (cpr == 2 * QC) {
#pragma unroll
            for (int u = 0; u < APT; ++u) {
                vat[u] = fvat[u];
                va[u] = *reinterpret_cast<const int4*>(fsrc[u] + c0 * 32);
            }
            return;
        }
        const int nch = rows_staged * cpr;
#pragma unroll
        for (int u = 0; u < APT; ++u) {
            const int i = u * 256 + tid;
            const int ic = i < nch ? i : nch - 1;  // past the end: a duplicate of the last piece
            const int m = ic / cpr, c = ic - m * cpr;
            vat[u] = m * KS + 16 * c;
            va[u] = reinterpret_cast<const int4*>(A + static_cast<size_t>(s_arow[m]) * K + c0 * 32)[c];
        }
    };
    auto store_a = [&](int off) {
#pragma unroll
        for (int u = 0; u < APT; ++u) *reinterpret_cast<int4*>(lds_a + off + vat[u]) = perm16_a(va[u]);
    };
    load_a(0);
    store_a(0);
    __syncthreads();
    for (int c0 = 0; c0 < Q; c0 += QC) {
        const int qn = min(QC, Q - c0);
        const bool more = c0 + QC < Q;
        if (more) load_a(c0 + QC);
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
        if (more) store_a(boff ^ kChunkBytes);
        __syncthreads();  // the chunk is consumed and the next one staged
        boff ^= kChunkBytes;
    }

    // epilogue: element v of tile t of this lane = row 32*t + 8*(v/4) + 4*h + v%4, column n
    if (EPI == kEpiSwiglu) {
        float* xu = reinterpret_cast<float*>(lds_a);  // [BM][64] up tile
        __syncthreads();                              // A chunk no longer read
        if (up_wave) {
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int m = 8 * (v >> 2) + 4 * h + (v & 3);
                xu[m * 64 + wcol * 32 + (l & 31)] = acc0[v];
                xu[(32 + m) * 64 + wcol * 32 + (l & 31)] = acc1[v];
            }
        }
        __syncthreads();
        if (!up_wave && col_ok) {
#pragma unroll
            for (int t = 0; t < 2; ++t) {
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    const int m = 32 * t + 8 * (v >> 2) + 4 * h + (v & 3);
                    if (m >= nr) continue;
                    const float xs = s_rs[m];
                    const float g = ((t ? acc1[v] : acc0[v]) * kOut) * xs;
                    const float u = (xu[m * 64 + wcol * 32 + (l & 31)] * kOut) * xs;
                    ep.out[static_cast<size_t>(r0 + m) * N + n] = silu_fast(g) * u;
                }
            }
        }
        return;
    }
    if (!col_ok) return;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const int m = 32 * t + 8 * (v >> 2) + 4 * h + (v & 3);
            if (m >= nr) continue;
            const float a = (t ? acc1[v] : acc0[v]) * kOut;
            if (EPI == kEpiPlain) {
                ep.out[static_cast<size_t>(r0 + m) * N + n] = a;
            } else {
                const float yv = a * s_rs[m];
                ep.out[static_cast<size_t>(s_dst[m]) * N + n] = s_gate[m] * yv;
            }
        }
    }
}

// Drop-in GEMM: implicit 64-row tiles over the M rows of one matrix,
// grid (row tile, column block).
template <int EPI, bool G16, bool TILED, bool EXACT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(G16 ? 3 : 4))) void s4_mfma_kernel(
    const int8_t* __restrict__ A, int M, int K, int N, Operand op0, Operand op1, EpiArgs ep) {
    const int r0 = blockIdx.x * BM;
    s4_tile<EPI, G16, TILED, EXACT>(A, K, N, op0, op1, ep, 0, r0, min(BM, M - r0), blockIdx.y);
}

// The layer's grouped GEMM, XCD-aware. Workgroups are dispatched to the 8
// XCDs round-robin (block b to XCD b % 8), and each XCD has its own L2. The
// units (row tile, column block) are ordered expert by expert, column block
// by column block, row tile by row tile, and cut into 8 contiguous equal
// parts, part x for XCD x: block b runs unit (b % 8) * per + b / 8. All row
// tiles of one expert's column block are then consecutive units of one XCD
// (except at the 7 cuts), dispatched together, so the weight slab comes from
// HBM once and the other row tiles read it from that XCD's L2; with the
// tiles dealt round-robin each row tile of a hot expert fetched the slab
// again through another XCD.
constexpr int kXcds = 8;

struct ExpertTiles {
    const int* nt;  // [kMaxE] row tiles of expert e
    const int* t0;  // [kMaxE] its first tile in the tile list
};

// Group 32: four blocks per CU (27 KB of LDS and at most 128 registers
// each); group 16 (two MFMAs per step) needs more registers and takes three.
template <int EPI, bool G16, bool TILED, bool EXACT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(G16 ? 3 : 4))) void s4_grouped_kernel(
    const int8_t* __restrict__ A, TileList tl, ExpertTiles et, int K, int N, Operand op0, Operand op1, EpiArgs ep) {
    constexpr int BNB = block_cols<EPI>();
    const int ncb = (N + BNB - 1) / BNB;
    const int units = *tl.n_tiles * ncb;
    const int per = (units + kXcds - 1) / kXcds;
    const int k = static_cast<int>(blockIdx.x) / kXcds;
    const int g = (static_cast<int>(blockIdx.x) % kXcds) * per + k;
    if (k >= per || g >= units) return;
    // units of expert e are [ncb * t0, ncb * (t0 + nt)), so g / ncb is one of its tiles
    const int e = tl.tile_e[g / ncb];
    const int t0 = et.t0[e], nt = et.nt[e];
    const int loc = g - ncb * t0;
    const int cb = loc / nt;
    const int tile = t0 + (loc - cb * nt);
    s4_tile<EPI, G16, TILED, EXACT>(A, K, N, op0, op1, ep, e, tl.tile_r0[tile], tl.tile_nr[tile], cb);
}

// ---- the int4 layer's MFMA-tiled weight layout -------------------------------
// Destination-ordered copies (8-byte units for the nibbles, floats for the
// scales), one thread per unit.
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
    reinterpret_cast<uint2*>(dst)[d] = *reinterpret_cast<const uint2*>(src + row * (K / 2) + q * 16 + h * 8);
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

// ---- quantize x + plan (one launch) -------------------------------------------
// Blocks [0, qblocks): quantize the token rows by `rule` (quantize_row_i8_te,
// decoder.rs:1647-1656, for the int4 layer; the dynamic rule of
// linear_int8_dynamic for the int8 one),
// four rows per block (one per 256 threads). The last block: the plan, a
// stable counting sort of the (token, slot) pairs by expert. Pairs whose
// expert is out of range set *err (the oracle's shape error). Output:
// perm[row] = pair id, experts' rows contiguous in increasing expert order,
// pair order kept inside an expert (= token order, then slot); tiles of up
// to 64 rows of one expert (expert, first row, row count) and their number;
// each expert's tile count and first tile.
constexpr int kPlanThreads = 1024;
constexpr int kPlanWaves = kPlanThreads / 64;
constexpr int kQRows = kPlanThreads / 256;  // token rows per quantize block
constexpr int kPlanPre = 4;  // rounds of pairs whose expert ids the plan block loads up front
// Up to this many rounds (8192 pairs) the counting pass keeps every (round,
// wave, expert) count, so the scatter needs no barrier between rounds.
constexpr int kPlanFastRounds = 8;

__device__ __forceinline__ int wave_excl_scan(int v, int lane) {
    int x = v;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int y = __shfl_up(x, o, 64);
        if (lane >= o) x += y;
    }
    return x - v;
}

// Lanes of the wave holding the same 7-bit id as this lane (ids >= 127 are
// "none" and match each other).
__device__ __forceinline__ unsigned long long match7(uint32_t e) {
    unsigned long long same = ~0ull;
#pragma unroll
    for (int b = 0; b < 7; ++b) {
        const unsigned long long bm = __ballot((e >> b) & 1u);
        same &= ((e >> b) & 1u) ? bm : ~bm;
    }
    return same;
}

__global__ __launch_bounds__(kPlanThreads) void i4_prep_kernel(const float* __restrict__ x, int T, int H, int rule,
                                                               int8_t* __restrict__ xq, float* __restrict__ xs,
                                                               const uint32_t* __restrict__ idx, int TK, int E,
                                                               int* __restrict__ perm, int* __restrict__ n_tiles,
                                                               int* __restrict__ tile_e, int* __restrict__ tile_r0,
                                                               int* __restrict__ tile_nr, int* __restrict__ exp_nt,
                                                               int* __restrict__ exp_t0, int* __restrict__ err) {
    __shared__ int s_cnt[kMaxE];
    __shared__ int s_base[kMaxE];
    __shared__ int s_wc[kPlanWaves][kMaxE];
    __shared__ unsigned short s_pre[kPlanFastRounds][kPlanWaves][kMaxE];  // counts, then their prefix
    __shared__ int s_err;
    __shared__ float s_red[kPlanWaves];
    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int lane = tid & 63;
    const int qblocks = (T + kQRows - 1) / kQRows;
    if (static_cast<int>(blockIdx.x) < qblocks) {
        const int sub = tid >> 8, st = tid & 255;  // row slot in the block, thread in the row
        const int row = blockIdx.x * kQRows + sub;
        const bool ok = row < T;
        const float* xr = x + static_cast<size_t>(ok ? row : 0) * H;
        // the row in registers (float4 loads all issued before the first use)
        // where it fits; the strided loop waits for each load in turn
        const int H4 = H >> 2;
        const bool vec = (H & 3) == 0 && H4 <= 2 * 256 && reinterpret_cast<uintptr_t>(x) % 16 == 0 &&
                         reinterpret_cast<uintptr_t>(xq) % 4 == 0;  // uniform
        float4 v[2] = {};
        float amax = 0.0f;
        if (vec) {
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int c = st + 256 * j;
                v[j] = reinterpret_cast<const float4*>(xr)[c < H4 ? c : H4 - 1];
                if (c < H4) amax = fmaxf(amax, fmaxf(fmaxf(fabsf(v[j].x), fabsf(v[j].y)), fmaxf(fabsf(v[j].z), fabsf(v[j].w))));
            }
        } else {
            for (int i = st; i < H; i += 256) amax = fmaxf(amax, fabsf(xr[i]));
        }
        amax = wave_max_f_full(amax);
        if (lane == 0) s_red[wave] = amax;
        __syncthreads();
        const int w0 = sub * 4;
        amax = fmaxf(fmaxf(s_red[w0], s_red[w0 + 1]), fmaxf(s_red[w0 + 2], s_red[w0 + 3]));
        const float a_scale = amax > 0.0f ? amax / 127.0f : 1.0f;
        const float inv = 1.0f / a_scale;
        if (ok) {
            int8_t* q = xq + static_cast<size_t>(row) * H;
            if (vec) {
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const int c = st + 256 * j;
                    if (c < H4) {
                        char4 o;
                        o.x = quant_rule(v[j].x, a_scale, inv, rule);
                        o.y = quant_rule(v[j].y, a_scale, inv, rule);
                        o.z = quant_rule(v[j].z, a_scale, inv, rule);
                        o.w = quant_rule(v[j].w, a_scale, inv, rule);
                        reinterpret_cast<char4*>(q)[c] = o;
                    }
                }
            } else {
                for (int i = st; i < H; i += 256) q[i] = quant_rule(xr[i], a_scale, inv, rule);
            }
            if (st == 0) xs[row] = a_scale;
        }
        return;
    }
    // the plan block: the expert ids of the first kPlanPre rounds of pairs are
    // requested once, up front (the counting and the scatter pass each read
    // every round; loaded per round, each round waited on its own load)
    uint32_t epre[kPlanPre];
#pragma unroll
    for (int r = 0; r < kPlanPre; ++r) {
        const int p = r * kPlanThreads + tid;
        epre[r] = p < TK ? idx[p] : 127u;
    }
    auto expert_of = [&](int c0) {  // c0: the round's first pair (uniform)
        const int r = c0 / kPlanThreads, p = c0 + tid;
        uint32_t e = 127u;
#pragma unroll
        for (int q = 0; q < kPlanPre; ++q)
            if (r == q) e = epre[q];
        if (r >= kPlanPre) e = p < TK ? idx[p] : 127u;
        return e;
    };
    const int rounds = (TK + kPlanThreads - 1) / kPlanThreads;
    const bool fast = rounds <= kPlanFastRounds;  // uniform
    if (tid < kMaxE) s_cnt[tid] = 0;
    for (int i = tid; i < kPlanWaves * kMaxE; i += kPlanThreads) (&s_wc[0][0])[i] = 0;
    if (fast)
        for (int i = tid; i < rounds * kPlanWaves * kMaxE; i += kPlanThreads) (&s_pre[0][0][0])[i] = 0;
    if (tid == 0) s_err = 0;
    __syncthreads();
    // counts: one LDS add per distinct expert per wave and round (and, in the
    // fast form, the wave's count of the round kept)
    for (int c0 = 0; c0 < TK; c0 += kPlanThreads) {
        const int p = c0 + tid;
        uint32_t e = expert_of(c0);
        if (p < TK && e >= static_cast<uint32_t>(E)) s_err = 1;
        if (e >= static_cast<uint32_t>(E)) e = 127u;
        const unsigned long long same = match7(e);
        if (e < 127u && (same & ((1ull << lane) - 1ull)) == 0ull) {
            atomicAdd(&s_cnt[e], __popcll(same));
            if (fast) s_pre[c0 / kPlanThreads][wave][e] = static_cast<unsigned short>(__popcll(same));
        }
    }
    __syncthreads();
    // wave 0 (lane = expert): row bases and the tile list (each expert's
    // tiles contiguous, in expert order)
    if (wave == 0) {
        const int c = lane < E ? s_cnt[lane] : 0;
        const int nt = (c + BM - 1) / BM;
        const int base = wave_excl_scan(c, lane);
        const int t0 = wave_excl_scan(nt, lane);
        s_base[lane] = base;
        for (int i = 0; i < nt; ++i) {
            tile_e[t0 + i] = lane;
            tile_r0[t0 + i] = base + BM * i;
            tile_nr[t0 + i] = min(BM, c - BM * i);
        }
        exp_nt[lane] = nt;
        exp_t0[lane] = t0;
        if (lane == 63) *n_tiles = t0 + nt;
        if (lane == 0) *err = s_err;
    }
    __syncthreads();
    if (fast) {
        // each expert's counts in (round, wave) order turned into exclusive
        // prefixes: pair p of round r, wave w lands at base + prefix + its
        // rank among the wave's pairs of its expert — the stable order, with
        // no barrier between rounds
        if (tid < kMaxE) {
            int run = 0;
            for (int r = 0; r < rounds; ++r)
                for (int w = 0; w < kPlanWaves; ++w) {
                    const int c = s_pre[r][w][tid];
                    s_pre[r][w][tid] = static_cast<unsigned short>(run);
                    run += c;
                }
        }
        __syncthreads();
        for (int c0 = 0; c0 < TK; c0 += kPlanThreads) {
            const int p = c0 + tid;
            uint32_t e = expert_of(c0);
            if (e >= static_cast<uint32_t>(E)) e = 127u;  // invalid: never placed
            const unsigned long long same = match7(e);
            const int rank = __popcll(same & ((1ull << lane) - 1ull));
            if (e < 127u) perm[s_base[e] + s_pre[c0 / kPlanThreads][wave][e] + rank] = p;
        }
        return;
    }
    // stable scatter, 1024 pairs per round: rank inside the wave by matching
    // expert ids with ballots, wave offsets from per-wave counts
    for (int c0 = 0; c0 < TK; c0 += kPlanThreads) {
        const int p = c0 + tid;
        uint32_t e = expert_of(c0);
        if (e >= static_cast<uint32_t>(E)) e = 127u;  // invalid: never placed
        const unsigned long long same = match7(e);
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
// ahead of it, the first K threads publish order[rank] = j. shared_y (the
// shared expert's output, nullable) is added last (decoder.rs:2176-2179);
// resid (nullable) is the decoder layer's residual, add_residual(h, mlp)
// (decoder.rs:2494, :2531), so the layer's separate add launch goes.
__global__ __launch_bounds__(256) void i4_combine_kernel(const float* __restrict__ ybuf,
                                                         const uint32_t* __restrict__ idx, int H, int K,
                                                         const float* __restrict__ shared_y,
                                                         float* __restrict__ out, const float* __restrict__ resid) {
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
    if (shared_y) o = o + shared_y[static_cast<size_t>(t) * H + c];
    if (resid) o = resid[static_cast<size_t>(t) * H + c] + o;
    out[static_cast<size_t>(t) * H + c] = o;
}

// two staged K chunks (26 KB; the SwiGLU up-tile exchange after the K loop needs 16 KB)
constexpr size_t kGemmLds = 2 * kChunkBytes > BM * 64 * 4 ? 2 * kChunkBytes : BM * 64 * 4;

template <int EPI, bool G16, bool TILED, bool EXACT>
hipError_t launch_gemm(hipStream_t s, const int8_t* A, int M, int K, int N, const Operand& op0, const Operand& op1,
                       const EpiArgs& ep) {
    constexpr int BNB = block_cols<EPI>();
    const dim3 grid((M + BM - 1) / BM, (N + BNB - 1) / BNB);
    FOCR_LAUNCH((s4_mfma_kernel<EPI, G16, TILED, EXACT>), grid, dim3(256), kGemmLds, s, A, M, K, N, op0, op1, ep);
    return hipGetLastError();
}

// One block per unit, max_units = the most units the plan can produce.
template <int EPI, bool G16>
hipError_t launch_grouped(hipStream_t s, const int8_t* A, const TileList& tl, const ExpertTiles& et, int K, int N,
                          const Operand& op0, const Operand& op1, const EpiArgs& ep, int max_tiles) {
    constexpr int BNB = block_cols<EPI>();
    const int max_units = max_tiles * ((N + BNB - 1) / BNB);
    const dim3 grid(static_cast<unsigned>(kXcds * ((max_units + kXcds - 1) / kXcds)));
    FOCR_LAUNCH((s4_grouped_kernel<EPI, G16, true, false>), grid, dim3(256), kGemmLds, s, A, tl, et, K, N, op0, op1,
                ep);
    return hipGetLastError();
}

template <int EPI>
hipError_t launch_grouped_g(hipStream_t s, int group, const int8_t* A, const TileList& tl, const ExpertTiles& et,
                            int K, int N, const Operand& op0, const Operand& op1, const EpiArgs& ep, int max_tiles) {
    if (group == 32) return launch_grouped<EPI, false>(s, A, tl, et, K, N, op0, op1, ep, max_tiles);
    return launch_grouped<EPI, true>(s, A, tl, et, K, N, op0, op1, ep, max_tiles);
}

}  // namespace

bool s4_mfma_supported(int group, int k) {
    return (group == 16 || group == 32) && k % 32 == 0 && k > 0 && k <= 16384;
}

size_t s4_tile_pad_bytes() { return kTilePadBytes; }

hipError_t launch_s4s8_mfma(hipStream_t s, const int8_t* a, const uint8_t* b, const float* scales, int group, int m,
                            int k, int n, float* out) {
    if (!s4_mfma_supported(group, k) || m <= 0 || n <= 0) return hipErrorInvalidValue;
    const Operand op0{b, scales};
    const EpiArgs ep{out, nullptr, nullptr, nullptr, 0};
    if (group == 32) return launch_gemm<kEpiPlain, false, false, true>(s, a, m, k, n, op0, Operand{nullptr, nullptr}, ep);
    return launch_gemm<kEpiPlain, true, false, true>(s, a, m, k, n, op0, Operand{nullptr, nullptr}, ep);
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
    return static_cast<size_t>(tk) + 3 * static_cast<size_t>(max_tiles) + 2 * kMaxE + 2;
}

MoePlan moe_plan_view(int* plan, int tk, int n_experts) {
    MoePlan p;
    p.max_tiles = (tk + BM - 1) / BM + n_experts;
    p.perm = plan;
    p.tile_e = p.perm + tk;
    p.tile_r0 = p.tile_e + p.max_tiles;
    p.tile_nr = p.tile_r0 + p.max_tiles;
    p.exp_nt = p.tile_nr + p.max_tiles;
    p.exp_t0 = p.exp_nt + kMaxE;
    p.n_tiles = p.exp_t0 + kMaxE;
    return p;
}

hipError_t launch_moe_prefill_plan(hipStream_t s, const float* x, int t, int H, int rule, int8_t* xq, float* xs,
                                   const uint32_t* idx, int top_k, int E, const MoePlan& p, int* err) {
    const int qblocks = (t + kQRows - 1) / kQRows;
    FOCR_LAUNCH(i4_prep_kernel, dim3(qblocks + 1), dim3(kPlanThreads), 0, s, x, t, H, rule, xq, xs, idx, t * top_k,
                E, p.perm, p.n_tiles, p.tile_e, p.tile_r0, p.tile_nr, p.exp_nt, p.exp_t0, err);
    return hipGetLastError();
}

hipError_t launch_moe_prefill_combine(hipStream_t s, const float* ybuf, const uint32_t* idx, int t, int H,
                                      int top_k, const float* shared_y, float* out, const float* resid) {
    FOCR_LAUNCH(i4_combine_kernel, dim3((H + 255) / 256, t), dim3(256), 0, s, ybuf, idx, H, top_k, shared_y, out,
                resid);
    return hipGetLastError();
}

hipError_t launch_moe_prefill_i4(hipStream_t s, const focr_hip_moe_layer_i4* L, const float* x, int t, int top_k,
                                 const uint32_t* idx, const float* gates, float* out, MoeI4Scratch& w,
                                 focr_hip_ctx* ctx) {
    const int H = static_cast<int>(L->hidden), I = static_cast<int>(L->inter), E = static_cast<int>(L->n_experts);
    const int group = static_cast<int>(L->group);
    const int TK = t * top_k;
    const MoePlan p = moe_plan_view(w.plan, TK, E);
    const int max_tiles = p.max_tiles;
    const int* perm = p.perm;
    hipError_t e;
    {
        ProfScope ps(ctx, "i4_prep");
        if ((e = launch_moe_prefill_plan(s, x, t, H, kQuantTiesEven, w.xq, w.xs, idx, top_k, E, p, w.err)) !=
            hipSuccess)
            return e;
    }
    const TileList tl{p.n_tiles, p.tile_e, p.tile_r0, p.tile_nr};
    const ExpertTiles et{p.exp_nt, p.exp_t0};
    {
        ProfScope ps(ctx, "i4_gate_up");
        const EpiArgs ep{w.act, perm, w.xs, nullptr, top_k};
        if ((e = launch_grouped_g<kEpiSwiglu>(s, group, w.xq, tl, et, H, I, Operand{L->wg, L->sg},
                                              Operand{L->wu, L->su}, ep, max_tiles)) != hipSuccess)
            return e;
    }
    {
        ProfScope ps(ctx, "i4_quantize_act");
        if ((e = launch_quantize_rows(s, w.act, TK, I, w.aq, w.as, kQuantTiesEven)) != hipSuccess) return e;
    }
    {
        ProfScope ps(ctx, "i4_down");
        const EpiArgs ep{w.ybuf, perm, w.as, gates, top_k};
        if ((e = launch_grouped_g<kEpiDown>(s, group, w.aq, tl, et, I, H, Operand{L->wd, L->sd},
                                            Operand{nullptr, nullptr}, ep, max_tiles)) != hipSuccess)
            return e;
    }
    {
        ProfScope ps(ctx, "i4_combine");
        if ((e = launch_moe_prefill_combine(s, w.ybuf, idx, t, H, top_k, nullptr, out)) != hipSuccess) return e;
    }
    return hipSuccess;
}

}  // namespace focr
