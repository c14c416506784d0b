// k_i8mfma.hip — int8 x int8 GEMMs on gfx950 matrix cores for prefill.
//
//   * nn::linear_int8_dynamic (nn.rs:151-173): rows quantized by the dynamic
//     activation rule (docs/focrq-format.md:296-320: x / scale, ties to even),
//     C = A · Bᵀ in i32 on v_mfma_i32_32x32x32_i8, y = ((f32)acc * a_s) * w_s
//     (+ bias), the decoder's dequant order (decoder.rs:1636).
//   * moe_block_i8 (decoder.rs:2142-2181) over an uploaded int8 MoE layer:
//     the prefill plan shared with the int4 layer (stable counting sort of the
//     (token, slot) pairs by expert into 64-row tiles), a grouped gate/up GEMM
//     with the SwiGLU epilogue (expert_mlp_i8, decoder.rs:2120-2135),
//     re-quantization of the act rows by the dynamic rule, a grouped down GEMM
//     whose epilogue multiplies by the pair's gate, the combine in ascending
//     expert order, and the shared expert (all rows, dense) added last; its
//     gate/up and down products run as extra units of the two grouped
//     launches.
//
// Integer sums are exact, so every i32 accumulator equals the CPU's; the f32
// outputs follow the reference's formulas (SiLU through expf).
//
// Block = 4 waves over a 64-row tile. Wave w computes 64 rows x 64 columns
// (2 x 2 MFMA tiles of 32 x 32); for SwiGLU 64 rows x 32 columns of the gate
// and the same 32 of the up matrix, so each (row, column)'s gate and up sums
// sit in the same lane and register: the epilogue needs no exchange.
// Operand layout of v_mfma_i32_32x32x32_i8: lane l holds A row l % 32 and B
// column l % 32, bytes 16 (l / 32) + [0, 16) of the 32-wide K step; C element
// v of lane l is row 8 (v / 4) + 4 (l / 32) + v % 4, column l % 32.
//
// Activations: 256-byte K chunks of the tile's 64 rows (16 KB) are staged in
// LDS through registers (two buffers; the next chunk's loads are in flight
// while the current one's 4 stages run, and land in the other buffer at the
// end), the 16-byte piece p of row r at slot p ^ (r & 15): the 16 rows a
// quarter-wave's fragment read touches then start on 16 different banks.
// With 32 KB of LDS and at most 168 registers a block, three blocks share a
// CU: measured against 512-byte chunks with four fragment stages in flight
// (two blocks a CU), the prefill layer's grouped gate/up at 256 / 1024 rows
// went 33.2 -> 31.5 / 54.4 -> 51.4 us and the down 41.8 -> 35.3 us at 1024
// rows; the depth of the fragment ring alone (two or four stages) moved
// nothing, so the two-stage ring pays for the third block's registers.
// (Direct global -> LDS loads would save the registers, but the compiler
// cannot tell the buffer they fill from the one being read and drains every
// load before each LDS read.)
// Weights go global -> VGPR, each lane loading exactly the 16-byte fragments
// its MFMAs take, two 64-byte K stages ahead, from a fragment-ordered copy
// (launch_retile_i8) made once per handle: a wave's fragment load is then
// 1 KB contiguous. Read in the upload layout ([E][N][K], output-channel-major,
// what decode uses), each load touched 32 rows — 32 cache lines — and the
// L1 address path, not the MFMA, bound the kernel (TA busy 74%, MFMA 12%).
#include <type_traits>

#include "focr_internal.hpp"
#include "k_common.hpp"

namespace focr {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

constexpr int BM = kMoePlanTileRows;  // 64 rows per block tile
constexpr int KB = 64;                // K bytes per stage (two MFMA K steps)
constexpr int KC = 256;               // K bytes per staged activation chunk
constexpr int PPR = KC / 16;          // 16-byte pieces per staged row (a multiple of 16: the swizzle)
constexpr int SPC = KC / KB;          // stages per chunk
constexpr int kXcds = 8;
constexpr int kRing = 2;              // K stages of weight fragments in flight
static_assert(PPR % 16 == 0, "the LDS swizzle permutes pieces within groups of 16");

enum I8Epi { kI8Linear = 0, kI8Swiglu = 1, kI8Down = 2 };

template <int EPI>
constexpr int bcols() {
    return EPI == kI8Swiglu ? 128 : 256;
}

struct I8Args {
    const int8_t* A;        // activation rows [rows][K]
    const float* a_scale;   // scale per A row
    const int* perm;        // MoE: sorted row -> pair id (t * top_k + j); null: direct rows
    int top_k;
    const int8_t* B0;       // weights [E][N][K] in the fragment order of launch_retile_i8
    const float* s0;        // [E][N]
    const int8_t* B1;       // SwiGLU: up weights (fragment order)
    const float* s1;
    const float* bias;      // linear: [N] or null
    const float* gates;     // down: [pairs]
    float* out;             // linear [rows][N]; SwiGLU act [rows][N]; down ybuf [pairs][N]
    int K, N;
};

// One block tile: rows [r0, r0 + nr) (nr <= 64) of expert e against column
// block cb. Every thread of the block calls it (it synchronises).
template <int EPI>
__device__ __forceinline__ void i8_tile(const I8Args& a, int e, int r0, int nr, int cb) {
    // two chunk buffers
    __shared__ __align__(16) int8_t lds_a0[BM * KC];
    __shared__ __align__(16) int8_t lds_a1[BM * KC];
    __shared__ int s_arow[BM];
    __shared__ int s_dst[BM];
    __shared__ float s_rs[BM];
    __shared__ float s_gate[BM];
    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int l = tid & 63;
    const int h = l >> 5;
    const int c32 = l & 31;
    const int K = a.K, N = a.N;
    const int S = K / KB;

    if (tid < BM) {
        const int row = r0 + (tid < nr ? tid : nr - 1);  // rows past nr repeat the last one, never stored
        int arow = row, dst = row;
        float g = 1.0f;
        if (a.perm) {
            const int pid = a.perm[row];
            dst = pid;
            if (EPI == kI8Swiglu) arow = pid / a.top_k;  // the pair's token row
            if (EPI == kI8Down) g = a.gates[pid];
        }
        s_arow[tid] = arow;
        s_dst[tid] = dst;
        s_rs[tid] = a.a_scale[arow];
        s_gate[tid] = g;
    }

    // this lane's two weight columns (tile j = 0, 1) and their fragment
    // streams: 1 KB per (column tile, 32-byte K step), lane l at 16 l
    const int NT = (N + 31) >> 5, KS = K >> 5;
    int col[2];
    const int8_t* bp[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int tile = EPI == kI8Swiglu ? cb * 4 + wave : cb * 8 + 2 * wave + j;
        col[j] = 32 * tile + c32;
        const int8_t* B = (EPI == kI8Swiglu && j == 1) ? a.B1 : a.B0;
        bp[j] = B + (static_cast<size_t>(e * NT + (tile < NT ? tile : NT - 1)) * KS * 64 + l) * 16;
    }
    // fragments f[2 j + s]: column tile j, K step s of stage st (clamped past the end)
    auto load_b = [&](int st, v4i (&f)[4]) {
        const int ss = st < S ? st : S - 1;
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int s = 0; s < 2; ++s)
                f[2 * j + s] = *reinterpret_cast<const v4i*>(bp[j] + static_cast<size_t>(2 * ss + s) * 1024);
    };
    // a ring of kRing stages of fragments, stage st in f[st % kRing], loaded
    // kRing stages ahead (SPC a multiple of kRing keeps the ring index a constant)
    v4i f[kRing][4];
#pragma unroll
    for (int q = 0; q < kRing; ++q) load_b(q, f[q]);
    __syncthreads();  // the row tables

    // Chunk c of the activations: 64 rows x PPR pieces of 16 bytes; thread tid
    // loads pieces tid + 256 i (row q / PPR, piece q % PPR: PPR threads read a
    // row's KC contiguous bytes) into registers, and stores piece p of row r
    // at LDS slot p ^ (r & 15). Pieces past K are clamped into the row (never
    // read).
    const int nchunks = (K + KC - 1) / KC;
    constexpr int APT = BM * KC / 16 / 256;  // pieces per thread per chunk
    auto load_chunk = [&](int c, v4i (&v)[APT]) {
#pragma unroll
        for (int i = 0; i < APT; ++i) {
            const int q = tid + 256 * i;
            const int r = q / PPR, p = q % PPR;
            int kb = c * KC + 16 * p;
            kb = kb < K ? kb : 0;
            v[i] = *reinterpret_cast<const v4i*>(a.A + static_cast<size_t>(s_arow[r]) * K + kb);
        }
    };
    auto store_chunk = [&](int8_t* base, const v4i (&v)[APT]) {
#pragma unroll
        for (int i = 0; i < APT; ++i) {
            const int q = tid + 256 * i;
            const int r = q / PPR, p = q % PPR;
            *reinterpret_cast<v4i*>(base + r * KC + 16 * (p ^ (r & 15))) = v[i];
        }
    };

    v16i acc00 = {}, acc01 = {}, acc10 = {}, acc11 = {};
    // live = false (a stage past K): the weight fragments are zeroed by a
    // select, so the MFMAs add nothing and the code stays branch-free (a
    // branch around them costs the compiler its exact load-count waits).
    auto compute = [&](const int8_t* buf, int ls, const v4i (&f)[4], bool live) {
        const v4i z = {0, 0, 0, 0};
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            const int c16 = 4 * ls + 2 * s + h;  // 16-byte piece of the staged row
            const v4i a0 = *reinterpret_cast<const v4i*>(buf + c32 * KC + 16 * (c16 ^ (c32 & 15)));
            const v4i a1 = *reinterpret_cast<const v4i*>(buf + (32 + c32) * KC + 16 * (c16 ^ ((32 + c32) & 15)));
            const v4i b0 = live ? f[s] : z;
            const v4i b1 = live ? f[2 + s] : z;
            acc00 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a0, b0, acc00, 0, 0, 0);
            acc01 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a0, b1, acc01, 0, 0, 0);
            acc10 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a1, b0, acc10, 0, 0, 0);
            acc11 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a1, b1, acc11, 0, 0, 0);
        }
    };

    static_assert(SPC % kRing == 0, "the fragment ring must divide a chunk's stages");
    // Chunk c: its SPC stages from LDS, the next chunk's loads in flight
    // meanwhile, stored to the other buffer at the end (the last chunk
    // reloads itself: every iteration is the same straight-line code, which
    // keeps the compiler's load-count waits exact). Stages past K (the last
    // chunk's tail) multiply zeros; their fragment loads still run (clamped
    // to the last stage).
    v4i av[APT];
    load_chunk(0, av);
    store_chunk(lds_a0, av);
    __syncthreads();
    for (int c = 0; c < nchunks; ++c) {
        const int8_t* buf = (c & 1) ? lds_a1 : lds_a0;
        int8_t* next = (c & 1) ? lds_a0 : lds_a1;
        load_chunk(c + 1 < nchunks ? c + 1 : c, av);
#pragma unroll
        for (int ls = 0; ls < SPC; ++ls) {
            const int st = c * SPC + ls;
            compute(buf, ls, f[ls % kRing], st < S);
            __builtin_amdgcn_sched_barrier(0);  // keep each stage's refill after its MFMAs
            load_b(st + kRing, f[ls % kRing]);
            __builtin_amdgcn_sched_barrier(0);
        }
        store_chunk(next, av);
        __syncthreads();  // chunk c + 1 is in LDS; chunk c's buffer is free
    }

    // epilogue
    const bool ok0 = col[0] < N, ok1 = col[1] < N;
    const float ws0 = a.s0[static_cast<size_t>(e) * N + (ok0 ? col[0] : 0)];
    const float ws1 = EPI == kI8Swiglu ? a.s1[static_cast<size_t>(e) * N + (ok0 ? col[0] : 0)]
                                       : a.s0[static_cast<size_t>(e) * N + (ok1 ? col[1] : 0)];
    const float b0 = (EPI == kI8Linear && a.bias) ? a.bias[ok0 ? col[0] : 0] : 0.0f;
    const float b1 = (EPI == kI8Linear && a.bias) ? a.bias[ok1 ? col[1] : 0] : 0.0f;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const int m = 32 * t + 8 * (v >> 2) + 4 * h + (v & 3);
            if (m >= nr) continue;
            const float rs = s_rs[m];
            const int i0 = t ? acc10[v] : acc00[v];
            const int i1 = t ? acc11[v] : acc01[v];
            if (EPI == kI8Swiglu) {
                if (!ok0) continue;
                const float g = (static_cast<float>(i0) * rs) * ws0;
                const float u = (static_cast<float>(i1) * rs) * ws1;
                a.out[static_cast<size_t>(r0 + m) * N + col[0]] = silu_f(g) * u;
            } else {
                const size_t orow = static_cast<size_t>(EPI == kI8Down ? s_dst[m] : r0 + m) * N;
                if (ok0) {
                    float y = (static_cast<float>(i0) * rs) * ws0;
                    if (EPI == kI8Linear && a.bias) y = y + b0;
                    if (EPI == kI8Down) y = s_gate[m] * y;
                    a.out[orow + col[0]] = y;
                }
                if (ok1) {
                    float y = (static_cast<float>(i1) * rs) * ws1;
                    if (EPI == kI8Linear && a.bias) y = y + b1;
                    if (EPI == kI8Down) y = s_gate[m] * y;
                    a.out[orow + col[1]] = y;
                }
            }
        }
    }
}

// Dense: grid (row tile, column block) over the M rows of one matrix.
template <int EPI>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3))) void i8_gemm_kernel(I8Args a, int M) {
    const int r0 = blockIdx.x * BM;
    i8_tile<EPI>(a, 0, r0, min(BM, M - r0), blockIdx.y);
}

// Grouped over the plan's tiles, XCD-aware like the int4 layer's: the units
// (tile, column block) are ordered expert by expert, column block by column
// block, tile by tile, and cut into 8 contiguous parts, part x for XCD x
// (block b runs unit (b % 8) * per + b / 8), so an expert's row tiles that
// share a weight slab run together on one XCD and its L2 serves the repeats.
// The first sh_blocks blocks (a multiple of 8; 0 for none) run a second,
// dense product in the same launch: `sh` over all sh_rows rows (the shared
// expert's gate/up, which reads the same quantized rows), its units (row
// tile, column block) ordered column block by column block and cut into 8
// contiguous parts the same way. Its blocks take the slots the routed units
// leave free, so its own launch and the idle CUs of its small grid go.
template <int EPI>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3))) void i8_grouped_kernel(
    I8Args a, const int* __restrict__ n_tiles, const int* __restrict__ tile_e, const int* __restrict__ tile_r0,
    const int* __restrict__ tile_nr, const int* __restrict__ exp_nt, const int* __restrict__ exp_t0, I8Args sh,
    int sh_rows, int sh_blocks) {
    constexpr int BNB = bcols<EPI>();
    int b = static_cast<int>(blockIdx.x);
    if (b < sh_blocks) {
        const int ncb_s = (sh.N + BNB - 1) / BNB;
        const int nt_s = (sh_rows + BM - 1) / BM;
        const int units_s = nt_s * ncb_s;
        const int per_s = sh_blocks / kXcds;
        const int ks = b / kXcds;
        const int gs = (b % kXcds) * per_s + ks;
        if (gs >= units_s) return;
        const int cb = gs / nt_s, r0 = (gs - cb * nt_s) * BM;
        i8_tile<EPI>(sh, 0, r0, min(BM, sh_rows - r0), cb);
        return;
    }
    b -= sh_blocks;
    const int ncb = (a.N + BNB - 1) / BNB;
    const int units = *n_tiles * ncb;
    const int per = (units + kXcds - 1) / kXcds;
    const int k = b / kXcds;
    const int g = (b % kXcds) * per + k;
    if (k >= per || g >= units) return;
    const int e = tile_e[g / ncb];
    const int t0 = exp_t0[e], nt = exp_nt[e];
    const int loc = g - ncb * t0;
    const int cb = loc / nt;
    const int tile = t0 + (loc - cb * nt);
    i8_tile<EPI>(a, e, tile_r0[tile], tile_nr[tile], cb);
}

// One thread per 16-byte destination unit d = ((e * NT + nt) * KS + ks) * 64
// + 32 h + c: column n = 32 nt + c of matrix e, bytes 32 ks + 16 h; zero for
// the padding columns n >= N.
__global__ __launch_bounds__(256) void retile_i8_kernel(const int8_t* __restrict__ src, int8_t* __restrict__ dst,
                                                        size_t units, int N, int K) {
    const size_t d = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x;
    if (d >= units) return;
    const int NT = (N + 31) >> 5, KS = K >> 5;
    const int c = static_cast<int>(d & 31);
    const int h = static_cast<int>((d >> 5) & 1);
    size_t r = d >> 6;
    const int ks = static_cast<int>(r % KS);
    r /= KS;
    const int nt = static_cast<int>(r % NT);
    const size_t e = r / NT;
    const int n = 32 * nt + c;
    v4i v = {0, 0, 0, 0};
    if (n < N) v = *reinterpret_cast<const v4i*>(src + (e * N + n) * K + 32 * ks + 16 * h);
    reinterpret_cast<v4i*>(dst)[d] = v;
}

}  // namespace

bool i8_mfma_supported(int k) { return k > 0 && k % KB == 0 && k <= 65536; }

size_t i8_tiled_bytes(int n_mats, int n, int k) {
    return static_cast<size_t>(n_mats) * static_cast<size_t>((n + 31) & ~31) * static_cast<size_t>(k);
}

hipError_t launch_retile_i8(hipStream_t s, const int8_t* src, int n_mats, int n, int k, int8_t* dst) {
    if (k % 32 || n <= 0 || n_mats <= 0) return hipErrorInvalidValue;
    const size_t units = i8_tiled_bytes(n_mats, n, k) / 16;
    FOCR_LAUNCH(retile_i8_kernel, dim3(static_cast<unsigned>((units + 255) / 256)), dim3(256), 0, s, src, dst, units,
                n, k);
    return hipGetLastError();
}

hipError_t launch_linear_i8(hipStream_t s, const int8_t* xq, const float* xs, int m, int k, const int8_t* w,
                            const float* ws, int n, const float* bias, float* y) {
    if (!i8_mfma_supported(k) || m <= 0 || n <= 0) return hipErrorInvalidValue;
    I8Args a{xq, xs, nullptr, 1, w, ws, nullptr, nullptr, bias, nullptr, y, k, n};
    const dim3 grid((m + BM - 1) / BM, (n + bcols<kI8Linear>() - 1) / bcols<kI8Linear>());
    FOCR_LAUNCH(i8_gemm_kernel<kI8Linear>, grid, dim3(256), 0, s, a, m);
    return hipGetLastError();
}

hipError_t launch_moe_prefill_i8(hipStream_t s, const focr_hip_moe_layer* L, const float* x, int t, int top_k,
                                 const uint32_t* idx, const float* gates, int with_shared, float* out,
                                 MoeI8Scratch& w, focr_hip_ctx* ctx, const float* resid) {
    const int H = static_cast<int>(L->hidden), I = static_cast<int>(L->inter), E = static_cast<int>(L->n_experts);
    const int TK = t * top_k;
    const MoePlan p = moe_plan_view(w.plan, TK, E);
    hipError_t e;
    {
        ProfScope ps(ctx, "i8_prep");
        if ((e = launch_moe_prefill_plan(s, x, t, H, kQuantDynamic, w.xq, w.xs, idx, top_k, E, p, w.err)) !=
            hipSuccess)
            return e;
    }
    // sh_rows > 0: the dense product `sh` over that many rows rides in the
    // same launch (its blocks first, a multiple of 8 of them)
    auto grouped = [&](auto epi, const I8Args& a, const I8Args& sh, int sh_rows) {
        constexpr int EPI = decltype(epi)::value;
        const int ncb = (a.N + bcols<EPI>() - 1) / bcols<EPI>();
        const int max_units = p.max_tiles * ncb;
        int sh_blocks = 0;
        if (sh_rows > 0) {
            const int units_s = ((sh_rows + BM - 1) / BM) * ((sh.N + bcols<EPI>() - 1) / bcols<EPI>());
            sh_blocks = kXcds * ((units_s + kXcds - 1) / kXcds);
        }
        const dim3 grid(static_cast<unsigned>(sh_blocks + kXcds * ((max_units + kXcds - 1) / kXcds)));
        FOCR_LAUNCH(i8_grouped_kernel<EPI>, grid, dim3(256), 0, s, a, p.n_tiles, p.tile_e, p.tile_r0, p.tile_nr,
                    p.exp_nt, p.exp_t0, sh, sh_rows, sh_blocks);
        return hipGetLastError();
    };
    const int SI = with_shared ? static_cast<int>(L->shared_inter) : 0;
    {
        ProfScope ps(ctx, "i8_gate_up");
        const I8Args a{w.xq, w.xs, p.perm, top_k, L->wg_mfma, L->sg, L->wu_mfma, L->su, nullptr, nullptr, w.act, H, I};
        // the shared expert's gate/up (every token row, SwiGLU) as extra units
        const I8Args sh{w.xq, w.xs, nullptr, 1, L->swg_mfma, L->ssg, L->swu_mfma, L->ssu, nullptr, nullptr,
                        w.shared_act, H, SI};
        if ((e = grouped(std::integral_constant<int, kI8Swiglu>(), a, sh, with_shared ? t : 0)) != hipSuccess)
            return e;
    }
    {
        ProfScope ps(ctx, "i8_quantize_act");
        // the routed act rows and (with the shared expert) its act rows in one launch
        const QuantRows routed{w.act, w.aq, w.as, TK, I};
        if (with_shared)
            e = launch_quantize_rows2(s, routed, QuantRows{w.shared_act, w.shared_aq, w.shared_as, t, SI},
                                      kQuantDynamic);
        else
            e = launch_quantize_rows(s, w.act, TK, I, w.aq, w.as, kQuantDynamic);
        if (e != hipSuccess) return e;
    }
    {
        ProfScope ps(ctx, "i8_down");
        // the shared expert's down product (K = shared_inter, all t rows, gate
        // 1: y = 1 * y, the dense product's value) as extra units: measured
        // against its own launch (the split-K GEMV at 256 rows, the tiled GEMM
        // above), the prefill layer went 0.653 -> 0.629 ms at chunks of 256
        // and 0.310 -> 0.291 ms at one 1024-row chunk, although its units run
        // twice the K of the routed ones
        const I8Args a{w.aq, w.as, p.perm, top_k, L->wd_mfma, L->sd, nullptr, nullptr, nullptr, gates, w.ybuf, I, H};
        const I8Args sh{w.shared_aq, w.shared_as, nullptr, 1, L->swd_mfma, L->ssd, nullptr, nullptr, nullptr,
                        nullptr, w.shared_y, SI, H};
        if ((e = grouped(std::integral_constant<int, kI8Down>(), a, sh, with_shared ? t : 0)) != hipSuccess)
            return e;
    }
    {
        ProfScope ps(ctx, "i8_combine");
        if ((e = launch_moe_prefill_combine(s, w.ybuf, idx, t, H, top_k, with_shared ? w.shared_y : nullptr, out,
                                            resid)) !=
            hipSuccess)
            return e;
    }
    return hipSuccess;
}

}  // namespace focr
