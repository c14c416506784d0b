// k_i8gemm.hip — the dense int8 GEMM of prefill (nn::linear_int8_dynamic,
// nn.rs:151-173) on large row counts: C = A . B^T in i32 on
// v_mfma_i32_32x32x32_i8, y = ((f32)acc * a_s[row]) * w_s[col] (+ bias), the
// decoder's dequant order (decoder.rs:1636). A is the quantized activation
// rows [M][K], B the weights ([N][K], output-channel-major), both in the
// tiled order of i8_tiled_act_off() (each 64-byte K stage of a row tile one
// contiguous run, already laid out as its LDS image): the quantizer writes
// A that way and the weights are retiled once per handle.
//
// Block = 4 waves on a 256 x 128 output tile (wave (wm, wn): rows 128 wm ..,
// columns 64 wn ..; 4 x 2 MFMA tiles of 32 x 32, 128 i32 accumulators per
// lane), two blocks per CU (73 KB of LDS and <= 256 VGPRs each), so one
// block's epilogue stores overlap the other's matrix-core work. K runs in
// 64-byte stages through a 3-deep LDS ring filled by direct global->LDS loads
// (global_load_lds_dwordx4, 1 KB contiguous per wave instruction: lane l
// lands at byte 16 l), issued two stages ahead, so no VGPRs stage the data.
// One barrier per stage; the waits on the loads are explicit (the compiler
// does not track the LDS side of these loads).
// LDS row layout: a staged row is 64 bytes = 4 slots of 16; slot s of row r
// holds K piece s ^ ((r >> 2) & 3) (the loading lane picks its source piece
// accordingly; swz() below). A fragment read (16 consecutive rows, one piece
// each) then touches 16 distinct 16-byte bank groups.
// Operand layout of v_mfma_i32_32x32x32_i8: lane l holds A row l % 32 and B
// column l % 32, bytes 16 (l / 32) + [0, 16) of the 32-wide K step; C element
// v of lane l is row 8 (v / 4) + 4 (l / 32) + v % 4, column l % 32.
#include "focr_internal.hpp"
#include "k_common.hpp"

namespace focr {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void;

constexpr int WM = 2, WN = 2;  // waves along the rows / columns of the block tile
constexpr int TI = 4, TJ = 2;  // 32 x 32 MFMA tiles per wave along the rows / columns
constexpr int NW = WM * WN;
// Only this 4-wave layout has run on hardware: an 8-wave variant (4 x 2 waves
// of 2 x 2 MFMA tiles, four waves per SIMD) did not finish in a timing run,
// cause not found, so other layouts are refused at compile time.
static_assert(WM == 2 && WN == 2 && TI == 4 && TJ == 2, "untested wave layout");
constexpr int WPE = 2;         // waves per SIMD: two blocks per CU
constexpr int TM = WM * 32 * TI;  // block rows (256)
constexpr int TN = WN * 32 * TJ;  // block columns (128)
constexpr int BK = 64;       // K bytes per stage
constexpr int NST = 3;       // LDS ring depth
constexpr int NTHR = 64 * NW;
constexpr int SR = BK / 16;  // 16-byte slots per staged row
constexpr int A_SLOTS = TM * SR, B_SLOTS = TN * SR, ST_SLOTS = A_SLOTS + B_SLOTS;
constexpr int A_LOADS = TM * BK / 1024 / NW;  // 1 KB load instructions per wave per stage
constexpr int B_LOADS = TN * BK / 1024 / NW;
static_assert(A_LOADS * NW * 1024 == TM * BK && B_LOADS * NW * 1024 == TN * BK && B_LOADS >= 1, "stage split");
constexpr int LOADS_PER_STAGE = A_LOADS + B_LOADS;

constexpr int RPI = 64 / SR;  // staged rows per 1 KB load instruction

// slot key of staged row r: the 256 / (16 SR) rows sharing one 256-byte bank
// line get distinct keys, so 16 consecutive rows read at one K piece touch 16
// distinct 16-byte bank groups
__device__ __forceinline__ int swz(int r) { return (r / (16 / SR)) & (SR - 1); }
// the activation order is the shared one of k_common.hpp (i8_tiled_act_off)
static_assert(TM == kI8TiledRows && BK == kI8TiledStage && SR == 4, "tiled activation order");

// s_waitcnt vmcnt(n) only (expcnt / lgkmcnt left alone), n < 64: the low 4
// bits of the count in bits 3:0, the high 2 in bits 15:14
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt field");
    __builtin_amdgcn_s_waitcnt((N & 15) | 0x0F70 | ((N >> 4) << 14));
}

// wait until at most `later` stages' loads (issued after the one waited
// for) are outstanding, later in [0, NST - 1]
template <int L = NST - 1>
__device__ __forceinline__ void wait_stage(int later) {
    static_assert(LOADS_PER_STAGE * (NST - 1) < 64, "vmcnt field");
    if constexpr (L == 0) {
        wait_vmcnt<0>();
    } else {
        if (later >= L) wait_vmcnt<LOADS_PER_STAGE * L>();
        else wait_stage<L - 1>(later);
    }
}

// LDS reads of the previous stage done, then the workgroup barrier; no fence,
// so loads still in flight to the LDS ring are not waited for. The lgkmcnt
// wait is also issued through the builtin so that the compiler's own wait
// bookkeeping knows nothing LDS/scalar is pending after it.
__device__ __forceinline__ void stage_barrier() {
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0); vmcnt, expcnt untouched
    asm volatile("s_barrier" ::: "memory");
}

struct GemmArgs {
    const int8_t* A;      // [M][K] in the tiled order, tile height TM
    const float* a_scale;  // [M]
    const int8_t* B;      // [N][K] in the tiled order, tile height TN
    const float* w_scale;  // [N]
    const float* bias;     // [N] or null
    float* out;            // [M][N]
    int M, N, K;
};

__global__ __launch_bounds__(NTHR) __attribute__((amdgpu_waves_per_eu(WPE, WPE))) void i8_gemm256_kernel(
    const GemmArgs a) {
    // [NST] stages of (A slots, B slots), then the TM activation scales. LDS
    // is indexed through this array (LDS, not flat, access).
    extern __shared__ v4i lds[];
    float* scl = reinterpret_cast<float*>(lds + NST * ST_SLOTS);
    const int tid = threadIdx.x;
    const int wave = tid >> 6, l = tid & 63;
    const int wm = wave / WN, wn = wave % WN;
    const int h = l >> 5, c32 = l & 31;
    const int m0 = blockIdx.x * TM, n0 = blockIdx.y * TN;
    const int K = a.K;
    const int nst = K / BK;

    for (int r = tid; r < TM; r += NTHR) scl[r] = a.a_scale[min(m0 + r, a.M - 1)];
    // this lane's two output columns: weight scale and bias in registers, loaded
    // before the main loop so that no load is pending when the stores start
    const bool has_bias = a.bias != nullptr;
    float wsr[TJ], bbr[TJ];
#pragma unroll
    for (int j = 0; j < TJ; ++j) {
        const int col = min(n0 + 32 * (TJ * wn + j) + c32, a.N - 1);
        wsr[j] = a.w_scale[col];
        bbr[j] = has_bias ? a.bias[col] : 0.0f;
    }

    // Both operands come in the tiled order (see i8_tiled_act_off): each stage of
    // a row tile is one contiguous run in the exact LDS image, so load
    // instruction i of the wave copies 1 KB (q = wave + NW i) of it.
    const size_t a_stage = static_cast<size_t>(TM) * BK, b_stage = static_cast<size_t>(TN) * BK;
    const int8_t* ga = a.A + blockIdx.x * nst * a_stage + 1024 * wave + 16 * l;
    const int8_t* gb = a.B + blockIdx.y * nst * b_stage + 1024 * wave + 16 * l;
    auto issue = [&](int st) {
        v4i* base = lds + (st % NST) * ST_SLOTS;
#pragma unroll
        for (int i = 0; i < A_LOADS; ++i)
            __builtin_amdgcn_global_load_lds(ga + st * a_stage + 1024 * NW * i, (lds_void*)(base + 64 * (wave + NW * i)), 16,
                                             0, 0);
#pragma unroll
        for (int i = 0; i < B_LOADS; ++i)
            __builtin_amdgcn_global_load_lds(gb + st * b_stage + 1024 * NW * i,
                                             (lds_void*)(base + A_SLOTS + 64 * (wave + NW * i)), 16, 0, 0);
    };

    v16i acc[TI][TJ];
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j) acc[i][j] = v16i{};

    int ar[TI], br[TJ];
#pragma unroll
    for (int i = 0; i < TI; ++i) ar[i] = 32 * (TI * wm + i) + c32;
#pragma unroll
    for (int j = 0; j < TJ; ++j) br[j] = 32 * (TJ * wn + j) + c32;

    // fragments of one 32-byte K step, double-buffered by step parity
    v4i fa[2][TI], fb[2][TJ];
    auto read_step = [&](const v4i* sa, int s, int buf) {
        const v4i* sb = sa + A_SLOTS;
        const int p = 2 * s + h;  // this lane's 16-byte piece of the 32-byte K step
#pragma unroll
        for (int i = 0; i < TI; ++i) fa[buf][i] = sa[ar[i] * SR + (p ^ swz(ar[i]))];
#pragma unroll
        for (int j = 0; j < TJ; ++j) fb[buf][j] = sb[br[j] * SR + (p ^ swz(br[j]))];
    };
    auto mfma_step = [&](int buf) {
#pragma unroll
        for (int i = 0; i < TI; ++i)
#pragma unroll
            for (int j = 0; j < TJ; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[buf][i], fb[buf][j], acc[i][j], 0, 0, 0);
    };
    constexpr int NS = BK / 32;  // K steps per stage

    // Software pipeline: the LDS reads of each K step are issued before the
    // MFMAs of the step before it, and the barrier that hands over stage c + 1
    // sits before stage c's last step, so the first reads of stage c + 1 run
    // under that step's MFMAs. After that barrier every wave has finished
    // reading stage c, whose slot stage c + NST then refills.
#pragma unroll
    for (int st = 0; st < NST; ++st)
        if (st < nst) issue(st);
    wait_stage(min(NST - 1, nst - 1));
    stage_barrier();
    read_step(lds, 0, 0);
    auto stage_steps = [&](const v4i* sa) {
#pragma unroll
        for (int s = 0; s < NS - 1; ++s) {
            read_step(sa, s + 1, (s + 1) & 1);
            mfma_step(s & 1);
            // one MFMA, then the next step's reads, then the other MFMAs:
            // the wait for this step's fragments (issued a whole step ago)
            // comes before the new reads, not after them (the compiler's
            // wait there is lgkmcnt(0)); the order is pinned because the
            // scheduler would sink the reads below to reuse registers
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, TI + TJ, 0);
            __builtin_amdgcn_sched_group_barrier(0x008, TI * TJ - 1, 0);
        }
    };
    // every stage but the last (peeled, so the loop body has no branch)
    for (int c = 0; c + 1 < nst; ++c) {
        stage_steps(lds + (c % NST) * ST_SLOTS);
        // stage c + 1 landed (up to NST - 2 later stages may be in flight)
        wait_stage(min(NST - 2, nst - 2 - c));
        stage_barrier();
        if (c + NST < nst) issue(c + NST);
        read_step(lds + ((c + 1) % NST) * ST_SLOTS, 0, NS & 1);
        mfma_step((NS - 1) & 1);
        __builtin_amdgcn_sched_group_barrier(0x100, TI + TJ, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, TI * TJ, 0);
    }
    stage_steps(lds + ((nst - 1) % NST) * ST_SLOTS);
    mfma_step((NS - 1) & 1);

    // epilogue: y = ((f32)acc * a_s) * w_s (+ bias). Element v of MFMA tile
    // (i, j) is row r0 + 8 (v / 4) + v % 4 (r0 = 32 (TI wm + i) + 4 h), so the
    // lane's row scales come as 16-byte LDS reads of 4 consecutive rows. Tiles
    // wholly inside the output store without per-element checks.
    const bool full = m0 + TM <= a.M && n0 + TN <= a.N;
    const v4f* s4 = reinterpret_cast<const v4f*>(scl);
#pragma unroll
    for (int i = 0; i < TI; ++i) {
        const int r0 = 32 * (TI * wm + i) + 4 * h;
        v4f rs[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) rs[q] = s4[(r0 + 8 * q) >> 2];
#pragma unroll
        for (int j = 0; j < TJ; ++j) {
            const int col = n0 + 32 * (TJ * wn + j) + c32;
            float y[16];
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                y[v] = (static_cast<float>(acc[i][j][v]) * rs[v >> 2][v & 3]) * wsr[j];
                if (has_bias) y[v] = y[v] + bbr[j];
            }
            // non-temporal: the f32 output (224 MB at M = 8192) streams past
            // the L2 instead of evicting the operand tiles the other blocks
            // re-read (121 -> 117 us at M = 8192, 30.5 -> 28.5 us at 2048)
            if (full) {
                float* o = a.out + static_cast<size_t>(m0 + r0) * a.N + col;
#pragma unroll
                for (int v = 0; v < 16; ++v)
                    __builtin_nontemporal_store(y[v], o + static_cast<size_t>(8 * (v >> 2) + (v & 3)) * a.N);
            } else if (col < a.N) {
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    const int row = m0 + r0 + 8 * (v >> 2) + (v & 3);
                    if (row < a.M) __builtin_nontemporal_store(y[v], a.out + static_cast<size_t>(row) * a.N + col);
                }
            }
        }
    }
}

// The tiled operand order: rows in tiles of T (256 for the activations, 128
// for the weights), each tile stored stage by stage (64 K bytes), each stage
// as T rows of 64 bytes with the 16-byte piece p of row r at slot
// p ^ swz(r) (the LDS image); for the activations i8_tiled_act_off
// (k_common.hpp) gives the byte offset of K piece p of row r.

// weights [N][K] -> tiled order (tile height TN), rows past N zero; one
// thread per output 16-byte unit
__global__ __launch_bounds__(256) void retile_tiled_kernel(const int8_t* __restrict__ w, int N, int K,
                                                           int8_t* __restrict__ wt, size_t units) {
    const size_t u = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x;
    if (u >= units) return;
    const int nst = K / BK;
    const int sl = static_cast<int>(u % SR), rr = static_cast<int>((u / SR) % TN);
    const size_t ts = u / (static_cast<size_t>(SR) * TN);
    const int st = static_cast<int>(ts % nst), t = static_cast<int>(ts / nst);
    const int n = t * TN + rr, p = st * SR + (sl ^ swz(rr));
    v4i v = {0, 0, 0, 0};
    if (n < N) v = *reinterpret_cast<const v4i*>(w + static_cast<size_t>(n) * K + 16 * p);
    reinterpret_cast<v4i*>(wt)[u] = v;
}

// nn::linear_int8_dynamic's activation quantization (nn.rs:151-173: amax over
// the row, a_scale = amax / 127 or 1 for an all-zero row, q = x / a_scale
// rounded by `rule`) written straight into the tiled order (tile height TM).
// One wave per row, four rows per block; lane l handles the float4s
// l + 64 j of the row (every load instruction reads 1 KB contiguous) and
// stores each as one 4-byte word of its 16-byte piece. Rows of the last tile
// past M are left unwritten (their products are never stored). F4L > 0: the
// lane's F4L float4s stay in registers between the amax and the quantize
// pass (x read once); F4L = 0: any K, x read twice. NORM (F4L > 0): the row
// is first RMS-normalised as the decoder's rms_norm does it (the sum of
// squares in f64, rstd = 1 / sqrt(ss / K + eps) rounded to f32, y = (x *
// rstd) * w), so the f32 normed rows never go to memory and their launch goes.
template <int F4L, bool NORM = false>
__global__ __launch_bounds__(256) void quantize_rows_tiled_kernel(const float* __restrict__ x, int M, int K,
                                                                  int8_t* __restrict__ xt, float* __restrict__ xs,
                                                                  int rule, const float* __restrict__ nw, float eps) {
    static_assert(!NORM || F4L > 0, "the normed row is held in registers");
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6), l = threadIdx.x & 63;
    if (row >= M) return;  // whole wave
    const v4f* xr = reinterpret_cast<const v4f*>(x + static_cast<size_t>(row) * K);
    const int nf = K / 4, nst = K / BK;
    auto absmax = [](float m, const v4f& v) {
        return fmaxf(fmaxf(fmaxf(fmaxf(m, fabsf(v[0])), fabsf(v[1])), fabsf(v[2])), fabsf(v[3]));
    };
    // float4 f = K elements 4 f .. 4 f + 3 = word f % 4 of K piece f / 4
    auto put = [&](int f, const v4f& v, float a_scale, float inv) {
        uint32_t word = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e)
            word |= static_cast<uint32_t>(static_cast<uint8_t>(quant_rule(v[e], a_scale, inv, rule))) << (8 * e);
        *reinterpret_cast<uint32_t*>(xt + i8_tiled_act_off(row, f >> 2, nst) + 4 * (f & 3)) = word;
    };
    float amax = 0.0f;
    if constexpr (F4L > 0) {
        v4f v[F4L];
#pragma unroll
        for (int j = 0; j < F4L; ++j) v[j] = l + 64 * j < nf ? xr[l + 64 * j] : v4f{0.0f, 0.0f, 0.0f, 0.0f};
        if constexpr (NORM) {
            const v4f* w4 = reinterpret_cast<const v4f*>(nw);
            v4f g[F4L];
#pragma unroll
            for (int j = 0; j < F4L; ++j) g[j] = l + 64 * j < nf ? w4[l + 64 * j] : v4f{0.0f, 0.0f, 0.0f, 0.0f};
            double ss = 0.0;
#pragma unroll
            for (int j = 0; j < F4L; ++j)
#pragma unroll
                for (int e = 0; e < 4; ++e) ss = fma(static_cast<double>(v[j][e]), static_cast<double>(v[j][e]), ss);
            ss = wave_sum_d_full(ss);
            const float rstd = static_cast<float>(1.0 / sqrt(ss / static_cast<double>(K) + static_cast<double>(eps)));
#pragma unroll
            for (int j = 0; j < F4L; ++j)
#pragma unroll
                for (int e = 0; e < 4; ++e) v[j][e] = (v[j][e] * rstd) * g[j][e];
        }
#pragma unroll
        for (int j = 0; j < F4L; ++j) amax = absmax(amax, v[j]);
        amax = wave_max_f_full(amax);
        const float a_scale = amax > 0.0f ? amax / 127.0f : 1.0f;
        const float inv = 1.0f / a_scale;
#pragma unroll
        for (int j = 0; j < F4L; ++j)
            if (l + 64 * j < nf) put(l + 64 * j, v[j], a_scale, inv);
        if (l == 0) xs[row] = a_scale;
    } else {
        for (int f = l; f < nf; f += 64) amax = absmax(amax, xr[f]);
        amax = wave_max_f_full(amax);
        const float a_scale = amax > 0.0f ? amax / 127.0f : 1.0f;
        const float inv = 1.0f / a_scale;
        for (int f = l; f < nf; f += 64) put(f, xr[f], a_scale, inv);
        if (l == 0) xs[row] = a_scale;
    }
}

}  // namespace

size_t i8_gemm256_lds_bytes() {
    return static_cast<size_t>(NST) * ST_SLOTS * 16 + TM * sizeof(float);
}

bool i8_gemm256_supported(int m, int n, int k) {
    return m >= TM && n > 0 && k >= BK && k % BK == 0 && i8_gemm256_lds_bytes() <= max_lds_per_block();
}

size_t i8_gemm256_a_bytes(int m, int k) { return static_cast<size_t>((m + TM - 1) / TM) * TM * k; }
size_t i8_gemm256_b_bytes(int n, int k) { return static_cast<size_t>((n + TN - 1) / TN) * TN * k; }

hipError_t launch_i8_gemm256_retile_b(hipStream_t s, const int8_t* w, int n, int k, int8_t* wt) {
    if (n <= 0 || k < BK || k % BK) return hipErrorInvalidValue;
    const size_t units = i8_gemm256_b_bytes(n, k) / 16;
    FOCR_LAUNCH(retile_tiled_kernel, dim3(static_cast<unsigned>((units + 255) / 256)), dim3(256), 0, s, w, n, k, wt,
                units);
    return hipGetLastError();
}

hipError_t launch_rms_norm_quantize_rows_tiled(hipStream_t s, const float* x, const float* nw, float eps, int m,
                                              int k, int8_t* xt, float* xs, int rule) {
    if (m <= 0 || k < BK || k % BK || !nw || reinterpret_cast<uintptr_t>(x) % 16 || reinterpret_cast<uintptr_t>(nw) % 16)
        return hipErrorInvalidValue;
    const dim3 grid(static_cast<unsigned>((m + 3) / 4));
    const int f4l = (k / 4 + 63) / 64;  // float4s per lane
    if (f4l <= 4)
        FOCR_LAUNCH((quantize_rows_tiled_kernel<4, true>), grid, dim3(256), 0, s, x, m, k, xt, xs, rule, nw, eps);
    else if (f4l <= 8)
        FOCR_LAUNCH((quantize_rows_tiled_kernel<8, true>), grid, dim3(256), 0, s, x, m, k, xt, xs, rule, nw, eps);
    else if (f4l <= 16)
        FOCR_LAUNCH((quantize_rows_tiled_kernel<16, true>), grid, dim3(256), 0, s, x, m, k, xt, xs, rule, nw, eps);
    else
        return hipErrorInvalidValue;  // rows wider than 4096: the separate norm
    return hipGetLastError();
}

hipError_t launch_quantize_rows_tiled(hipStream_t s, const float* x, int m, int k, int8_t* xt, float* xs, int rule) {
    if (m <= 0 || k < BK || k % BK) return hipErrorInvalidValue;
    const dim3 grid(static_cast<unsigned>((m + 3) / 4));
    const int f4l = (k / 4 + 63) / 64;  // float4s per lane
    if (f4l <= 4)
        FOCR_LAUNCH(quantize_rows_tiled_kernel<4>, grid, dim3(256), 0, s, x, m, k, xt, xs, rule, nullptr,
                    0.0f);
    else if (f4l <= 8)
        FOCR_LAUNCH(quantize_rows_tiled_kernel<8>, grid, dim3(256), 0, s, x, m, k, xt, xs, rule, nullptr,
                    0.0f);
    else if (f4l <= 16)
        FOCR_LAUNCH(quantize_rows_tiled_kernel<16>, grid, dim3(256), 0, s, x, m, k, xt, xs, rule, nullptr,
                    0.0f);
    else if (f4l <= 28)
        FOCR_LAUNCH(quantize_rows_tiled_kernel<28>, grid, dim3(256), 0, s, x, m, k, xt, xs, rule, nullptr,
                    0.0f);
    else
        FOCR_LAUNCH(quantize_rows_tiled_kernel<0>, grid, dim3(256), 0, s, x, m, k, xt, xs, rule, nullptr,
                    0.0f);
    return hipGetLastError();
}

hipError_t launch_i8_gemm256(hipStream_t s, const int8_t* xt, const float* xs, int m, int k, const int8_t* wt,
                             const float* ws, int n, const float* bias, float* y) {
    if (!i8_gemm256_supported(m, n, k)) return hipErrorInvalidValue;
    GemmArgs a{xt, xs, wt, ws, bias, y, m, n, k};
    const dim3 grid((m + TM - 1) / TM, (n + TN - 1) / TN);
    FOCR_LAUNCH(i8_gemm256_kernel, grid, dim3(NTHR), i8_gemm256_lds_bytes(), s, a);
    return hipGetLastError();
}

}  // namespace focr
