// k_attn.hip — causal prefill attention (decoder.rs:568-640 prefill_attention,
// :1282-1340 chunk_prefill_attention) on the f32 matrix cores.
//
// A chunk's cs queries (global positions c0 .. c0 + cs - 1) attend keys
// [0, t] of the f32 prefix, per head, softmax(q.k * 1/sqrt(128)) . v. The
// scores and the P.V products are f32 MFMAs (v_mfma_f32_16x16x4_f32: exact
// f32 products, f32 accumulation), so the result matches the reference's
// f32 attention to rounding.
//
// Block = 4 waves on one head and 64 query rows (16 per wave); the block
// walks its key range in tiles of 32 keys, staged in LDS and shared by the
// waves (34 KB, so three blocks share a CU). Per wave and 16-key subtile,
// S^T = K . Q^T (A = 16 keys x 4 dims from
// LDS, B = 4 dims x 16 query rows from registers), so the accumulator lands
// with lane (g = lane / 16, j = lane % 16) holding S[row j][keys 4g .. 4g + 3]
// — exactly the B operand P^T[key][row j] the P.V product needs (keys taken in
// the order 16n + 4g + r), with A = V^T from LDS: the softmax probabilities
// never leave their registers. Output dims are taken in the order
// 8 * (4g + r') + m, so each lane ends holding 32 consecutive dims of its row.
// Dims of the score dot are taken in the order 32g + s (s = 0..31).
//
// The scores are kept in base-2 units: the kernel's scale is
// log2(e) / sqrt(128), so exp(s / sqrt(128) - max) is exp2 of the scaled
// score minus its max (the hardware v_exp_f32, about 1 ulp; the argument's
// extra rounding is ~|x| * 2^-24, far inside the attention's 1e-4).
//
// Long prefixes are split into key ranges over more blocks (split-K); each
// writes its running max, denominator and unnormalised output, and a merge
// kernel folds them (log-sum-exp). A row whose keys all lie in other ranges
// contributes max -inf and nothing else. The ranges hold equal numbers of
// tiles, sized so the blocks that have keys fill the GPU about once (the
// causal chunk's row tiles need different numbers of tiles).
#include "focr_internal.hpp"
#include "k_common.hpp"

namespace focr {
namespace {

constexpr int kD = 128;          // head_dim
constexpr int kKT = 32;          // keys per LDS tile
constexpr int kLdsRow = kD + 4;  // padded LDS row (floats)
constexpr int kBlocksPerCu = 3;  // the kernel's residency (LDS 34 KB, waves_per_eu 3)
constexpr float kLog2e = 1.4426950408889634f;
typedef float v4f __attribute__((ext_vector_type(4)));

struct AttnArgs {
    const float* q;  // row i, head h at q + i * ldq + h * hq
    const float* k;  // key j, head h at k + j * ldk + h * hk
    const float* v;
    float* out;      // single range: normalised context, out + i * ldo + h * ho
    float* part_o;   // split: [split][head][row][kD] unnormalised
    float* part_ml;  // split: [split][head][row][2] (base-2 max, denominator)
    int ldq, hq, ldk, hk, ldv, hv, ldo, ho;
    int cs, c0, c1, heads, split_len, nsplit;
    float scale;     // log2(e) / sqrt(head_dim)
};

// Combine lane l's value with lanes l ^ 16, l ^ 32, l ^ 48 (the four 16-lane
// rows): gfx950's v_permlane16_swap / v_permlane32_swap of a value with itself
// put both partners of an xor-16 (xor-32) pair in each lane (VALU; the
// shuffle form went through ds_bpermute at LDS latency). The pairs combine as
// the xor butterfly did: (r0 op r1) op (r2 op r3) in every lane.
__device__ __forceinline__ float perm16_lo(float v, float& hi) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    hi = __uint_as_float(r[1]);
    return __uint_as_float(r[0]);
}
__device__ __forceinline__ float perm32_lo(float v, float& hi) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    hi = __uint_as_float(r[1]);
    return __uint_as_float(r[0]);
}
__device__ __forceinline__ float wave16_max(float v) {
    float b;
    const float a = perm16_lo(v, b);
    v = fmaxf(a, b);
    const float c = perm32_lo(v, b);
    return fmaxf(c, b);
}
__device__ __forceinline__ float wave16_sum(float v) {
    float b;
    const float a = perm16_lo(v, b);
    v = a + b;
    const float c = perm32_lo(v, b);
    return c + b;
}

constexpr int kSub = kKT / 16;             // 16-key MFMA subtiles per tile
constexpr int kPieces = kKT * kD / 4 / 256;  // float4 of one matrix per thread and tile

__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(kBlocksPerCu))) void attn_prefill_kernel(
    const AttnArgs a) {
    extern __shared__ float4 lds_kv4[];  // K tile then V tile, [kKT][kLdsRow] floats each
    float* lk = reinterpret_cast<float*>(lds_kv4);
    float* lv = lk + kKT * kLdsRow;
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int g = lane >> 4, j = lane & 15;
    const int h = blockIdx.y;
    const int split = blockIdx.z;
    const int row0 = blockIdx.x * 64;            // block's first chunk row
    const int wrow = row0 + wave * 16 + j;        // this lane's chunk row
    const int qrow = wrow < a.cs ? wrow : a.cs - 1;
    const int t = a.c0 + wrow;                    // its global position
    // keys this block needs: [0, min(c1, c0 + row0 + 64)), this split's part
    const int kmax = min(a.c1, a.c0 + row0 + 64);
    const int ks = split * a.split_len;
    const int ke = min(ks + a.split_len, kmax);
    // a range past the row tile's last key: nothing to do or write (the
    // merge skips it by the same bound); block-uniform
    if (ks >= ke) return;

    // Q fragment: qf[s] = q[row j][32g + s], s = 0..31
    float qf[32];
    {
        const float4* qp = reinterpret_cast<const float4*>(a.q + static_cast<size_t>(qrow) * a.ldq +
                                                           static_cast<size_t>(h) * a.hq + 32 * g);
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const v4f x = *reinterpret_cast<const v4f*>(qp + u);
            qf[4 * u] = x.x;
            qf[4 * u + 1] = x.y;
            qf[4 * u + 2] = x.z;
            qf[4 * u + 3] = x.w;
        }
    }
    v4f oacc[8];
#pragma unroll
    for (int m = 0; m < 8; ++m) oacc[m] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
    float m_run = -INFINITY, l_run = 0.0f;

    // tile loads: 32 keys x 128 floats = 1024 float4 per matrix, 4 per thread
    const int c4 = threadIdx.x & 31;  // float4 column
    const int r8 = threadIdx.x >> 5;  // 8 rows per pass
    const float* kh = a.k + static_cast<size_t>(h) * a.hk + 4 * c4;
    const float* vh = a.v + static_cast<size_t>(h) * a.hv + 4 * c4;
    // Tile loads of keys kb .. kb + kKT - 1 (rows clamped into the prefix; a
    // row past the range end is never used) and their LDS stores.
    v4f pk[kPieces], pv[kPieces];
    auto load_tile = [&](int kb) {
#pragma unroll
        for (int p = 0; p < kPieces; ++p) {
            int key = kb + r8 + 8 * p;
            key = key < a.c1 ? key : a.c1 - 1;
            pk[p] = *reinterpret_cast<const v4f*>(kh + static_cast<size_t>(key) * a.ldk);
            pv[p] = *reinterpret_cast<const v4f*>(vh + static_cast<size_t>(key) * a.ldv);
        }
    };
    auto store_tile = [&]() {
#pragma unroll
        for (int p = 0; p < kPieces; ++p) {
            *reinterpret_cast<v4f*>(lk + (r8 + 8 * p) * kLdsRow + 4 * c4) = pk[p];
            *reinterpret_cast<v4f*>(lv + (r8 + 8 * p) * kLdsRow + 4 * c4) = pv[p];
        }
    };
    if (ks < ke) {
        load_tile(ks);
        store_tile();
    }
    // every load so far (the Q fragment too) complete on every path into
    // the loop, so the loop's first MFMAs wait for none of the tile loads
    // issued inside it (vmcnt(0): the counter drains in issue order)
    __builtin_amdgcn_s_waitcnt(0x0F70);
    __syncthreads();
    // Each iteration issues the next tile's loads first, consumes the
    // current tile from LDS while they are in flight, then (after every wave
    // has read it) stores the next tile over it. The loads are consumed in
    // the iteration that issues them: a load carried into the next iteration
    // was folded with the one before the loop into a single load at the top
    // of the loop, which waited out a full memory round trip on every tile.
    for (int kb = ks; kb < ke; kb += kKT) {
        const bool more = kb + kKT < ke;
        if (more) load_tile(kb + kKT);
        __builtin_amdgcn_sched_barrier(0);  // the loads go out before the tile's MFMAs

        // S^T for the subtiles of 16 keys; each score dot runs as two
        // 16-step MFMA chains (dims 32g + 16h + [0, 16), h = 0, 1) added at
        // the end, halving the f32 accumulation chain of the 128-term dot.
        // The 2 * kSub chains advance together: each step reads their four
        // dims of K (one 16-byte LDS read per chain) and issues one MFMA per
        // chain and dim, so a chain's dependent MFMAs interleave with the
        // other chains' (each chain's own order is unchanged: u, then dim).
        v4f sc[kSub][2];
#pragma unroll
        for (int n = 0; n < kSub; ++n) sc[n][0] = sc[n][1] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int u2 = 0; u2 < 4; ++u2) {
            v4f kf[kSub][2];
#pragma unroll
            for (int n = 0; n < kSub; ++n)
#pragma unroll
                for (int hh = 0; hh < 2; ++hh)
                    kf[n][hh] = *reinterpret_cast<const v4f*>(lk + (16 * n + j) * kLdsRow + 32 * g + 16 * hh + 4 * u2);
#pragma unroll
            for (int c = 0; c < 4; ++c)
#pragma unroll
                for (int n = 0; n < kSub; ++n)
#pragma unroll
                    for (int hh = 0; hh < 2; ++hh)
                        sc[n][hh] = __builtin_amdgcn_mfma_f32_16x16x4f32(kf[n][hh][c], qf[16 * hh + 4 * u2 + c],
                                                                         sc[n][hh], 0, 0, 0);
        }
        v4f sacc[kSub];
#pragma unroll
        for (int n = 0; n < kSub; ++n) sacc[n] = sc[n][0] + sc[n][1];
        // scale, causal / range mask, online softmax (row j over 4 lanes)
        float pr[kSub][4];
        float tmax = -INFINITY;
#pragma unroll
        for (int n = 0; n < kSub; ++n)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int key = kb + 16 * n + 4 * g + r;
                const float sv = sacc[n][r] * a.scale;
                const bool ok = key <= t && key < ke;
                pr[n][r] = ok ? sv : -INFINITY;
                tmax = fmaxf(tmax, pr[n][r]);
            }
        tmax = wave16_max(tmax);
        const float m_new = fmaxf(m_run, tmax);
        const float corr = m_run == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m_run - m_new);
        float tsum = 0.0f;
#pragma unroll
        for (int n = 0; n < kSub; ++n)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float p = pr[n][r] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(pr[n][r] - m_new);
                pr[n][r] = p;
                tsum += p;
            }
        tsum = wave16_sum(tsum);
        l_run = l_run * corr + tsum;
        m_run = m_new;
        // the running output rescaled to the new max, then this tile's
        // V^T . P^T accumulated into it (step (n, r) is key kb + 16n + 4g + r)
#pragma unroll
        for (int m = 0; m < 8; ++m) oacc[m] = oacc[m] * corr;
#pragma unroll
        for (int n = 0; n < kSub; ++n)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float* vr = lv + (16 * n + 4 * g + r) * kLdsRow + 8 * j;
                const v4f v0 = *reinterpret_cast<const v4f*>(vr);
                const v4f v1 = *reinterpret_cast<const v4f*>(vr + 4);
                const float b = pr[n][r];
                oacc[0] = __builtin_amdgcn_mfma_f32_16x16x4f32(v0.x, b, oacc[0], 0, 0, 0);
                oacc[1] = __builtin_amdgcn_mfma_f32_16x16x4f32(v0.y, b, oacc[1], 0, 0, 0);
                oacc[2] = __builtin_amdgcn_mfma_f32_16x16x4f32(v0.z, b, oacc[2], 0, 0, 0);
                oacc[3] = __builtin_amdgcn_mfma_f32_16x16x4f32(v0.w, b, oacc[3], 0, 0, 0);
                oacc[4] = __builtin_amdgcn_mfma_f32_16x16x4f32(v1.x, b, oacc[4], 0, 0, 0);
                oacc[5] = __builtin_amdgcn_mfma_f32_16x16x4f32(v1.y, b, oacc[5], 0, 0, 0);
                oacc[6] = __builtin_amdgcn_mfma_f32_16x16x4f32(v1.z, b, oacc[6], 0, 0, 0);
                oacc[7] = __builtin_amdgcn_mfma_f32_16x16x4f32(v1.w, b, oacc[7], 0, 0, 0);
            }
        if (more) {  // block-uniform
            __syncthreads();  // every wave is done with this tile
            store_tile();
            __syncthreads();
        }
    }
    if (wrow >= a.cs) return;
    // lane (g, j) holds O[row j][32g + 8r' + m] in oacc[m][r']
    if (a.nsplit == 1) {
        const float inv = 1.0f / l_run;
        float* op = a.out + static_cast<size_t>(wrow) * a.ldo + static_cast<size_t>(h) * a.ho + 32 * g;
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
            float4 x0, x1;
            x0.x = oacc[0][rr] * inv;
            x0.y = oacc[1][rr] * inv;
            x0.z = oacc[2][rr] * inv;
            x0.w = oacc[3][rr] * inv;
            x1.x = oacc[4][rr] * inv;
            x1.y = oacc[5][rr] * inv;
            x1.z = oacc[6][rr] * inv;
            x1.w = oacc[7][rr] * inv;
            *reinterpret_cast<float4*>(op + 8 * rr) = x0;
            *reinterpret_cast<float4*>(op + 8 * rr + 4) = x1;
        }
        return;
    }
    const size_t pidx = (static_cast<size_t>(split) * a.heads + h) * a.cs + wrow;
    float* op = a.part_o + pidx * kD + 32 * g;
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
        *reinterpret_cast<float4*>(op + 8 * rr) = make_float4(oacc[0][rr], oacc[1][rr], oacc[2][rr], oacc[3][rr]);
        *reinterpret_cast<float4*>(op + 8 * rr + 4) = make_float4(oacc[4][rr], oacc[5][rr], oacc[6][rr], oacc[7][rr]);
    }
    if (g == 0) *reinterpret_cast<float2*>(a.part_ml + pidx * 2) = make_float2(m_run, l_run);
}

// Fold the key ranges: out = sum_s 2^(m_s - M) O_s / sum_s 2^(m_s - M) l_s,
// M = max_s m_s, the maxima in base-2 units (a range with no key of the row
// has m = -inf, l = 0, O = 0).
// Thread = one dim of one (row, head).
// Only the ranges below the row tile's last key were written (ns of them).
// Up to kMergeBatch ranges, every range's (max, denominator) and output
// value are requested at once (clamped duplicates past ns, never used),
// then folded in split order; a loop that loaded one split at a time waited
// on each in turn. More splits take that loop. Both fold the same values in
// the same order.
constexpr int kMergeBatch = 16;

__global__ __launch_bounds__(128) void attn_merge_kernel(const AttnArgs a) {
    const int row = blockIdx.x, h = blockIdx.y, d = threadIdx.x;
    // the row's 64-row tile has keys [0, kmax): the ranges from kmax on had
    // no block write them
    const int kmax = min(a.c1, a.c0 + (row / 64 + 1) * 64);
    const int ns = min(a.nsplit, (kmax + a.split_len - 1) / a.split_len);
    float den = 0.0f, acc = 0.0f;
    if (ns <= kMergeBatch) {
        float ms[kMergeBatch], ls[kMergeBatch], os[kMergeBatch];
#pragma unroll
        for (int s = 0; s < kMergeBatch; ++s) {
            const int sc = s < ns ? s : ns - 1;
            const size_t pidx = (static_cast<size_t>(sc) * a.heads + h) * a.cs + row;
            ms[s] = a.part_ml[pidx * 2];
            ls[s] = a.part_ml[pidx * 2 + 1];
            os[s] = a.part_o[pidx * kD + d];
        }
        // every use unconditional (a guarded use lets the compiler sink the
        // load under the guard, one wait per split again): the duplicates
        // past ns repeat the last written range's max, and an unused range
        // adds a selected +0 (the sums never hold -0, so x + 0 == x)
        float M = -INFINITY;
#pragma unroll
        for (int s = 0; s < kMergeBatch; ++s) M = fmaxf(M, ms[s]);
#pragma unroll
        for (int s = 0; s < kMergeBatch; ++s) {
            const bool use = s < ns && ms[s] != -INFINITY;
            const float w = __builtin_amdgcn_exp2f((use ? ms[s] : M) - M);
            const float dl = w * ls[s], da = w * os[s];
            den += use ? dl : 0.0f;
            acc += use ? da : 0.0f;
        }
    } else {
        float M = -INFINITY;
        for (int s = 0; s < ns; ++s)
            M = fmaxf(M, a.part_ml[((static_cast<size_t>(s) * a.heads + h) * a.cs + row) * 2]);
        for (int s = 0; s < ns; ++s) {
            const size_t pidx = (static_cast<size_t>(s) * a.heads + h) * a.cs + row;
            const float ms = a.part_ml[pidx * 2];
            if (ms == -INFINITY) continue;
            const float w = __builtin_amdgcn_exp2f(ms - M);
            den += w * a.part_ml[pidx * 2 + 1];
            acc += w * a.part_o[pidx * kD + d];
        }
    }
    a.out[static_cast<size_t>(row) * a.ldo + static_cast<size_t>(h) * a.ho + d] = acc / den;
}

// The same merge with the next product's activation quantization fused in
// (o_proj's linear_int8_dynamic: the dynamic rule over the whole output row):
// one block per row over every head, thread t folding the float4 groups
// t + 256 i of the row's heads * 128 values exactly as attn_merge_kernel
// folds each value (the same splits, order and expressions), then the row's
// amax, a_scale = amax / 127 (1 for a zero row) and the codes as the row
// quantizers form them, written row-major (TILED false) or in the 256 x 128
// GEMM's tiled order, four codes to a word. The f32 context rows are never
// stored and the quantize launch goes.
constexpr int kMqGroups = 2;  // float4 groups per thread: rows up to 2048 values

template <bool TILED>
__global__ __launch_bounds__(256) void attn_merge_quant_kernel(const AttnArgs a, int8_t* __restrict__ xq,
                                                               float* __restrict__ xs) {
    __shared__ float red[4];
    const int row = blockIdx.x, tid = threadIdx.x;
    const int D = a.heads * kD, D4 = D >> 2;
    const int kmax = min(a.c1, a.c0 + (row / 64 + 1) * 64);
    const int ns = min(a.nsplit, (kmax + a.split_len - 1) / a.split_len);
    float4 val[kMqGroups];
    float amax = 0.0f;
#pragma unroll
    for (int gi = 0; gi < kMqGroups; ++gi) {
        const int g4 = tid + 256 * gi;
        float4 r = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (g4 < D4) {
            const int h = (4 * g4) / kD, d = (4 * g4) % kD;
            float den = 0.0f;
            float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            if (ns <= kMergeBatch) {
                float ms[kMergeBatch], ls[kMergeBatch];
                float4 os[kMergeBatch];
#pragma unroll
                for (int s = 0; s < kMergeBatch; ++s) {
                    const int sc = s < ns ? s : ns - 1;
                    const size_t pidx = (static_cast<size_t>(sc) * a.heads + h) * a.cs + row;
                    ms[s] = a.part_ml[pidx * 2];
                    ls[s] = a.part_ml[pidx * 2 + 1];
                    os[s] = *reinterpret_cast<const float4*>(a.part_o + pidx * kD + d);
                }
                float M = -INFINITY;
#pragma unroll
                for (int s = 0; s < kMergeBatch; ++s) M = fmaxf(M, ms[s]);
#pragma unroll
                for (int s = 0; s < kMergeBatch; ++s) {
                    const bool use = s < ns && ms[s] != -INFINITY;
                    const float w = __builtin_amdgcn_exp2f((use ? ms[s] : M) - M);
                    const float dl = w * ls[s];
                    den += use ? dl : 0.0f;
                    acc.x += use ? w * os[s].x : 0.0f;
                    acc.y += use ? w * os[s].y : 0.0f;
                    acc.z += use ? w * os[s].z : 0.0f;
                    acc.w += use ? w * os[s].w : 0.0f;
                }
            } else {
                float M = -INFINITY;
                for (int s = 0; s < ns; ++s)
                    M = fmaxf(M, a.part_ml[((static_cast<size_t>(s) * a.heads + h) * a.cs + row) * 2]);
                for (int s = 0; s < ns; ++s) {
                    const size_t pidx = (static_cast<size_t>(s) * a.heads + h) * a.cs + row;
                    const float ms = a.part_ml[pidx * 2];
                    if (ms == -INFINITY) continue;
                    const float w = __builtin_amdgcn_exp2f(ms - M);
                    den += w * a.part_ml[pidx * 2 + 1];
                    const float4 o = *reinterpret_cast<const float4*>(a.part_o + pidx * kD + d);
                    acc.x += w * o.x;
                    acc.y += w * o.y;
                    acc.z += w * o.z;
                    acc.w += w * o.w;
                }
            }
            r = make_float4(acc.x / den, acc.y / den, acc.z / den, acc.w / den);
            amax = fmaxf(amax, fmaxf(fmaxf(fabsf(r.x), fabsf(r.y)), fmaxf(fabsf(r.z), fabsf(r.w))));
        }
        val[gi] = r;
    }
    amax = wave_max_f_full(amax);
    if ((tid & 63) == 0) red[tid >> 6] = amax;
    __syncthreads();
    amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    const float a_scale = amax > 0.0f ? amax / 127.0f : 1.0f;
    const float inv = 1.0f / a_scale;
    const int nst = D / kI8TiledStage;
#pragma unroll
    for (int gi = 0; gi < kMqGroups; ++gi) {
        const int g4 = tid + 256 * gi;
        if (g4 >= D4) continue;
        const float4 r = val[gi];
        const uint32_t word = static_cast<uint32_t>(static_cast<uint8_t>(quant_rule(r.x, a_scale, inv, kQuantDynamic))) |
                              static_cast<uint32_t>(static_cast<uint8_t>(quant_rule(r.y, a_scale, inv, kQuantDynamic))) << 8 |
                              static_cast<uint32_t>(static_cast<uint8_t>(quant_rule(r.z, a_scale, inv, kQuantDynamic))) << 16 |
                              static_cast<uint32_t>(static_cast<uint8_t>(quant_rule(r.w, a_scale, inv, kQuantDynamic))) << 24;
        const size_t off = TILED ? i8_tiled_act_off(row, g4 >> 2, nst) + 4 * (g4 & 3) : static_cast<size_t>(row) * D + 4 * g4;
        *reinterpret_cast<uint32_t*>(xq + off) = word;
    }
    if (tid == 0) xs[row] = a_scale;
}

// Chunk rows [cs][heads*128] (token-major) into a cache's head-major
// reference block: ref[h][c0 + i][:] = chunk[i][h*128 ..]. Thread = one
// float4 of one (row, head), K and V together.
__global__ __launch_bounds__(256) void attn_scatter_kv_kernel(const float* __restrict__ kc,
                                                              const float* __restrict__ vc, int cs, int heads,
                                                              float* __restrict__ ref_k, float* __restrict__ ref_v,
                                                              int cap, int c0) {
    const int idx = blockIdx.x * 256 + threadIdx.x;  // (row, head, float4)
    const int per_row = heads * (kD / 4);
    if (idx >= cs * per_row) return;
    const int i = idx / per_row;
    const int rem = idx - i * per_row;
    const int h = rem / (kD / 4), c = rem - h * (kD / 4);
    const size_t src = static_cast<size_t>(i) * heads * kD + h * kD + 4 * c;
    const size_t dst = (static_cast<size_t>(h) * cap + c0 + i) * kD + 4 * c;
    *reinterpret_cast<v4f*>(ref_k + dst) = *reinterpret_cast<const v4f*>(kc + src);
    *reinterpret_cast<v4f*>(ref_v + dst) = *reinterpret_cast<const v4f*>(vc + src);
}

}  // namespace

hipError_t launch_attn_scatter_kv(hipStream_t s, const float* k_chunk, const float* v_chunk, int cs, int heads,
                                  float* ref_k, float* ref_v, int cap, int c0) {
    if (cs < 1 || heads < 1 || c0 < 0 || c0 + cs > cap) return hipErrorInvalidValue;
    const int n = cs * heads * (kD / 4);
    FOCR_LAUNCH(attn_scatter_kv_kernel, dim3((n + 255) / 256), dim3(256), 0, s, k_chunk, v_chunk, cs, heads, ref_k,
                ref_v, cap, c0);
    return hipGetLastError();
}

size_t attn_partials_bytes(int cs, int heads, int nsplit) {
    return static_cast<size_t>(nsplit) * heads * cs * (kD + 2) * sizeof(float);
}

int attn_pick_splits(int cs, int c1, int heads, int cu_count, int* split_len) {
    // Row tile i (64 rows) needs the tiles of keys [0, min(c1, c0 + 64 (i + 1))):
    // ranges of B tiles give sum over i of ceil(n_i / B) blocks with keys per
    // head, and B is the smallest that keeps those within one residency of
    // the GPU (blocks past a row tile's keys exit at once).
    const int c0 = c1 - cs;
    const int qtiles = (cs + 63) / 64;
    const long long slots = static_cast<long long>(kBlocksPerCu) * (cu_count > 0 ? cu_count : 1);
    int per = 1;  // tiles per range
    for (;; ++per) {
        long long blocks = 0;
        for (int i = 0; i < qtiles; ++i) {
            const int n = (min(c1, c0 + 64 * (i + 1)) + kKT - 1) / kKT;
            blocks += (n + per - 1) / per;
        }
        if (blocks * heads <= slots || static_cast<long long>(per) * kKT >= c1) break;
    }
    const int len = per * kKT;
    *split_len = len;
    return (c1 + len - 1) / len;
}

hipError_t launch_attn_prefill(hipStream_t s, const AttnGeom& gm, const float* q, const float* k, const float* v,
                               float* out, int cs, int c0, int c1, int heads, int head_dim, int nsplit,
                               int split_len, float* part, AttnQuantOut* qo) {
    if (head_dim != kD || cs < 1 || c1 < 1 || c0 < 0 || c0 + cs != c1 || heads < 1 || nsplit < 1 ||
        split_len % kKT != 0 || static_cast<long long>(nsplit) * split_len < c1)
        return hipErrorInvalidValue;
    AttnArgs a{q, k, v, out, nullptr, nullptr, gm.ldq, gm.hq, gm.ldk, gm.hk, gm.ldv, gm.hv, gm.ldo, gm.ho,
               cs, c0, c1, heads, split_len, nsplit, kLog2e / sqrtf(static_cast<float>(head_dim))};
    if (nsplit > 1) {
        a.part_o = part;
        a.part_ml = part + static_cast<size_t>(nsplit) * heads * cs * kD;
    }
    const dim3 grid((cs + 63) / 64, heads, nsplit);
    FOCR_LAUNCH(attn_prefill_kernel, grid, dim3(256), 2 * kKT * kLdsRow * sizeof(float), s, a);
    hipError_t e = hipGetLastError();
    if (qo) qo->done = false;
    if (e != hipSuccess || nsplit == 1) return e;
    const int D = heads * kD;
    if (qo && D % kI8TiledStage == 0 && D <= 4 * 256 * kMqGroups) {
        if (qo->tiled)
            FOCR_LAUNCH(attn_merge_quant_kernel<true>, dim3(cs), dim3(256), 0, s, a, qo->xq, qo->xs);
        else
            FOCR_LAUNCH(attn_merge_quant_kernel<false>, dim3(cs), dim3(256), 0, s, a, qo->xq, qo->xs);
        qo->done = true;
        return hipGetLastError();
    }
    FOCR_LAUNCH(attn_merge_kernel, dim3(cs, heads), dim3(kD), 0, s, a);
    return hipGetLastError();
}

}  // namespace focr
