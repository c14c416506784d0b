// k_rswa.hip — R-SWA ring write and split-K decode attention
// (rswa.rs:451-513 write_decode_step, :894-939 decode_attention_scalar,
// :1320-1367 batched_decode_attention).
//
// Layout in HBM, per stream, head-major f32 (the reference's RingCache
// regions, rswa.rs:112-119): ref K [10][cap][128], ref V, ring K
// [10][128][128], ring V. The valid keys of a stream are
// ref[0..prefill_len) ++ ring[0..ring_len) in physical slot order; no mask.
//
// Attention is flash-decoding: grid (key chunk, head, stream); a block
// scores 64 keys (two 128-dim keys per wave step, 32 lanes x float4 each),
// takes the chunk's max / exp / sum, accumulates p . V with float4 loads and
// writes (m, l, acc[128]); a merge kernel combines the chunks with the
// log-sum-exp rule. HBM-bound: every K and V byte is read once.
#include "focr_internal.hpp"
#include "k_common.hpp"

namespace focr {
namespace {

constexpr int H = kNumHeads;
constexpr int D = kHeadDim;
constexpr int W = kRingWindow;
constexpr int KC = 64;  // keys per chunk
constexpr int kPart = D + 2;

struct Geom {
    float* base;
    size_t stream_floats;
    size_t cap;
    __device__ __forceinline__ float* ref_k(size_t s) const { return base + s * stream_floats; }
    __device__ __forceinline__ float* ref_v(size_t s) const { return ref_k(s) + static_cast<size_t>(H) * cap * D; }
    __device__ __forceinline__ float* ring_k(size_t s) const { return ref_v(s) + static_cast<size_t>(H) * cap * D; }
    __device__ __forceinline__ float* ring_v(size_t s) const { return ring_k(s) + static_cast<size_t>(H) * W * D; }
};

Geom geom_of(const focr_hip_rswa* c) { return Geom{c->base, c->stream_floats(), c->ref_capacity}; }

__global__ __launch_bounds__(D) void rswa_write_kernel(Geom g, size_t s0, RswaStepArgs a,
                                                       const float* __restrict__ k_steps,
                                                       const float* __restrict__ v_steps) {
    const int si = blockIdx.x;
    const int kv = blockIdx.y;
    const int h = blockIdx.z;
    const size_t s = s0 + si;
    const float* src = (kv ? v_steps : k_steps) + (static_cast<size_t>(si) * H + h) * D;
    float* dst = (kv ? g.ring_v(s) : g.ring_k(s)) + (static_cast<size_t>(h) * W + a.slot[si]) * D;
    dst[threadIdx.x] = src[threadIdx.x];
}

__global__ __launch_bounds__(256) void rswa_chunk_kernel(Geom g, size_t s0, RswaStepArgs a,
                                                         const float* __restrict__ q, float scale,
                                                         float* __restrict__ partials,
                                                         int max_chunks) {
    __shared__ float sc[KC];
    __shared__ float4 accs[8][D / 4];
    __shared__ float s_ml[2];
    const int chunk = blockIdx.x;
    const int h = blockIdx.y;
    const int si = blockIdx.z;
    const size_t s = s0 + si;
    const int P = static_cast<int>(a.prefill_len[si]);
    const int N = P + static_cast<int>(a.ring_len[si]);
    if (chunk * KC >= N) return;
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int half = lane >> 5;
    const int dl = lane & 31;
    const float* qh = q + (static_cast<size_t>(si) * H + h) * D;
    const float4 qv = reinterpret_cast<const float4*>(qh)[dl];
    const float* rk = g.ref_k(s) + static_cast<size_t>(h) * g.cap * D;
    const float* rv = g.ref_v(s) + static_cast<size_t>(h) * g.cap * D;
    const float* gk = g.ring_k(s) + static_cast<size_t>(h) * W * D;
    const float* gv = g.ring_v(s) + static_cast<size_t>(h) * W * D;

    // scores: wave w covers keys [w*16, w*16+16), two keys per step; all
    // eight K-row loads of a lane are in flight before the first dot
    float4 kv[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int key = chunk * KC + wave * 16 + 2 * i + half;
        const float* kr = key < P ? rk + static_cast<size_t>(key) * D : gk + static_cast<size_t>(key - P) * D;
        kv[i] = key < N ? reinterpret_cast<const float4*>(kr)[dl] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int j = wave * 16 + 2 * i + half;
        const int key = chunk * KC + j;
        // the 32-lane dot: 16-lane row sums by DPP, then the two rows of each
        // half wave read back as scalars (every lane is active here)
        const float d16 = row16_sum_f(qv.x * kv[i].x + qv.y * kv[i].y + qv.z * kv[i].z + qv.w * kv[i].w);
        const float d = half ? lane_f(d16, 32) + lane_f(d16, 48) : lane_f(d16, 0) + lane_f(d16, 16);
        if (dl == 0) sc[j] = key < N ? d * scale : -INFINITY;
    }
    // p . V: 8 key groups x 32 lanes (float4 of the head dim each); the V
    // loads do not depend on the softmax, so issue them before the barrier
    const int grp = threadIdx.x >> 5;
    const int dq = threadIdx.x & 31;
    float4 vv[KC / 8];
#pragma unroll
    for (int i = 0; i < KC / 8; ++i) {
        const int key = chunk * KC + grp + 8 * i;
        const float* vr = key < P ? rv + static_cast<size_t>(key) * D : gv + static_cast<size_t>(key - P) * D;
        vv[i] = key < N ? reinterpret_cast<const float4*>(vr)[dq] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
    __syncthreads();
    if (wave == 0) {
        const float v = sc[lane];
        const float m = wave_max_f_full(v);
        const float p = v == -INFINITY ? 0.0f : expf(v - m);
        const float l = wave_sum_f_full(p);
        sc[lane] = p;
        if (lane == 0) {
            s_ml[0] = m;
            s_ml[1] = l;
        }
    }
    __syncthreads();
    float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
    for (int i = 0; i < KC / 8; ++i) {
        const float p = sc[grp + 8 * i];
        acc.x += p * vv[i].x;
        acc.y += p * vv[i].y;
        acc.z += p * vv[i].z;
        acc.w += p * vv[i].w;
    }
    accs[grp][dq] = acc;
    __syncthreads();
    float* part = partials + ((static_cast<size_t>(si) * H + h) * max_chunks + chunk) * kPart;
    if (threadIdx.x < D) {
        const int d4 = threadIdx.x >> 2, c = threadIdx.x & 3;
        float sum = 0.0f;
#pragma unroll
        for (int gI = 0; gI < 8; ++gI) {
            const float4 v = accs[gI][d4];
            sum += c == 0 ? v.x : c == 1 ? v.y : c == 2 ? v.z : v.w;
        }
        part[2 + threadIdx.x] = sum;
    }
    if (threadIdx.x == 0) {
        part[0] = s_ml[0];
        part[1] = s_ml[1];
    }
}

// Log-sum-exp merge of a (stream, head)'s chunk partials: M = max m_c,
// f_c = exp(m_c - M) computed once per chunk, then every head-dim lane sums
// independent loads acc_c[d] * f_c.
__global__ __launch_bounds__(D) void rswa_merge_kernel(RswaStepArgs a, const float* __restrict__ partials,
                                                       int max_chunks, float* __restrict__ out) {
    __shared__ float s_f[1024];
    __shared__ float s_red[D / 64][2];
    const int h = blockIdx.x;
    const int si = blockIdx.y;
    const int N = static_cast<int>(a.prefill_len[si] + a.ring_len[si]);
    const int nch = (N + KC - 1) / KC;
    const float* base = partials + (static_cast<size_t>(si) * H + h) * max_chunks * kPart;
    float m = -INFINITY;
    for (int c = threadIdx.x; c < nch; c += D) m = fmaxf(m, base[c * kPart]);
    m = wave_max_f_full(m);
    if ((threadIdx.x & 63) == 0) s_red[threadIdx.x >> 6][0] = m;
    __syncthreads();
    const float M = fmaxf(s_red[0][0], s_red[1][0]);
    float acc = 0.0f, L = 0.0f;
    for (int c0 = 0; c0 < nch; c0 += 1024) {
        const int cn = min(1024, nch - c0);
        __syncthreads();
        for (int c = threadIdx.x; c < cn; c += D) s_f[c] = expf(base[(c0 + c) * kPart] - M);
        __syncthreads();
        int c = 0;
        for (; c + 4 <= cn; c += 4) {
            const float a0 = base[(c0 + c) * kPart + 2 + threadIdx.x];
            const float a1 = base[(c0 + c + 1) * kPart + 2 + threadIdx.x];
            const float a2 = base[(c0 + c + 2) * kPart + 2 + threadIdx.x];
            const float a3 = base[(c0 + c + 3) * kPart + 2 + threadIdx.x];
            const float l0 = base[(c0 + c) * kPart + 1];
            const float l1 = base[(c0 + c + 1) * kPart + 1];
            const float l2 = base[(c0 + c + 2) * kPart + 1];
            const float l3 = base[(c0 + c + 3) * kPart + 1];
            acc += a0 * s_f[c];
            acc += a1 * s_f[c + 1];
            acc += a2 * s_f[c + 2];
            acc += a3 * s_f[c + 3];
            L += l0 * s_f[c];
            L += l1 * s_f[c + 1];
            L += l2 * s_f[c + 2];
            L += l3 * s_f[c + 3];
        }
        for (; c < cn; ++c) {
            acc += base[(c0 + c) * kPart + 2 + threadIdx.x] * s_f[c];
            L += base[(c0 + c) * kPart + 1] * s_f[c];
        }
    }
    const float inv = L > 0.0f ? 1.0f / L : 0.0f;
    out[(static_cast<size_t>(si) * H + h) * D + threadIdx.x] = acc * inv;
}

}  // namespace

size_t rswa_partials_bytes(size_t n_streams, size_t max_keys) {
    const size_t max_chunks = (max_keys + KC - 1) / KC;
    return n_streams * H * max_chunks * kPart * sizeof(float);
}

hipError_t launch_rswa_write(hipStream_t s, const focr_hip_rswa* c, size_t s0,
                             const RswaStepArgs& a, const float* k_steps, const float* v_steps) {
    if (a.n == 0) return hipSuccess;
    FOCR_LAUNCH(rswa_write_kernel, dim3(a.n, 2, H), dim3(D), 0, s, geom_of(c), s0, a,
                       k_steps, v_steps);
    return hipGetLastError();
}

hipError_t launch_rswa_attention(hipStream_t s, const focr_hip_rswa* c, size_t s0,
                                 const RswaStepArgs& a, const float* q, float* out,
                                 float* partials, int, focr_hip_ctx* ctx) {
    if (a.n == 0) return hipSuccess;
    const int max_chunks = static_cast<int>((c->ref_capacity + W + KC - 1) / KC);
    const float scale = 1.0f / sqrtf(static_cast<float>(D));  // rswa.rs:52-55
    {
        ProfScope ps(ctx, "rswa_chunk");
        FOCR_LAUNCH(rswa_chunk_kernel, dim3(max_chunks, H, a.n), dim3(256), 0, s, geom_of(c),
                           s0, a, q, scale, partials, max_chunks);
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    {
        ProfScope ps(ctx, "rswa_merge");
        FOCR_LAUNCH(rswa_merge_kernel, dim3(H, a.n), dim3(D), 0, s, a, partials, max_chunks, out);
    }
    return hipGetLastError();
}

}  // namespace focr
