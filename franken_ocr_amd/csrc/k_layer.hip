// k_layer.hip — the decode layer's small ops around the GEMVs, attention and
// MoE kernels (decode_step_with_cache_i8, decoder.rs:2542-2627; batched form
// batched_decode_step_i8_streams, :2812-2933):
//
//   * RMSNorm of each row (nn::rms_norm, nn.rs:240-253), either fused with
//     quantize_row_i8 of the normed row for the qkv GEMV (the reference's
//     FOCR_FUSE_NORM_QUANT form, byte-identical to norm-then-quantize,
//     decoder.rs:1680-1706), or fused with the residual add before it
//     (add_residual, decoder.rs:529-546, then the post-attention norm);
//   * RoPE of q and k at each stream's own position (RopeTable::build +
//     apply_rope, decoder.rs:150-268), splitting the fused qkv row into the
//     contiguous q / k / v rows the ring write and attention take;
//   * a row-wise add (the dense MLP's residual).
//
// RMSNorm arithmetic (ft-kernel-cpu's rms_norm_forward_f32 is not in the
// reference tree, so this build fixes it): the sum of squares in f64,
// rstd = (float)(1 / sqrt(ss / n + eps)) in f64, y = (x * rstd) * w in f32.
#include "focr_internal.hpp"
#include "k_common.hpp"

namespace focr {
namespace {

constexpr int kThreads = 256;

// Sum of (double)v^2 over a row by the whole block; every thread gets it.
__device__ __forceinline__ double block_sum_sq(const float* __restrict__ r, int n, double* red) {
    double ss = 0.0;
    for (int i = threadIdx.x; i < n; i += kThreads) {
        const double v = static_cast<double>(r[i]);
        ss = fma(v, v, ss);
    }
    ss = wave_sum_d_full(ss);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
    __syncthreads();
    double t = 0.0;
#pragma unroll
    for (int w = 0; w < kThreads / 64; ++w) t += red[w];
    return t;
}

// MODE 0: y = rms_norm(x) * w, then quantize_row_i8 (half away) -> xq, xs.
// MODE 1: h = x + a (written), y = rms_norm(h) * w (written, f32).
// MODE 2: y = rms_norm(x) * w (f32; w null: no weight).
// One block per row; n <= 4096 (the row is staged in LDS).
template <int MODE>
__global__ __launch_bounds__(kThreads) void rms_norm_rows_kernel(const float* __restrict__ x,
                                                                 const float* __restrict__ a,
                                                                 const float* __restrict__ w, int n, float eps,
                                                                 float* __restrict__ h, float* __restrict__ y,
                                                                 int8_t* __restrict__ xq, float* __restrict__ xs) {
    __shared__ float s_row[4096];
    __shared__ double s_red[kThreads / 64];
    __shared__ float s_max[kThreads / 64];
    const size_t base = static_cast<size_t>(blockIdx.x) * n;
    for (int i = threadIdx.x; i < n; i += kThreads) {
        float v = x[base + i];
        if (MODE == 1) {
            v = v + a[base + i];
            h[base + i] = v;
        }
        s_row[i] = v;
    }
    __syncthreads();
    const double ss = block_sum_sq(s_row, n, s_red);
    const float rstd = static_cast<float>(1.0 / sqrt(ss / static_cast<double>(n) + static_cast<double>(eps)));
    if (MODE == 1) {
        for (int i = threadIdx.x; i < n; i += kThreads) y[base + i] = (s_row[i] * rstd) * w[i];
        return;
    }
    if (MODE == 2) {
        for (int i = threadIdx.x; i < n; i += kThreads) {
            const float v = s_row[i] * rstd;
            y[base + i] = w ? v * w[i] : v;
        }
        return;
    }
    float amax = 0.0f;
    for (int i = threadIdx.x; i < n; i += kThreads) {
        const float v = (s_row[i] * rstd) * w[i];
        s_row[i] = v;  // each thread rewrites only its own elements
        amax = fmaxf(amax, fabsf(v));
    }
    amax = wave_max_f_full(amax);
    if ((threadIdx.x & 63) == 0) s_max[threadIdx.x >> 6] = amax;
    __syncthreads();
    amax = s_max[0];
#pragma unroll
    for (int wv = 1; wv < kThreads / 64; ++wv) amax = fmaxf(amax, s_max[wv]);
    const float a_scale = amax > 0.0f ? amax / 127.0f : 1.0f;
    const float inv = 1.0f / a_scale;
    for (int i = threadIdx.x; i < n; i += kThreads) xq[base + i] = quant_i8(s_row[i], inv, false);
    if (threadIdx.x == 0) xs[blockIdx.x] = a_scale;
}

// The same three modes with the row held in registers: thread t takes
// float4 chunks t + 256 j (j < NC; n % 4 == 0, 1024 NC >= n, 16-byte aligned
// rows), every load issued before the first use (the strided loops above wait
// for each load in turn). Sum of squares: per thread over its chunks, the
// wave by DPP, the four waves in order (f64 throughout, another order than
// the loop above: rstd, rounded to f32, can differ in the last bit only when
// the f64 value sits on an f32 rounding boundary).
template <int MODE, int NC>
__global__ __launch_bounds__(kThreads) void rms_norm_rows_vec_kernel(const float* __restrict__ x,
                                                                     const float* __restrict__ a,
                                                                     const float* __restrict__ w, int n, float eps,
                                                                     float* __restrict__ h, float* __restrict__ y,
                                                                     int8_t* __restrict__ xq, float* __restrict__ xs) {
    __shared__ double s_red[kThreads / 64];
    __shared__ float s_max[kThreads / 64];
    const size_t base = static_cast<size_t>(blockIdx.x) * n;
    const int n4 = n >> 2;
    const float4* x4 = reinterpret_cast<const float4*>(x + base);
    const float4* a4 = MODE == 1 ? reinterpret_cast<const float4*>(a + base) : nullptr;
    const float4* w4 = reinterpret_cast<const float4*>(w);
    float4 v[NC], g[NC];
#pragma unroll
    for (int j = 0; j < NC; ++j) {
        const int c = static_cast<int>(threadIdx.x) + kThreads * j;
        const int cc = c < n4 ? c : n4 - 1;  // past the row: its last chunk again (unused)
        v[j] = x4[cc];
        if (MODE == 1) {
            const float4 b = a4[cc];
            v[j] = make_float4(v[j].x + b.x, v[j].y + b.y, v[j].z + b.z, v[j].w + b.w);
        }
        g[j] = w ? w4[cc] : make_float4(1.f, 1.f, 1.f, 1.f);
    }
    double ss = 0.0;
#pragma unroll
    for (int j = 0; j < NC; ++j) {
        if (static_cast<int>(threadIdx.x) + kThreads * j < n4) {
            ss = fma(static_cast<double>(v[j].x), static_cast<double>(v[j].x), ss);
            ss = fma(static_cast<double>(v[j].y), static_cast<double>(v[j].y), ss);
            ss = fma(static_cast<double>(v[j].z), static_cast<double>(v[j].z), ss);
            ss = fma(static_cast<double>(v[j].w), static_cast<double>(v[j].w), ss);
        }
    }
    ss = wave_sum_d_full(ss);
    if ((threadIdx.x & 63) == 0) s_red[threadIdx.x >> 6] = ss;
    __syncthreads();
    double tot = 0.0;
#pragma unroll
    for (int wv = 0; wv < kThreads / 64; ++wv) tot += s_red[wv];
    const float rstd = static_cast<float>(1.0 / sqrt(tot / static_cast<double>(n) + static_cast<double>(eps)));
    float amax = 0.0f;
#pragma unroll
    for (int j = 0; j < NC; ++j) {
        const int c = static_cast<int>(threadIdx.x) + kThreads * j;
        if (c >= n4) continue;
        const float4 t = v[j];
        float4 o = make_float4(t.x * rstd, t.y * rstd, t.z * rstd, t.w * rstd);
        if (MODE != 2 || w) o = make_float4(o.x * g[j].x, o.y * g[j].y, o.z * g[j].z, o.w * g[j].w);
        if (MODE == 1) reinterpret_cast<float4*>(h + base)[c] = t;
        if (MODE != 0) {
            reinterpret_cast<float4*>(y + base)[c] = o;
        } else {
            v[j] = o;
            amax = fmaxf(amax, fmaxf(fmaxf(fabsf(o.x), fabsf(o.y)), fmaxf(fabsf(o.z), fabsf(o.w))));
        }
    }
    if (MODE != 0) return;
    amax = wave_max_f_full(amax);
    if ((threadIdx.x & 63) == 0) s_max[threadIdx.x >> 6] = amax;
    __syncthreads();
    amax = s_max[0];
#pragma unroll
    for (int wv = 1; wv < kThreads / 64; ++wv) amax = fmaxf(amax, s_max[wv]);
    const float a_scale = amax > 0.0f ? amax / 127.0f : 1.0f;
    const float inv = 1.0f / a_scale;
#pragma unroll
    for (int j = 0; j < NC; ++j) {
        const int c = static_cast<int>(threadIdx.x) + kThreads * j;
        if (c >= n4) continue;
        char4 q;
        q.x = quant_i8(v[j].x, inv, false);
        q.y = quant_i8(v[j].y, inv, false);
        q.z = quant_i8(v[j].z, inv, false);
        q.w = quant_i8(v[j].w, inv, false);
        reinterpret_cast<char4*>(xq + base)[c] = q;
    }
    if (threadIdx.x == 0) xs[blockIdx.x] = a_scale;
}

// Launch MODE over rows: the register form where the shape and alignment
// allow, else the staged-row kernel.
template <int MODE>
hipError_t launch_rms_norm_mode(hipStream_t s, const float* x, const float* a, const float* w, int rows, int n,
                                float eps, float* h, float* y, int8_t* xq, float* xs) {
    auto al16 = [](const void* p) { return p == nullptr || reinterpret_cast<uintptr_t>(p) % 16 == 0; };
    const bool vec = n % 4 == 0 && n <= 4 * 4 * kThreads && al16(x) && al16(a) && al16(w) && al16(h) && al16(y) &&
                     (xq == nullptr || reinterpret_cast<uintptr_t>(xq) % 4 == 0);
    if (vec && n <= 2 * 4 * kThreads)
        FOCR_LAUNCH((rms_norm_rows_vec_kernel<MODE, 2>), dim3(rows), dim3(kThreads), 0, s, x, a, w, n, eps, h, y, xq,
                    xs);
    else if (vec)
        FOCR_LAUNCH((rms_norm_rows_vec_kernel<MODE, 4>), dim3(rows), dim3(kThreads), 0, s, x, a, w, n, eps, h, y, xq,
                    xs);
    else
        FOCR_LAUNCH(rms_norm_rows_kernel<MODE>, dim3(rows), dim3(kThreads), 0, s, x, a, w, n, eps, h, y, xq, xs);
    return hipGetLastError();
}

// One block per stream: the fused row qkv [3D] -> q, k rotated at
// pos.p[s] (inv_freq [half], the reference's f64-then-f32 table) and v
// copied: q [D] contiguous; k and v [D] contiguous, or (ring.k[0] set)
// straight into the stream's R-SWA ring slot — the ring write
// (rswa.rs:451-466) fused in. Thread = (head, i < half) pairs. The positions
// and slots ride in the kernel arguments (no copy per step).
__global__ __launch_bounds__(kThreads) void rope_split_kernel(const float* __restrict__ qkv, RopePositions pos,
                                                              const float* __restrict__ inv_freq, int n_heads,
                                                              int head_dim, float* __restrict__ q,
                                                              float* __restrict__ k, float* __restrict__ v,
                                                              RopeRing ring) {
    const int s = blockIdx.x;
    const int D = n_heads * head_dim;
    const int half = head_dim >> 1;
    const float* row = qkv + static_cast<size_t>(s) * 3 * D;
    const float p = static_cast<float>(pos.p[s]);
    for (int t = threadIdx.x; t < n_heads * half; t += kThreads) {
        const int hd = t / half, i = t - hd * half;
        const float angle = p * inv_freq[i];
        float sn, cs;
        sincosf(angle, &sn, &cs);
        const int j0 = hd * head_dim + i, j1 = j0 + half;
        const float qa = row[j0], qb = row[j1];
        const float ka = row[D + j0], kb = row[D + j1];
        q[static_cast<size_t>(s) * D + j0] = qa * cs - qb * sn;
        q[static_cast<size_t>(s) * D + j1] = qb * cs + qa * sn;
        float* kr = ring.k[0] ? ring.k[s] + static_cast<size_t>(hd) * ring.head_stride
                              : k + static_cast<size_t>(s) * D + static_cast<size_t>(hd) * head_dim;
        kr[i] = ka * cs - kb * sn;
        kr[i + half] = kb * cs + ka * sn;
    }
    for (int j = threadIdx.x; j < D; j += kThreads) {
        const int hd = j / head_dim, i = j - hd * head_dim;
        float* vr = ring.v[0] ? ring.v[s] + static_cast<size_t>(hd) * ring.head_stride
                              : v + static_cast<size_t>(s) * D + static_cast<size_t>(hd) * head_dim;
        vr[i] = row[2 * D + j];
    }
}

// Chunked prefill (decoder.rs:2470-2482): fused qkv rows [rows][3 D] of
// the positions c0 .. c0 + rows split into q, k (RoPE at the row's position,
// RopeTable::build + apply_rope, decoder.rs:170-268: the same expressions as
// rope_split_kernel) and v. q is token-major [rows][D]; k and v element
// (row r, head h, dim d) go to kv.k / kv.v + r * row_stride + h * head_stride
// + d: token-major, or the stream's head-major reference block at c0 (the
// attention's K / V, so no separate copy). One block per row: the row's
// head_dim / 2 sin / cos pairs once (the angle p * inv_freq[i] is the same
// for every head and for q and k), then the rotations four pairs per thread.
struct RopeKv {
    float* k;
    float* v;
    size_t row_stride, head_stride;
};
constexpr int kRopeMaxHalf = 256;

__global__ __launch_bounds__(kThreads) void rope_rows_kernel(const float* __restrict__ qkv, int c0,
                                                             const float* __restrict__ inv_freq, int n_heads,
                                                             int head_dim, float* __restrict__ q, const RopeKv kv) {
    __shared__ float s_sn[kRopeMaxHalf], s_cs[kRopeMaxHalf];
    const int r = blockIdx.x;
    const int D = n_heads * head_dim;
    const int half = head_dim >> 1;
    const float* row = qkv + static_cast<size_t>(r) * 3 * D;
    const float p = static_cast<float>(c0 + r);
    for (int i = threadIdx.x; i < half; i += kThreads) {
        const float angle = p * inv_freq[i];
        float sn, cs;
        sincosf(angle, &sn, &cs);
        s_sn[i] = sn;
        s_cs[i] = cs;
    }
    __syncthreads();
    float* qr = q + static_cast<size_t>(r) * D;
    float* kr = kv.k + static_cast<size_t>(r) * kv.row_stride;
    float* vr = kv.v + static_cast<size_t>(r) * kv.row_stride;
    const int q4 = half >> 2;  // groups of four pairs per head
    for (int t = threadIdx.x; t < n_heads * q4; t += kThreads) {
        const int hd = t / q4, i = 4 * (t - hd * q4);
        const int j0 = hd * head_dim + i, j1 = j0 + half;
        const float4 qa = *reinterpret_cast<const float4*>(row + j0), qb = *reinterpret_cast<const float4*>(row + j1);
        const float4 ka = *reinterpret_cast<const float4*>(row + D + j0);
        const float4 kb = *reinterpret_cast<const float4*>(row + D + j1);
        const float4 sn = *reinterpret_cast<const float4*>(s_sn + i), cs = *reinterpret_cast<const float4*>(s_cs + i);
        const size_t o0 = hd * kv.head_stride + i, o1 = o0 + half;
        *reinterpret_cast<float4*>(qr + j0) = make_float4(qa.x * cs.x - qb.x * sn.x, qa.y * cs.y - qb.y * sn.y,
                                                          qa.z * cs.z - qb.z * sn.z, qa.w * cs.w - qb.w * sn.w);
        *reinterpret_cast<float4*>(qr + j1) = make_float4(qb.x * cs.x + qa.x * sn.x, qb.y * cs.y + qa.y * sn.y,
                                                          qb.z * cs.z + qa.z * sn.z, qb.w * cs.w + qa.w * sn.w);
        *reinterpret_cast<float4*>(kr + o0) = make_float4(ka.x * cs.x - kb.x * sn.x, ka.y * cs.y - kb.y * sn.y,
                                                          ka.z * cs.z - kb.z * sn.z, ka.w * cs.w - kb.w * sn.w);
        *reinterpret_cast<float4*>(kr + o1) = make_float4(kb.x * cs.x + ka.x * sn.x, kb.y * cs.y + ka.y * sn.y,
                                                          kb.z * cs.z + ka.z * sn.z, kb.w * cs.w + ka.w * sn.w);
    }
    const int d4 = head_dim >> 2;
    for (int f = threadIdx.x; f < n_heads * d4; f += kThreads) {
        const int hd = f / d4, d = 4 * (f - hd * d4);
        *reinterpret_cast<float4*>(vr + hd * kv.head_stride + d) =
            *reinterpret_cast<const float4*>(row + 2 * D + hd * head_dim + d);
    }
}

// act = silu(g) * u (decoder.rs:1746-1752), the dense MLP's SwiGLU.
__global__ __launch_bounds__(kThreads) void silu_mul_kernel(const float* __restrict__ g, const float* __restrict__ u,
                                                            float* __restrict__ act, size_t n) {
    const size_t i = static_cast<size_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (i < n) act[i] = silu_f(g[i]) * u[i];
}

__global__ __launch_bounds__(kThreads) void add_rows_kernel(const float* __restrict__ a, const float* __restrict__ b,
                                                            float* __restrict__ out, size_t n) {
    const size_t i = static_cast<size_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (i < n) out[i] = a[i] + b[i];
}

}  // namespace

hipError_t launch_rms_norm_quant(hipStream_t s, const float* x, const float* w, int rows, int n, float eps,
                                 int8_t* xq, float* xs) {
    if (n > 4096 || rows < 1) return hipErrorInvalidValue;
    return launch_rms_norm_mode<0>(s, x, nullptr, w, rows, n, eps, nullptr, nullptr, xq, xs);
}

hipError_t launch_residual_rms_norm(hipStream_t s, const float* x, const float* a, const float* w, int rows, int n,
                                    float eps, float* h, float* y) {
    if (n > 4096 || rows < 1) return hipErrorInvalidValue;
    return launch_rms_norm_mode<1>(s, x, a, w, rows, n, eps, h, y, nullptr, nullptr);
}

hipError_t launch_rms_norm(hipStream_t s, const float* x, const float* w, int rows, int n, float eps, float* y) {
    if (n > 4096 || rows < 1) return hipErrorInvalidValue;
    return launch_rms_norm_mode<2>(s, x, nullptr, w, rows, n, eps, nullptr, y, nullptr, nullptr);
}

hipError_t launch_rope_split(hipStream_t s, const float* qkv, const RopePositions& pos, const float* inv_freq,
                             int streams, int n_heads, int head_dim, float* q, float* k, float* v,
                             const RopeRing* ring) {
    if (head_dim % 2 || streams < 1 || streams > RopePositions::kMax) return hipErrorInvalidValue;
    RopeRing r{};
    if (ring) {
        for (int i = 0; i < streams; ++i)
            if (!ring->k[i] || !ring->v[i]) return hipErrorInvalidValue;
        r = *ring;
    } else if (!k || !v) {
        return hipErrorInvalidValue;
    }
    FOCR_LAUNCH(rope_split_kernel, dim3(streams), dim3(kThreads), 0, s, qkv, pos, inv_freq, n_heads, head_dim, q, k,
                v, r);
    return hipGetLastError();
}

hipError_t launch_rope_rows(hipStream_t s, const float* qkv, int rows, int c0, const float* inv_freq, int n_heads,
                            int head_dim, float* q, float* k, float* v, size_t kv_row_stride,
                            size_t kv_head_stride) {
    // float4 rotations: head_dim a multiple of 8 (four pairs per thread), the
    // row and head strides multiples of 4 floats (16-byte aligned stores)
    if (rows < 1 || c0 < 0 || n_heads < 1 || head_dim < 8 || head_dim % 8 || head_dim / 2 > kRopeMaxHalf || !qkv ||
        !inv_freq || !q || !k || !v || kv_row_stride % 4 || kv_head_stride % 4)
        return hipErrorInvalidValue;
    FOCR_LAUNCH(rope_rows_kernel, dim3(static_cast<unsigned>(rows)), dim3(kThreads), 0, s, qkv, c0, inv_freq,
                n_heads, head_dim, q, RopeKv{k, v, kv_row_stride, kv_head_stride});
    return hipGetLastError();
}

hipError_t launch_silu_mul(hipStream_t s, const float* g, const float* u, float* act, size_t n) {
    FOCR_LAUNCH(silu_mul_kernel, dim3(static_cast<unsigned>((n + kThreads - 1) / kThreads)), dim3(kThreads), 0, s, g,
                u, act, n);
    return hipGetLastError();
}

hipError_t launch_add_rows(hipStream_t s, const float* a, const float* b, float* out, size_t n) {
    FOCR_LAUNCH(add_rows_kernel, dim3(static_cast<unsigned>((n + kThreads - 1) / kThreads)), dim3(kThreads), 0, s, a,
                b, out, n);
    return hipGetLastError();
}

}  // namespace focr
