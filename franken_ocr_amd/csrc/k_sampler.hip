// k_sampler.hip — the greedy decode sampler on the device.
//
// sampler.rs:191-235 for_each_sliding_window_ngram_ban is a pure function of
// a stream's generated sequence, so it runs before the LM-head GEMV and
// leaves a ban bitmap (one bit per vocab id) per stream; the GEMV epilogue
// (or the argmax over given logits) reads the bit and treats a banned id as
// -inf, which is byte-for-byte the reference's masked copy followed by
// argmax_row (sampler.rs:168-186, :245-257, :346-395; decoder.rs:2319-2357).
// The finish kernel folds the per-block argmax keys into the token, flags
// EOS (sampler.rs:143-150) and appends the token to the device-resident
// history, so a decode loop needs no host round trip per token.
#include "focr_internal.hpp"
#include "k_common.hpp"

namespace focr {
namespace {

constexpr int kThreads = 256;

__global__ __launch_bounds__(kThreads) void sampler_prep_kernel(const float* __restrict__ x, int K,
                                                                int8_t* __restrict__ xq, float* __restrict__ xs,
                                                                SamplerArgs a) {
    __shared__ float red[kThreads / 64];
    const int r = blockIdx.x;
    if (x) {
        const float* xr = x + static_cast<size_t>(r) * K;
        int8_t* qr = xq + static_cast<size_t>(r) * K;
        // the row in registers (all loads in flight at once) where it fits
        const bool vec = K % 4 == 0 && reinterpret_cast<uintptr_t>(xr) % 16 == 0 &&
                         reinterpret_cast<uintptr_t>(qr) % 4 == 0;  // uniform
        if (vec && K <= 2 * 4 * kThreads)
            block_quantize_row_vec<kThreads, 2>(xr, K, qr, xs + r, false, red);
        else if (vec && K <= 8 * 4 * kThreads)
            block_quantize_row_vec<kThreads, 8>(xr, K, qr, xs + r, false, red);
        else
            block_quantize_row<kThreads>(xr, K, qr, xs + r, false, red);
    }

    uint32_t* bits = a.ban_bits + static_cast<size_t>(r) * a.ban_words;
    for (int w = threadIdx.x; w < a.ban_words; w += kThreads) bits[w] = 0u;
    const uint32_t raw_len = a.history_len ? a.history_len[r] : 0u;
    if (threadIdx.x == 0) a.err[r] = raw_len > static_cast<uint32_t>(a.cap) ? 1 : 0;
    __syncthreads();  // the bitmap is clear before any bit is set

    const int L = raw_len > static_cast<uint32_t>(a.cap) ? a.cap : static_cast<int>(raw_len);
    const int n = a.ngram;
    if (n <= 0 || L < n) return;
    const int start = a.window == 0 ? 0 : (L > a.window ? L - a.window : 0);
    const int end = L - n + 1;  // >= 1
    if (end <= start) return;
    const uint32_t* seq = a.history + static_cast<size_t>(r) * a.cap;
    const uint32_t* prefix = seq + (L - (n - 1));  // the last n-1 tokens
    for (int idx = start + static_cast<int>(threadIdx.x); idx < end; idx += kThreads) {
        bool match = true;
        for (int j = 0; j < n - 1; ++j)
            if (seq[idx + j] != prefix[j]) {
                match = false;
                break;
            }
        if (!match) continue;
        const uint32_t banned = seq[idx + n - 1];
        bool white = false;
        for (int j = 0; j < a.n_white; ++j) white |= a.whitelist[j] == banned;
        if (white || banned >= static_cast<uint32_t>(a.vocab)) continue;
        atomicOr(bits + (banned >> 5), 1u << (banned & 31));
    }
}

__global__ __launch_bounds__(kThreads) void sample_finish_kernel(const uint64_t* __restrict__ keys, int nparts,
                                                                 uint32_t eos, uint32_t* __restrict__ tokens,
                                                                 uint8_t* __restrict__ is_eos, SamplerArgs a) {
    __shared__ uint64_t red[kThreads / 64];
    const int r = blockIdx.x;
    uint64_t b = thread_max_keys<kThreads>(keys + static_cast<size_t>(r) * nparts, nparts);
    b = wave_max_u64_full(b);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = b;
    __syncthreads();
    if (threadIdx.x != 0) return;
    uint64_t best = red[0];
#pragma unroll
    for (int i = 1; i < kThreads / 64; ++i) best = red[i] > best ? red[i] : best;
    const uint32_t tok = argmax_key_index(best);
    tokens[r] = tok;
    if (is_eos) is_eos[r] = tok == eos ? 1 : 0;
    if (a.history_mut) {
        const uint32_t L = a.history_len[r];
        if (L < static_cast<uint32_t>(a.cap)) {
            a.history_mut[static_cast<size_t>(r) * a.cap + L] = tok;
            a.history_len[r] = L + 1;
        } else {
            a.err[r] |= 2;
        }
    }
}

}  // namespace

hipError_t launch_sampler_prep(hipStream_t s, int m, const float* x, int k, int8_t* xq, float* xs,
                               const SamplerArgs& a) {
    if (m <= 0) return hipSuccess;
    FOCR_LAUNCH(sampler_prep_kernel, dim3(m), dim3(kThreads), 0, s, x, k, xq, xs, a);
    return hipGetLastError();
}

hipError_t launch_sample_finish(hipStream_t s, int m, const uint64_t* keys, int nparts, uint32_t eos,
                                uint32_t* tokens, uint8_t* is_eos, const SamplerArgs& a) {
    if (m <= 0) return hipSuccess;
    FOCR_LAUNCH(sample_finish_kernel, dim3(m), dim3(kThreads), 0, s, keys, nparts, eos, tokens, is_eos, a);
    return hipGetLastError();
}

}  // namespace focr
