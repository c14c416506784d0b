// focr_engine.cpp — C ABI, layer 2: the runtime self-test, uploaded weights
// and the device-resident engine ops (GEMV, LM head + argmax, MoE decode,
// R-SWA), plus the GPU-timed profiling counters.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <limits>
#include <memory>
#include <new>
#include <string>
#include <vector>

#include "focr_internal.hpp"

using namespace focr;

namespace {

std::string fmt(const char* f, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, f);
    vsnprintf(buf, sizeof(buf), f, ap);
    va_end(ap);
    return buf;
}

struct Guard {
    std::lock_guard<std::mutex> lk;
    explicit Guard(focr_hip_ctx* c) : lk(c->mu) { clear_error(); }
};

#define ENGINE_CTX(ctx)                                                   \
    if (!(ctx)) return fail(FOCR_HIP_E_BAD_HANDLE, "null focr_hip_ctx"); \
    Guard guard_(ctx);                                                    \
    FOCR_HIP_TRY((ctx)->bind(), "hipSetDevice")

// dispatch.rs:340-347 xs32
uint32_t xs32(uint32_t& s) {
    s ^= s << 13;
    s ^= s >> 17;
    s ^= s << 5;
    return s;
}

struct Shape {
    const char* label;
    size_t m, k, n;
    uint32_t seed;
};

// dispatch.rs:352-368 SELFTEST_SHAPES
const Shape kShapes[] = {
    {"edge:1x1x1", 1, 1, 1, 0x11111111u},
    {"edge:1x7x3", 1, 7, 3, 0x22222222u},
    {"edge:2x3x2", 2, 3, 2, 0x33333333u},
    {"ktail:1x15x8", 1, 15, 8, 0x44444444u},
    {"ktail:1x16x8", 1, 16, 8, 0x55555555u},
    {"ktail:1x17x8", 1, 17, 8, 0x66666666u},
    {"ktail:4x33x5", 4, 33, 5, 0x77777777u},
    {"model:attn_proj_gemv", 1, 1280, 128, 0x0badc0deu},
    {"model:o_proj_gemv", 1, 1280, 1280, 0x12345678u},
    {"model:expert_down_gemv", 1, 6848, 256, 0x9abcdef0u},
    {"model:prefill_tile", 4, 1280, 64, 0x0f0f0f0fu},
    {"overflow:max_mag_k6848", 1, 6848, 4, 0u},
};

// The self-test's in-process check: a plain i32 dot, as scalar.rs:103-115.
template <typename TA>
void scalar_check(const TA* a, const int8_t* b, size_t m, size_t k, size_t n, int32_t* out) {
    for (size_t i = 0; i < m; ++i)
        for (size_t o = 0; o < n; ++o) {
            uint32_t acc = 0;
            for (size_t p = 0; p < k; ++p) acc += static_cast<uint32_t>(static_cast<int32_t>(a[i * k + p]) * b[o * k + p]);
            out[i * n + o] = static_cast<int32_t>(static_cast<uint32_t>(out[i * n + o]) + acc);
        }
}

void append(std::string& j, const char* f, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, f);
    vsnprintf(buf, sizeof(buf), f, ap);
    va_end(ap);
    j += buf;
}

}  // namespace

extern "C" {

int32_t focr_hip_selftest(focr_hip_ctx* ctx, char* json, size_t cap, int32_t* all_ok) {
    if (!ctx) return fail(FOCR_HIP_E_BAD_HANDLE, "null focr_hip_ctx");
    bool ok_all = true;
    std::string j = "{\"selected\":\"gfx950\",\"feature\":\"gfx950+mfma-i8\",\"available\":[\"gfx950\"],\"cases\":[";
    bool first = true;
    for (const Shape& sh : kShapes) {
        for (int dom = 0; dom < 2; ++dom) {
            const size_t mk = sh.m * sh.k, nk = sh.n * sh.k, mn = sh.m * sh.n;
            std::vector<int8_t> as(mk), b(nk);
            std::vector<uint8_t> au(mk);
            if (sh.seed == 0) {
                // worst-case magnitude (dispatch.rs:382-385, :403-404)
                std::fill(as.begin(), as.end(), static_cast<int8_t>(127));
                std::fill(au.begin(), au.end(), static_cast<uint8_t>(255));
                std::fill(b.begin(), b.end(), static_cast<int8_t>(-128));
            } else {
                uint32_t st = dom == 0 ? (sh.seed | 1u) : (((sh.seed << 7) | (sh.seed >> 25)) | 1u);
                for (size_t i = 0; i < mk; ++i) {
                    const uint32_t v = xs32(st) & 0xffu;
                    as[i] = static_cast<int8_t>(static_cast<uint8_t>(v));
                    au[i] = static_cast<uint8_t>(v);
                }
                for (size_t i = 0; i < nk; ++i) b[i] = static_cast<int8_t>(static_cast<uint8_t>(xs32(st) & 0xffu));
            }
            std::vector<int32_t> got(mn, 0), want(mn, 0);
            int32_t st;
            if (dom == 0) {
                st = focr_hip_igemm_s8s8(ctx, as.data(), mk, b.data(), nk, sh.m, sh.k, sh.n, got.data(), mn);
                scalar_check(as.data(), b.data(), sh.m, sh.k, sh.n, want.data());
            } else {
                st = focr_hip_igemm_u8s8(ctx, au.data(), mk, b.data(), nk, sh.m, sh.k, sh.n, got.data(), mn);
                scalar_check(au.data(), b.data(), sh.m, sh.k, sh.n, want.data());
            }
            if (st) return st;
            size_t mism = 0, first_bad = 0;
            for (size_t i = 0; i < mn; ++i)
                if (got[i] != want[i]) {
                    if (!mism) first_bad = i;
                    ++mism;
                }
            ok_all = ok_all && mism == 0;
            append(j, "%s{\"kind\":\"%s\",\"label\":\"%s\",\"m\":%zu,\"k\":%zu,\"n\":%zu,\"ok\":%s,\"mismatches\":%zu",
                   first ? "" : ",", dom == 0 ? "s8s8" : "u8s8", sh.label, sh.m, sh.k, sh.n, mism ? "false" : "true",
                   mism);
            if (mism)
                append(j, ",\"first_bad\":[%zu,%d,%d]", first_bad, got[first_bad], want[first_bad]);
            j += "}";
            first = false;
        }
    }
    append(j, "],\"all_ok\":%s}", ok_all ? "true" : "false");
    if (all_ok) *all_ok = ok_all ? 1 : 0;
    if (json && cap) snprintf(json, cap, "%s", j.c_str());
    return FOCR_HIP_OK;
}

// ---- QInt8 handles ---------------------------------------------------------

int32_t focr_hip_qint8_upload(focr_hip_ctx* ctx, const int8_t* w, const float* scales, size_t n, size_t k,
                              focr_hip_qint8** out) {
    ENGINE_CTX(ctx);
    if (!out) return fail(FOCR_HIP_E_ARG, "qint8_upload: null out");
    *out = nullptr;
    if (n * k && (!w || !scales)) return fail(FOCR_HIP_E_ARG, "qint8_upload: null host pointer");
    if (k % 16 != 0 || k == 0 || n == 0 || n > static_cast<size_t>(std::numeric_limits<int32_t>::max()))
        return fail(FOCR_HIP_E_SHAPE, fmt("QInt8: gfx950 tier needs k a positive multiple of 16 and 0 < n < 2^31 (n=%zu k=%zu)", n, k));
    std::unique_ptr<focr_hip_qint8> q(new focr_hip_qint8());
    q->ctx = ctx;
    q->n = n;
    q->k = k;
    q->owned = true;
    FOCR_HIP_TRY(hipMalloc(reinterpret_cast<void**>(&q->w), n * k), "hipMalloc qint8 w");
    hipError_t e = hipMalloc(reinterpret_cast<void**>(&q->scales), n * sizeof(float));
    if (e != hipSuccess) {
        hipFree(q->w);
        return hip_fail(e, "hipMalloc qint8 scales");
    }
    FOCR_HIP_TRY(hipMemcpyAsync(q->w, w, n * k, hipMemcpyHostToDevice, ctx->stream), "H2D qint8 w");
    FOCR_HIP_TRY(hipMemcpyAsync(q->scales, scales, n * sizeof(float), hipMemcpyHostToDevice, ctx->stream), "H2D scales");
    FOCR_HIP_TRY(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
    *out = q.release();
    return FOCR_HIP_OK;
}

int32_t focr_hip_qint8_from_device(focr_hip_ctx* ctx, const int8_t* w, const float* scales, size_t n, size_t k,
                                   focr_hip_qint8** out) {
    ENGINE_CTX(ctx);
    if (!out) return fail(FOCR_HIP_E_ARG, "qint8_from_device: null out");
    *out = nullptr;
    if (!w || !scales) return fail(FOCR_HIP_E_ARG, "qint8_from_device: null device pointer");
    if (k % 16 != 0 || k == 0 || n == 0 || n > static_cast<size_t>(std::numeric_limits<int32_t>::max()))
        return fail(FOCR_HIP_E_SHAPE, fmt("QInt8: gfx950 tier needs k a positive multiple of 16 and 0 < n < 2^31 (n=%zu k=%zu)", n, k));
    if (reinterpret_cast<uintptr_t>(w) % 16 != 0)
        return fail(FOCR_HIP_E_ARG, "qint8_from_device: weights must be 16-byte aligned");
    focr_hip_qint8* q = new focr_hip_qint8();
    q->ctx = ctx;
    q->w = const_cast<int8_t*>(w);
    q->scales = const_cast<float*>(scales);
    q->n = n;
    q->k = k;
    q->owned = false;
    *out = q;
    return FOCR_HIP_OK;
}

int32_t focr_hip_qint8_free(focr_hip_qint8* w) {
    if (!w) return FOCR_HIP_OK;
    if (w->owned || w->w_mfma || w->w_tiled) {
        hipSetDevice(w->ctx->device);
        hipStreamSynchronize(w->ctx->stream);
    }
    if (w->owned) {
        hipFree(w->w);
        hipFree(w->scales);
    }
    hipFree(w->w_mfma);
    hipFree(w->w_tiled);
    delete w;
    return FOCR_HIP_OK;
}

// ---- GEMV / LM head ------------------------------------------------------

int32_t focr_hip_quantize_rows_i8(focr_hip_ctx* ctx, const float* x, size_t m, size_t k, int8_t* xq,
                                  float* a_scales, int32_t rule) {
    ENGINE_CTX(ctx);
    if (rule < 0 || rule > kQuantRuleDynamic) return fail(FOCR_HIP_E_ARG, fmt("quantize_rows_i8: unknown rule %d", rule));
    if (m == 0) return FOCR_HIP_OK;
    if (!x || !xq || !a_scales) return fail(FOCR_HIP_E_ARG, "quantize_rows_i8: null device pointer");
    if (m > 65535 || k > static_cast<size_t>(std::numeric_limits<int32_t>::max()))
        return fail(FOCR_HIP_E_SHAPE, "quantize_rows_i8: too many rows");
    ProfScope ps(ctx, "quantize_rows");
    FOCR_HIP_TRY(launch_quantize_rows(ctx->stream, x, (int)m, (int)k, xq, a_scales, rule), "quantize launch");
    return FOCR_HIP_OK;
}

static int32_t gemv_checks(const char* name, const focr_hip_qint8* w, size_t m) {
    if (!w) return fail(FOCR_HIP_E_BAD_HANDLE, fmt("%s: null weight handle", name));
    if (m < 1 || m > 32) return fail(FOCR_HIP_E_SHAPE, fmt("%s: m %zu outside 1..=32 for one call", name, m));
    if (m * w->k > 57344) return fail(FOCR_HIP_E_SHAPE, fmt("%s: m*k %zu exceeds the 56 KiB LDS stage", name, m * w->k));
    return FOCR_HIP_OK;
}

int32_t focr_hip_gemv_i8_prequant(focr_hip_ctx* ctx, const focr_hip_qint8* w, const int8_t* xq,
                                  const float* a_scales, size_t m, float* y, int32_t* acc) {
    ENGINE_CTX(ctx);
    int32_t st = gemv_checks("gemv_i8_prequant", w, m);
    if (st) return st;
    if (!xq || !a_scales || !y) return fail(FOCR_HIP_E_ARG, "gemv_i8_prequant: null device pointer");
    ProfScope ps(ctx, "gemv_i8");
    FOCR_HIP_TRY(launch_gemv_i8(ctx->stream, w->w, w->scales, (int)w->n, (int)w->k, xq, a_scales, (int)m, y, acc,
                                nullptr, nullptr, ctx->cu_count),
                 "gemv launch");
    return FOCR_HIP_OK;
}

int32_t focr_hip_gemv_i8(focr_hip_ctx* ctx, const focr_hip_qint8* w, const float* x, size_t m, float* y) {
    ENGINE_CTX(ctx);
    int32_t st = gemv_checks("gemv_i8", w, m);
    if (st) return st;
    if (!x || !y) return fail(FOCR_HIP_E_ARG, "gemv_i8: null device pointer");
    int8_t* xq = static_cast<int8_t*>(ctx->scratch_get(kScrXq, m * w->k));
    float* xs = static_cast<float*>(ctx->scratch_get(kScrXs, m * sizeof(float)));
    if (!xq || !xs) return FOCR_HIP_E_OOM;
    // quantize_row_i8 + the GEMV (one launch where the rows fit the blocks'
    // own quantization)
    ProfScope ps(ctx, "gemv_i8");
    FOCR_HIP_TRY(launch_gemv_i8_f32(ctx->stream, w->w, w->scales, (int)w->n, (int)w->k, x, nullptr, 0.0f, (int)m, y,
                                    xq, xs, ctx->cu_count),
                 "gemv launch");
    return FOCR_HIP_OK;
}

static int32_t lm_head_i8_impl(focr_hip_ctx* ctx, const focr_hip_qint8* w, const float* x, size_t m, float* logits,
                            uint32_t* argmax) {
    int32_t st = gemv_checks("lm_head_i8", w, m);
    if (st) return st;
    if (!x || !argmax) return fail(FOCR_HIP_E_ARG, "lm_head_i8: null device pointer");
    int8_t* xq = static_cast<int8_t*>(ctx->scratch_get(kScrXq, m * w->k));
    float* xs = static_cast<float*>(ctx->scratch_get(kScrXs, m * sizeof(float)));
    const int nparts = gemv_i8_nparts((int)w->n, ctx->cu_count);
    uint64_t* keys = static_cast<uint64_t*>(ctx->scratch_get(kScrArg, m * nparts * sizeof(uint64_t)));
    float* y = logits ? logits : static_cast<float*>(ctx->scratch_get(kScrLogits, m * w->n * sizeof(float)));
    if (!xq || !xs || !keys || !y) return FOCR_HIP_E_OOM;
    int np = 0;
    // the GEMV blocks quantize the rows themselves where the shape allows (one
    // launch fewer)
    hipError_t fe;
    {
        ProfScope ps(ctx, "lm_head_gemv");
        fe = launch_gemv_i8_f32_keys(ctx->stream, w->w, w->scales, (int)w->n, (int)w->k, x, (int)m, y, keys, &np,
                                     ctx->cu_count);
        if (fe != hipErrorNotSupported) FOCR_HIP_TRY(fe, "lm_head gemv launch");
    }
    if (fe == hipErrorNotSupported) {
        {
            ProfScope ps(ctx, "quantize_rows");
            FOCR_HIP_TRY(launch_quantize_rows(ctx->stream, x, (int)m, (int)w->k, xq, xs, false), "quantize launch");
        }
        ProfScope ps(ctx, "lm_head_gemv");
        FOCR_HIP_TRY(launch_gemv_i8(ctx->stream, w->w, w->scales, (int)w->n, (int)w->k, xq, xs, (int)m, y, nullptr,
                                    keys, &np, ctx->cu_count),
                     "lm_head gemv launch");
    }
    ProfScope ps(ctx, "argmax_reduce");
    FOCR_HIP_TRY(launch_argmax_reduce(ctx->stream, keys, (int)m, np, argmax), "argmax launch");
    return FOCR_HIP_OK;
}

int32_t focr_hip_lm_head_i8(focr_hip_ctx* ctx, const focr_hip_qint8* w, const float* x, size_t m, float* logits,
                            uint32_t* argmax) {
    ENGINE_CTX(ctx);
    return lm_head_i8_impl(ctx, w, x, m, logits, argmax);
}

}  // extern "C"

// ---- greedy sampler --------------------------------------------------------

namespace {

int32_t sampler_args(focr_hip_ctx* ctx, const char* name, size_t m, size_t vocab, uint32_t* history,
                     size_t history_cap, uint32_t* history_len, size_t ngram_size, size_t window,
                     const uint32_t* whitelist, size_t n_whitelist, float temperature, int32_t append,
                     SamplerArgs& a) {
    // sampler.rs:362-367: temperature > 0 is outside the greedy spine (a NaN
    // temperature is greedy, sampler.rs:96-100).
    if (temperature > 0.0f)
        return fail(FOCR_HIP_E_NOT_IMPLEMENTED,
                    fmt("native_engine::sampler::%s — temperature>0 sampling is outside the greedy fp32 spine", name));
    if (vocab == 0) return fail(FOCR_HIP_E_SHAPE, "sampler::argmax_row: empty logits row");
    const size_t imax = static_cast<size_t>(std::numeric_limits<int32_t>::max());
    if (history_cap > imax || ngram_size > imax || window > imax || n_whitelist > 4096 || vocab > imax)
        return fail(FOCR_HIP_E_SHAPE, fmt("%s: history_cap / ngram_size / window / whitelist exceed the gfx950 tier "
                                          "limits", name));
    if ((ngram_size > 0 || append) && (!history || !history_len || history_cap == 0))
        return fail(FOCR_HIP_E_ARG, fmt("%s: the no-repeat-ngram ban and append need history, history_len and a "
                                        "positive history_cap", name));
    if (n_whitelist && !whitelist) return fail(FOCR_HIP_E_ARG, fmt("%s: null whitelist", name));
    const size_t words = (vocab + 31) / 32;
    a.history = history;
    a.history_mut = append ? history : nullptr;
    a.history_len = history_len;
    a.cap = static_cast<int>(history_cap);
    a.ngram = static_cast<int>(ngram_size);
    a.window = static_cast<int>(window);
    a.whitelist = whitelist;
    a.n_white = static_cast<int>(n_whitelist);
    a.vocab = static_cast<int>(vocab);
    a.ban_words = static_cast<int>(words);
    a.ban_bits = static_cast<uint32_t*>(ctx->scratch_get(kScrBan, m * words * sizeof(uint32_t)));
    a.err = static_cast<int*>(ctx->scratch_get(kScrFlag, m * sizeof(int)));
    if (!a.ban_bits || !a.err) return FOCR_HIP_E_OOM;
    return FOCR_HIP_OK;
}

int32_t sampler_check(focr_hip_ctx* ctx, const SamplerArgs& a, size_t m) {
    std::vector<int> flags(m);
    FOCR_HIP_TRY(hipMemcpyAsync(flags.data(), a.err, m * sizeof(int), hipMemcpyDeviceToHost, ctx->stream),
                 "D2H sampler flags");
    FOCR_HIP_TRY(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
    for (size_t r = 0; r < m; ++r) {
        if (flags[r] & 1)
            return fail(FOCR_HIP_E_SHAPE, fmt("sampler: history_len of row %zu exceeds history_cap %d", r, a.cap));
        if (flags[r] & 2)
            return fail(FOCR_HIP_E_SHAPE, fmt("sampler: row %zu history is full (history_cap %d); the token was not "
                                              "appended", r, a.cap));
    }
    return FOCR_HIP_OK;
}

}  // namespace

extern "C" {

static int32_t lm_head_sample_i8_impl(focr_hip_ctx* ctx, const focr_hip_qint8* w, const float* x, size_t m,
                                   uint32_t* history, size_t history_cap, uint32_t* history_len, size_t ngram_size,
                                   size_t window, const uint32_t* whitelist, size_t n_whitelist, float temperature,
                                   uint32_t eos_token_id, int32_t append, float* logits, uint32_t* tokens,
                                   uint8_t* is_eos, int32_t check) {
    int32_t st = gemv_checks("lm_head_sample_i8", w, m);
    if (st) return st;
    if (!x || !tokens) return fail(FOCR_HIP_E_ARG, "lm_head_sample_i8: null device pointer");
    SamplerArgs a;
    if ((st = sampler_args(ctx, "decode_step_premasked", m, w->n, history, history_cap, history_len, ngram_size,
                           window, whitelist, n_whitelist, temperature, append, a)))
        return st;
    int8_t* xq = static_cast<int8_t*>(ctx->scratch_get(kScrXq, m * w->k));
    float* xs = static_cast<float*>(ctx->scratch_get(kScrXs, m * sizeof(float)));
    const int nparts = gemv_i8_nparts((int)w->n, ctx->cu_count);
    uint64_t* keys = static_cast<uint64_t*>(ctx->scratch_get(kScrArg, m * nparts * sizeof(uint64_t)));
    float* y = logits ? logits : static_cast<float*>(ctx->scratch_get(kScrLogits, m * w->n * sizeof(float)));
    if (!xq || !xs || !keys || !y) return FOCR_HIP_E_OOM;
    {
        ProfScope ps(ctx, "sampler_prep");
        FOCR_HIP_TRY(launch_sampler_prep(ctx->stream, (int)m, x, (int)w->k, xq, xs, a), "sampler_prep launch");
    }
    int np = 0;
    {
        ProfScope ps(ctx, "lm_head_gemv");
        FOCR_HIP_TRY(launch_gemv_i8_banned(ctx->stream, w->w, w->scales, (int)w->n, (int)w->k, xq, xs, (int)m, y,
                                           nullptr, keys, &np, ctx->cu_count, a.ban_bits, a.ban_words),
                     "lm_head gemv launch");
    }
    {
        ProfScope ps(ctx, "sample_finish");
        FOCR_HIP_TRY(launch_sample_finish(ctx->stream, (int)m, keys, np, eos_token_id, tokens, is_eos, a),
                     "sample_finish launch");
    }
    return check ? sampler_check(ctx, a, m) : FOCR_HIP_OK;
}

int32_t focr_hip_lm_head_sample_i8(focr_hip_ctx* ctx, const focr_hip_qint8* w, const float* x, size_t m,
                                   uint32_t* history, size_t history_cap, uint32_t* history_len, size_t ngram_size,
                                   size_t window, const uint32_t* whitelist, size_t n_whitelist, float temperature,
                                   uint32_t eos_token_id, int32_t append, float* logits, uint32_t* tokens,
                                   uint8_t* is_eos, int32_t check) {
    ENGINE_CTX(ctx);
    return lm_head_sample_i8_impl(ctx, w, x, m, history, history_cap, history_len, ngram_size, window, whitelist,
                                  n_whitelist, temperature, eos_token_id, append, logits, tokens, is_eos, check);
}

int32_t focr_hip_sample_rows(focr_hip_ctx* ctx, const float* logits, size_t m, size_t n, uint32_t* history,
                             size_t history_cap, uint32_t* history_len, size_t ngram_size, size_t window,
                             const uint32_t* whitelist, size_t n_whitelist, float temperature, uint32_t eos_token_id,
                             int32_t append, uint32_t* tokens, uint8_t* is_eos, int32_t check) {
    ENGINE_CTX(ctx);
    if (m == 0) return FOCR_HIP_OK;
    if (!logits || !tokens) return fail(FOCR_HIP_E_ARG, "sample_rows: null device pointer");
    if (m > 65535) return fail(FOCR_HIP_E_SHAPE, "sample_rows: m exceeds the gfx950 tier limit of 65535 rows");
    SamplerArgs a;
    int32_t st = sampler_args(ctx, "sample", m, n, history, history_cap, history_len, ngram_size, window, whitelist,
                              n_whitelist, temperature, append, a);
    if (st) return st;
    const int nparts = static_cast<int>(std::min<size_t>(256, (n + 4095) / 4096));
    uint64_t* keys = static_cast<uint64_t*>(ctx->scratch_get(kScrArg, m * nparts * sizeof(uint64_t)));
    if (!keys) return FOCR_HIP_E_OOM;
    ProfScope ps(ctx, "sample_rows");
    FOCR_HIP_TRY(launch_sampler_prep(ctx->stream, (int)m, nullptr, 0, nullptr, nullptr, a), "sampler_prep launch");
    FOCR_HIP_TRY(launch_argmax_partial(ctx->stream, logits, (int)m, (int)n, keys, nparts, a.ban_bits, a.ban_words),
                 "argmax launch");
    FOCR_HIP_TRY(launch_sample_finish(ctx->stream, (int)m, keys, nparts, eos_token_id, tokens, is_eos, a),
                 "sample_finish launch");
    return check ? sampler_check(ctx, a, m) : FOCR_HIP_OK;
}

int32_t focr_hip_argmax_rows(focr_hip_ctx* ctx, const float* logits, size_t m, size_t n, uint32_t* argmax) {
    ENGINE_CTX(ctx);
    if (m == 0) return FOCR_HIP_OK;
    if (n == 0) return fail(FOCR_HIP_E_SHAPE, "sampler::argmax_row: empty logits row");
    if (!logits || !argmax) return fail(FOCR_HIP_E_ARG, "argmax_rows: null device pointer");
    if (m > 65535 || n > static_cast<size_t>(std::numeric_limits<int32_t>::max()))
        return fail(FOCR_HIP_E_SHAPE, "argmax_rows: shape exceeds the gfx950 tier limit");
    const int nparts = static_cast<int>(std::min<size_t>(256, (n + 4095) / 4096));
    uint64_t* keys = static_cast<uint64_t*>(ctx->scratch_get(kScrArg, m * nparts * sizeof(uint64_t)));
    if (!keys) return FOCR_HIP_E_OOM;
    ProfScope ps(ctx, "argmax_rows");
    FOCR_HIP_TRY(launch_argmax_rows(ctx->stream, logits, (int)m, (int)n, keys, nparts, argmax), "argmax launch");
    return FOCR_HIP_OK;
}

}  // extern "C"

// ---- MoE layer ---------------------------------------------------------------

namespace {

template <typename T>
int32_t upload(focr_hip_ctx* ctx, T** dst, const T* src, size_t count, bool from_device, const char* what) {
    if (from_device) {
        *dst = const_cast<T*>(src);
        return FOCR_HIP_OK;
    }
    FOCR_HIP_TRY(hipMalloc(reinterpret_cast<void**>(dst), std::max<size_t>(count * sizeof(T), 16)), what);
    FOCR_HIP_TRY(hipMemcpyAsync(*dst, src, count * sizeof(T), hipMemcpyHostToDevice, ctx->stream), what);
    return FOCR_HIP_OK;
}

void free_moe(focr_hip_moe_layer* L) {
    if (L->owned) {
        hipFree(L->router);
        hipFree(L->wg);
        hipFree(L->wu);
        hipFree(L->wd);
        hipFree(L->sg);
        hipFree(L->su);
        hipFree(L->sd);
    }
    if (L->shared_owned) {
        hipFree(L->swg);
        hipFree(L->swu);
        hipFree(L->swd);
        hipFree(L->ssg);
        hipFree(L->ssu);
        hipFree(L->ssd);
    }
    for (int8_t* p : {L->wg_mfma, L->wu_mfma, L->wd_mfma, L->swg_mfma, L->swu_mfma, L->swd_mfma})
        hipFree(p);
}

}  // namespace

extern "C" {

int32_t focr_hip_moe_layer_create(focr_hip_ctx* ctx, size_t hidden, size_t inter, size_t n_experts, size_t top_k,
                                  const float* router, const int8_t* wg, const float* sg, const int8_t* wu,
                                  const float* su, const int8_t* wd, const float* sd, int32_t from_device,
                                  focr_hip_moe_layer** out) {
    ENGINE_CTX(ctx);
    if (!out) return fail(FOCR_HIP_E_ARG, "moe_layer_create: null out");
    *out = nullptr;
    if (!router || !wg || !sg || !wu || !su || !wd || !sd) return fail(FOCR_HIP_E_ARG, "moe_layer_create: null pointer");
    if (n_experts < top_k) return fail(FOCR_HIP_E_SHAPE, fmt("moe::route: n_routed_experts %zu < top_k %zu", n_experts, top_k));
    if (n_experts < 1 || n_experts > 64 || top_k < 1 || top_k > 8)
        return fail(FOCR_HIP_E_SHAPE, fmt("moe_layer_create: gfx950 tier supports 1..=64 experts and top_k 1..=8 (got %zu, %zu)", n_experts, top_k));
    if (hidden % 16 || inter % 16 || hidden == 0 || inter == 0 || hidden > 2048 || inter > 2048)
        return fail(FOCR_HIP_E_SHAPE, fmt("moe_layer_create: hidden/inter must be multiples of 16 in 16..=2048 (got %zu, %zu)", hidden, inter));
    std::unique_ptr<focr_hip_moe_layer> L(new focr_hip_moe_layer());
    L->ctx = ctx;
    L->hidden = hidden;
    L->inter = inter;
    L->n_experts = n_experts;
    L->top_k = top_k;
    L->owned = !from_device;
    const size_t E = n_experts;
    int32_t st = FOCR_HIP_OK;
    if ((st = upload(ctx, &L->router, router, E * hidden, from_device, "router")) ||
        (st = upload(ctx, &L->wg, wg, E * inter * hidden, from_device, "w_gate")) ||
        (st = upload(ctx, &L->sg, sg, E * inter, from_device, "s_gate")) ||
        (st = upload(ctx, &L->wu, wu, E * inter * hidden, from_device, "w_up")) ||
        (st = upload(ctx, &L->su, su, E * inter, from_device, "s_up")) ||
        (st = upload(ctx, &L->wd, wd, E * hidden * inter, from_device, "w_down")) ||
        (st = upload(ctx, &L->sd, sd, E * hidden, from_device, "s_down"))) {
        hipStreamSynchronize(ctx->stream);
        free_moe(L.get());
        return st;
    }
    FOCR_HIP_TRY(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
    *out = L.release();
    return FOCR_HIP_OK;
}

int32_t focr_hip_moe_layer_set_shared(focr_hip_moe_layer* L, size_t shared_inter, const int8_t* wg, const float* sg,
                                      const int8_t* wu, const float* su, const int8_t* wd, const float* sd,
                                      int32_t from_device) {
    if (!L) return fail(FOCR_HIP_E_BAD_HANDLE, "null moe layer");
    focr_hip_ctx* ctx = L->ctx;
    ENGINE_CTX(ctx);
    if (!wg || !sg || !wu || !su || !wd || !sd) return fail(FOCR_HIP_E_ARG, "moe_layer_set_shared: null pointer");
    if (shared_inter % 16 || shared_inter == 0 || shared_inter > 2048)
        return fail(FOCR_HIP_E_SHAPE, fmt("moe_layer_set_shared: shared_inter must be a multiple of 16 in 16..=2048 (got %zu)", shared_inter));
    const size_t h = L->hidden;
    focr_hip_moe_layer tmp = *L;
    tmp.shared_owned = !from_device;
    int32_t st = FOCR_HIP_OK;
    if ((st = upload(ctx, &tmp.swg, wg, shared_inter * h, from_device, "shared w_gate")) ||
        (st = upload(ctx, &tmp.ssg, sg, shared_inter, from_device, "shared s_gate")) ||
        (st = upload(ctx, &tmp.swu, wu, shared_inter * h, from_device, "shared w_up")) ||
        (st = upload(ctx, &tmp.ssu, su, shared_inter, from_device, "shared s_up")) ||
        (st = upload(ctx, &tmp.swd, wd, h * shared_inter, from_device, "shared w_down")) ||
        (st = upload(ctx, &tmp.ssd, sd, h, from_device, "shared s_down")))
        return st;
    FOCR_HIP_TRY(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
    if (L->shared_owned) {
        hipFree(L->swg);
        hipFree(L->swu);
        hipFree(L->swd);
        hipFree(L->ssg);
        hipFree(L->ssu);
        hipFree(L->ssd);
    }
    for (int8_t** p : {&L->swg_mfma, &L->swu_mfma, &L->swd_mfma}) {  // rebuilt by the next prefill
        hipFree(*p);
        *p = nullptr;
    }
    L->shared_inter = shared_inter;
    L->swg = tmp.swg;
    L->ssg = tmp.ssg;
    L->swu = tmp.swu;
    L->ssu = tmp.ssu;
    L->swd = tmp.swd;
    L->ssd = tmp.ssd;
    L->shared_owned = tmp.shared_owned;
    return FOCR_HIP_OK;
}

int32_t focr_hip_moe_layer_free(focr_hip_moe_layer* L) {
    if (!L) return FOCR_HIP_OK;
    hipSetDevice(L->ctx->device);
    hipStreamSynchronize(L->ctx->stream);
    free_moe(L);
    delete L;
    return FOCR_HIP_OK;
}

}  // extern "C"

namespace {

struct MoeScratch {
    int8_t* xq;
    float* xs;
    uint32_t* idx;
    float* gates;
    int* flag;
    float* act;
    float* shared_act;
    float* shared_y;
    int8_t* shared_aq;  // [t][shared_inter] quantized shared act rows
    float* shared_as;   // [t]
    float* ybuf;  // [pairs][hidden] weighted expert outputs (grouped down path only)
    void* sel;
    void* xchg;   // the route's cross-block exchange (moe_route_xchg_bytes)
};

// Where an entry point's intermediates live: the context's grow-only slots
// (hipMalloc when a slot grows), or consecutive 256-byte aligned pieces of
// the static per-device array (never allocates). In counting mode nothing is
// handed out for use: `used` totals the bytes a call would carve.
struct ScratchSource {
    focr_hip_ctx* ctx = nullptr;
    char* base = nullptr;  // the static array; null selects the context's slots
    size_t cap = 0, used = 0;
    bool counting = false;
    void* get(int slot, size_t bytes) {
        if (!base && !counting) return ctx->scratch_get(slot, bytes);
        const size_t off = (used + 255) & ~static_cast<size_t>(255);
        used = off + (bytes ? bytes : 16);
        if (counting) return reinterpret_cast<void*>(static_cast<uintptr_t>(256));  // placeholder, never dereferenced
        return used <= cap ? base + off : nullptr;
    }
};

int32_t moe_scratch(ScratchSource& src, const focr_hip_moe_layer* L, size_t t, bool with_shared, MoeScratch* s) {
    const size_t pairs = t * L->top_k;
    // the route's exchange comes first: in the static array it is then always
    // at offset 0 (zero from load time, and only the route writes there); a
    // context slot is zeroed once, when it is allocated
    const size_t xb = moe_route_xchg_bytes(kMoeMaxT);  // one size for every decode call
    const bool fresh = !src.base && !src.counting && src.ctx->scratch[kScrRouteX].cap < xb;
    s->xchg = src.get(kScrRouteX, xb);
    if (!s->xchg) return FOCR_HIP_E_OOM;
    if (fresh && hipMemsetAsync(s->xchg, 0, src.ctx->scratch[kScrRouteX].cap, src.ctx->stream) != hipSuccess)
        return FOCR_HIP_E_OOM;
    const size_t sel_off = (pairs * 8 + 255) & ~static_cast<size_t>(255);
    char* route = static_cast<char*>(src.get(kScrRoute, sel_off + moe_sel_bytes()));
    s->xq = static_cast<int8_t*>(src.get(kScrXq, t * L->hidden));
    s->xs = static_cast<float*>(src.get(kScrXs, t * sizeof(float)));
    s->act = static_cast<float*>(src.get(kScrAct, (pairs * L->inter + (with_shared ? t * L->shared_inter : 0)) * sizeof(float)));
    char* shb = with_shared ? static_cast<char*>(src.get(
                                  kScrShared, t * L->hidden * sizeof(float) + 256 + t * L->shared_inter + 256 + t * 4))
                            : nullptr;
    s->shared_y = reinterpret_cast<float*>(shb);
    s->shared_aq = shb ? reinterpret_cast<int8_t*>(shb + ((t * L->hidden * sizeof(float) + 255) & ~size_t(255))) : nullptr;
    s->shared_as = shb ? reinterpret_cast<float*>(reinterpret_cast<char*>(s->shared_aq) + ((t * L->shared_inter + 255) & ~size_t(255)))
                       : nullptr;
    s->flag = static_cast<int*>(src.get(kScrFlag, t * sizeof(int)));
    const bool grouped = static_cast<int>(t) >= kMoeGroupedDownT;
    s->ybuf = grouped ? static_cast<float*>(src.get(kScrY, pairs * L->hidden * sizeof(float))) : nullptr;
    if (!route || !s->xq || !s->xs || !s->act || !s->flag || (with_shared && !s->shared_y) || (grouped && !s->ybuf))
        return FOCR_HIP_E_OOM;
    s->idx = reinterpret_cast<uint32_t*>(route);
    s->gates = reinterpret_cast<float*>(route + pairs * 4);
    s->sel = route ? route + sel_off : nullptr;
    s->shared_act = with_shared ? s->act + pairs * L->inter : nullptr;
    return FOCR_HIP_OK;
}

int32_t moe_checks(const char* name, const focr_hip_moe_layer* L, const float* hidden, size_t t, int32_t with_shared) {
    if (!L) return fail(FOCR_HIP_E_BAD_HANDLE, fmt("%s: null moe layer", name));
    if (!hidden) return fail(FOCR_HIP_E_ARG, fmt("%s: null hidden", name));
    if (t < 1 || t > static_cast<size_t>(kMoeMaxT))
        return fail(FOCR_HIP_E_SHAPE, fmt("%s: t %zu outside 1..=%d for one call", name, t, kMoeMaxT));
    if (with_shared && !L->swg) return fail(FOCR_HIP_E_ARG, fmt("%s: with_shared set but no shared expert uploaded", name));
    return FOCR_HIP_OK;
}

// The route kernel writes flag[t] = 1 for a token with fewer than top_k
// finite router scores (moe.rs:261-265). Reading it synchronises.
// token_base: the first row's index in the caller's call (chunked calls).
int32_t check_route_flags(focr_hip_ctx* ctx, const int* dflag, size_t t, size_t token_base = 0) {
    std::vector<int> flags(t);
    FOCR_HIP_TRY(hipMemcpyAsync(flags.data(), dflag, t * sizeof(int), hipMemcpyDeviceToHost, ctx->stream),
                 "D2H route flag");
    FOCR_HIP_TRY(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
    for (size_t i = 0; i < t; ++i)
        if (flags[i])
            return fail(FOCR_HIP_E_ROUTE, fmt("moe::route: no finite router score for token %zu", token_base + i));
    return FOCR_HIP_OK;
}

int32_t launch_route(focr_hip_ctx* ctx, const focr_hip_moe_layer* L, const float* hidden, size_t t, int32_t norm_topk,
                     float routed_scale, const MoeScratch& s, uint32_t* idx, float* gates, float* probs,
                     void* sel, const MoeRouteNorm* norm = nullptr) {
    const MoeDims d{(int)t, (int)L->hidden, (int)L->inter, (int)L->n_experts, (int)L->top_k};
    ProfScope ps(ctx, "moe_route");
    FOCR_HIP_TRY(launch_moe_route(ctx->stream, d, hidden, L->router, norm_topk, routed_scale, s.xq, s.xs, idx, gates,
                                  probs, s.flag, sel, s.xchg, ctx->route_wait_ticks, norm),
                 "route launch");
    return FOCR_HIP_OK;
}

}  // namespace

extern "C" {

// route (moe.rs:181-266) of t rows (up to kRouteRowsMax) without the decode
// kernels' selection matrices: idx / gates [t][top_k], probs [t][E]
// (nullable), flag [t] (1: fewer than top_k finite scores). Rows up to 1280
// wide take the many-row route (a logits kernel that reads the router once
// per 8 tokens, then the rank kernel; the logits in the logits slot): the
// split route's arithmetic, bit for bit. Wider rows take the split route
// kernel; its exchange buffer grows to t tokens (zeroed when it grows) and a
// one-thread launch advances the buffer's counter after it.
constexpr size_t kRouteRowsMax = 16384;
static int32_t route_rows_impl(focr_hip_ctx* ctx, const focr_hip_moe_layer* L, const float* x, size_t t,
                               int32_t norm_topk, float routed_scale, uint32_t* idx, float* gates, float* probs,
                               int* flag) {
    if (moe_route_rows_supported(static_cast<int>(L->hidden))) {
        float* lg = static_cast<float*>(ctx->scratch_get(kScrLogits, t * L->n_experts * sizeof(float)));
        if (!lg) return FOCR_HIP_E_OOM;
        const MoeDims d{(int)t, (int)L->hidden, (int)L->inter, (int)L->n_experts, (int)L->top_k};
        ProfScope ps(ctx, "moe_route");
        FOCR_HIP_TRY(launch_moe_route_rows(ctx->stream, d, x, L->router, norm_topk, routed_scale, idx, gates, probs,
                                           flag, lg),
                     "route launch");
        return FOCR_HIP_OK;
    }
    const size_t xb = moe_route_xchg_bytes(t);
    const bool grow = ctx->scratch[kScrRouteX].cap < xb;
    void* xchg = ctx->scratch_get(kScrRouteX, xb);
    int8_t* xq = static_cast<int8_t*>(ctx->scratch_get(kScrXq, t * L->hidden));
    float* xs = static_cast<float*>(ctx->scratch_get(kScrXs, t * sizeof(float)));
    if (!xchg || !xq || !xs) return FOCR_HIP_E_OOM;
    if (grow) FOCR_HIP_TRY(hipMemsetAsync(xchg, 0, ctx->scratch[kScrRouteX].cap, ctx->stream), "route exchange zero");
    const MoeDims d{(int)t, (int)L->hidden, (int)L->inter, (int)L->n_experts, (int)L->top_k};
    {
        ProfScope ps(ctx, "moe_route");
        FOCR_HIP_TRY(launch_moe_route(ctx->stream, d, x, L->router, norm_topk, routed_scale, xq, xs, idx, gates, probs,
                                      flag, nullptr, xchg, ctx->route_wait_ticks),
                     "route launch");
    }
    FOCR_HIP_TRY(launch_route_epoch_bump(ctx->stream, xchg), "route epoch launch");
    return FOCR_HIP_OK;
}

int32_t focr_hip_moe_route(focr_hip_ctx* ctx, const focr_hip_moe_layer* L, const float* hidden, size_t t,
                           int32_t norm_topk, float routed_scale, uint32_t* idx, float* gates, float* probs) {
    ENGINE_CTX(ctx);
    if (t > static_cast<size_t>(kMoeMaxT)) {
        // prefill-sized calls (moe.rs:181-243 routes every row of a chunk)
        if (!L) return fail(FOCR_HIP_E_BAD_HANDLE, "moe_route: null moe layer");
        if (!hidden) return fail(FOCR_HIP_E_ARG, "moe_route: null hidden");
        if (t > kRouteRowsMax)
            return fail(FOCR_HIP_E_SHAPE, fmt("moe_route: t %zu outside 1..=%zu for one call", t, kRouteRowsMax));
        if (!idx || !gates) return fail(FOCR_HIP_E_ARG, "moe_route: idx and gates are required above 64 rows");
        int* flag = static_cast<int*>(ctx->scratch_get(kScrFlag, t * sizeof(int)));
        if (!flag) return FOCR_HIP_E_OOM;
        int32_t st = route_rows_impl(ctx, L, hidden, t, norm_topk, routed_scale, idx, gates, probs, flag);
        if (st) return st;
        return check_route_flags(ctx, flag, t);
    }
    int32_t st = moe_checks("moe_route", L, hidden, t, 0);
    if (st) return st;
    MoeScratch s;
    ScratchSource src{ctx};
    if ((st = moe_scratch(src, L, t, false, &s))) return st;
    if ((st = launch_route(ctx, L, hidden, t, norm_topk, routed_scale, s, idx ? idx : s.idx, gates ? gates : s.gates,
                           probs, nullptr)))
        return st;
    FOCR_HIP_TRY(launch_route_epoch_bump(ctx->stream, s.xchg), "route epoch launch");
    return check_route_flags(ctx, s.flag, t);
}

}  // extern "C"

namespace {

// decode_mlp_i8 over t rows; with resid non-null, out = resid + the layer's
// output (the decode layer's residual, decoder.rs:2625). With static_scratch
// the intermediates are carved from the per-device static array instead of
// the context's slots, and nothing is allocated.
// norm: route rms_norm(hidden + norm->attn) * norm->w instead of hidden (the
// decoder layer's residual + post-attention norm, folded into the route
// kernel, which writes hidden + attn to norm->h_out; resid is then that).
int32_t moe_decode_impl(focr_hip_ctx* ctx, const focr_hip_moe_layer* L, const float* hidden, size_t t,
                        int32_t norm_topk, float routed_scale, int32_t with_shared, float* out, uint32_t* idx,
                        float* gates, int32_t check_route, const float* resid, bool static_scratch = false,
                        const MoeRouteNorm* norm = nullptr, size_t token_base = 0) {
    const char* name = static_scratch ? "moe_decode_noalloc" : "moe_decode";
    int32_t st = moe_checks(name, L, hidden, t, with_shared);
    if (st) return st;
    if (!out) return fail(FOCR_HIP_E_ARG, fmt("%s: null out", name));
    MoeScratch s;
    ScratchSource src{ctx};
    std::unique_ptr<StaticScratchOrder> order;
    if (static_scratch) {
        if (!ctx->static_scratch) ctx->static_scratch_err = static_scratch_init(ctx->device, &ctx->static_scratch);
        if (!ctx->static_scratch)
            return hip_fail(ctx->static_scratch_err != hipSuccess ? ctx->static_scratch_err : hipErrorInvalidSymbol,
                            "moe_decode_noalloc: static scratch address");
        ScratchSource count{ctx, nullptr, 0, 0, true};
        moe_scratch(count, L, t, with_shared != 0, &s);
        if (count.used > kStaticScratchBytes)
            return fail(FOCR_HIP_E_SHAPE, fmt("moe_decode_noalloc: t %zu needs %zu bytes of scratch; the static "
                                              "buffer holds %zu",
                                              t, count.used, kStaticScratchBytes));
        src = ScratchSource{ctx, static_cast<char*>(ctx->static_scratch), kStaticScratchBytes, 0, false};
        // every launch below is ordered after the device's previous call on
        // the array; this call's completion is recorded when `order` ends
        order = std::make_unique<StaticScratchOrder>(ctx->device, ctx->stream);
        if (order->err() != hipSuccess) return hip_fail(order->err(), "moe_decode_noalloc: order after the previous call");
    }
    if ((st = moe_scratch(src, L, t, with_shared != 0, &s))) return st;
    const MoeDims d{(int)t, (int)L->hidden, (int)L->inter, (int)L->n_experts, (int)L->top_k};
    uint32_t* di = idx ? idx : s.idx;
    float* dg = gates ? gates : s.gates;
    hipStream_t str = ctx->stream;
    if ((st = launch_route(ctx, L, hidden, t, norm_topk, routed_scale, s, di, dg, nullptr, s.sel, norm))) return st;
    hipError_t e = hipSuccess;
    {
        // the shared expert's gate/up rows ride in the same launch as extra blocks
        const MoeSharedGateUp shgu{L->swg, L->swu, L->ssg, L->ssu, s.shared_act, (int)L->shared_inter};
        ProfScope ps(ctx, "moe_gate_up");
        e = launch_moe_gate_up(str, d, s.sel, s.xq, s.xs, L->wg, L->sg, L->wu, L->su, s.act, (int)L->inter, false,
                               with_shared ? &shgu : nullptr, s.xchg);
        // the gate/up launch advances the route's counter; without it the next
        // call's route would take this call's records for its own
        if (e != hipSuccess) launch_route_epoch_bump(str, s.xchg);
    }
    if (e == hipSuccess && with_shared) {
        {
            // quantize_row_i8 of the act rows, then the int8 GEMV: the same
            // products, scales and rounding as the expert's down projection
            // (decoder.rs:1753-1754), with the GEMV's full-grid weight stream
            ProfScope ps(ctx, "moe_shared_down");
            const int SI = (int)L->shared_inter;
            const int rows = 57344 / SI < 32 ? 57344 / SI : 32;  // the GEMV's activation stage: m * k <= 56 KiB
            for (int r0 = 0; e == hipSuccess && r0 < (int)t; r0 += rows) {
                const int mr = (int)t - r0 < rows ? (int)t - r0 : rows;
                e = launch_gemv_i8_f32(str, L->swd, L->ssd, (int)L->hidden, SI, s.shared_act + (size_t)r0 * SI,
                                       nullptr, 0.0f, mr, s.shared_y + (size_t)r0 * L->hidden,
                                       s.shared_aq + (size_t)r0 * SI, s.shared_as + r0, ctx->cu_count);
            }
        }
    }
    if (e == hipSuccess && s.ybuf) {
        {
            ProfScope ps(ctx, "moe_down");
            e = launch_moe_down(str, d, s.sel, s.act, L->wd, L->sd, s.ybuf, (int)L->inter, false);
        }
        if (e == hipSuccess) {
            ProfScope ps(ctx, "moe_combine");
            e = launch_moe_combine(str, d, s.ybuf, s.flag, with_shared ? s.shared_y : nullptr, resid, out);
        }
    } else if (e == hipSuccess) {
        ProfScope ps(ctx, "moe_down_combine");
        e = launch_moe_down_combine(str, d, di, dg, s.flag, s.act, L->wd, L->sd, with_shared ? s.shared_y : nullptr,
                                    resid, out, (int)L->inter);
    }
    if (e != hipSuccess) return hip_fail(e, "moe_decode launch");
    if (check_route) return check_route_flags(ctx, s.flag, t, token_base);
    return FOCR_HIP_OK;
}

}  // namespace

extern "C" {

// Calls of more than kMoeMaxT rows run as consecutive chunks of kMoeMaxT
// (every token's routing and expert outputs are independent of the others',
// so the rows are the ones a single call would give).
constexpr size_t kMoeDecodeMaxT = 16384;
static int32_t moe_decode_chunked(focr_hip_ctx* ctx, const focr_hip_moe_layer* L, const float* hidden, size_t t,
                                  int32_t norm_topk, float routed_scale, int32_t with_shared, float* out,
                                  uint32_t* idx, float* gates, int32_t check_route, bool static_scratch) {
    if (t <= static_cast<size_t>(kMoeMaxT))
        return moe_decode_impl(ctx, L, hidden, t, norm_topk, routed_scale, with_shared, out, idx, gates, check_route,
                               nullptr, static_scratch);
    const char* name = static_scratch ? "moe_decode_noalloc" : "moe_decode";
    if (!L) return fail(FOCR_HIP_E_BAD_HANDLE, fmt("%s: null moe layer", name));
    if (!hidden || !out) return fail(FOCR_HIP_E_ARG, fmt("%s: null hidden or out", name));
    if (t > kMoeDecodeMaxT)
        return fail(FOCR_HIP_E_SHAPE, fmt("%s: t %zu outside 1..=%zu for one call", name, t, kMoeDecodeMaxT));
    const size_t H = L->hidden, K = L->top_k;
    for (size_t t0 = 0; t0 < t; t0 += kMoeMaxT) {
        const size_t n = std::min<size_t>(kMoeMaxT, t - t0);
        int32_t st = moe_decode_impl(ctx, L, hidden + t0 * H, n, norm_topk, routed_scale, with_shared, out + t0 * H,
                                     idx ? idx + t0 * K : nullptr, gates ? gates + t0 * K : nullptr, check_route,
                                     nullptr, static_scratch, nullptr, t0);
        if (st) return st;
    }
    return FOCR_HIP_OK;
}

int32_t focr_hip_moe_decode(focr_hip_ctx* ctx, const focr_hip_moe_layer* L, const float* hidden, size_t t,
                            int32_t norm_topk, float routed_scale, int32_t with_shared, float* out, uint32_t* idx,
                            float* gates, int32_t check_route) {
    ENGINE_CTX(ctx);
    return moe_decode_chunked(ctx, L, hidden, t, norm_topk, routed_scale, with_shared, out, idx, gates, check_route,
                              false);
}

int32_t focr_hip_moe_decode_noalloc(focr_hip_ctx* ctx, const focr_hip_moe_layer* L, const float* hidden, size_t t,
                                    int32_t norm_topk, float routed_scale, int32_t with_shared, float* out,
                                    uint32_t* idx, float* gates, int32_t check_route) {
    ENGINE_CTX(ctx);
    return moe_decode_impl(ctx, L, hidden, t, norm_topk, routed_scale, with_shared, out, idx, gates, check_route,
                           nullptr, true);
}

size_t focr_hip_static_scratch_bytes(void) { return kStaticScratchBytes; }

// ---- int4 MoE layer (chunked prefill) ------------------------------------------

}  // extern "C"

namespace {

void free_moe_i4(focr_hip_moe_layer_i4* L) {
    if (!L->owned) return;
    hipFree(L->wg);
    hipFree(L->wu);
    hipFree(L->wd);
    hipFree(L->sg);
    hipFree(L->su);
    hipFree(L->sd);
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

extern "C" {

int32_t focr_hip_moe_layer_i4_create(focr_hip_ctx* ctx, size_t hidden, size_t inter, size_t n_experts, size_t group,
                                     const uint8_t* wg, const float* sg, const uint8_t* wu, const float* su,
                                     const uint8_t* wd, const float* sd, int32_t from_device,
                                     focr_hip_moe_layer_i4** out) {
    ENGINE_CTX(ctx);
    if (!out) return fail(FOCR_HIP_E_ARG, "moe_layer_i4_create: null out");
    *out = nullptr;
    if (!wg || !sg || !wu || !su || !wd || !sd) return fail(FOCR_HIP_E_ARG, "moe_layer_i4_create: null pointer");
    if (group != 16 && group != 32)
        return fail(FOCR_HIP_E_SHAPE, fmt("igemm_s4s8_packed: group_size %zu must be 16 or 32", group));
    if (n_experts < 1 || n_experts > 64)
        return fail(FOCR_HIP_E_SHAPE, fmt("moe_layer_i4_create: gfx950 tier supports 1..=64 experts (got %zu)", n_experts));
    if (hidden % 32 || inter % 32 || hidden == 0 || inter == 0 || hidden > 4096 || inter > 4096)
        return fail(FOCR_HIP_E_SHAPE, fmt("moe_layer_i4_create: hidden/inter must be multiples of 32 in 32..=4096 "
                                          "(got %zu, %zu)", hidden, inter));
    if (from_device && (!aligned16(wg) || !aligned16(wu) || !aligned16(wd) || !aligned16(sg) || !aligned16(su) ||
                        !aligned16(sd)))
        return fail(FOCR_HIP_E_ARG, "moe_layer_i4_create: device arrays must be 16-byte aligned");
    // The layer always owns its weights, in the MFMA-tiled layout: the
    // reference-layout arrays (uploaded to staging, or the caller's device
    // arrays) are re-tiled once on the device.
    std::unique_ptr<focr_hip_moe_layer_i4> L(new focr_hip_moe_layer_i4());
    L->ctx = ctx;
    L->hidden = hidden;
    L->inter = inter;
    L->n_experts = n_experts;
    L->group = group;
    L->owned = true;
    const size_t E = n_experts;
    const size_t nb_gu = E * inter * (hidden / 2), ns_gu = E * inter * (hidden / group);
    const size_t nb_d = E * hidden * (inter / 2), ns_d = E * hidden * (inter / group);
    struct Src {
        const uint8_t* b;
        const float* s;
        size_t nb, ns;
        uint8_t** bt;
        float** st;
        int n, k;
    } srcs[3] = {{wg, sg, nb_gu, ns_gu, &L->wg, &L->sg, (int)inter, (int)hidden},
                 {wu, su, nb_gu, ns_gu, &L->wu, &L->su, (int)inter, (int)hidden},
                 {wd, sd, nb_d, ns_d, &L->wd, &L->sd, (int)hidden, (int)inter}};
    int32_t st = FOCR_HIP_OK;
    for (auto& m : srcs) {
        uint8_t* sb = nullptr;  // reference-layout source (staging copy, or the caller's array)
        float* ss = nullptr;
        st = upload(ctx, &sb, m.b, m.nb, from_device, "int4 weights");
        if (!st) st = upload(ctx, &ss, m.s, m.ns, from_device, "int4 scales");
        hipError_t e = hipSuccess;
        if (!st) e = hipMalloc(reinterpret_cast<void**>(m.bt), m.nb + s4_tile_pad_bytes());
        if (!st && e == hipSuccess)
            e = hipMalloc(reinterpret_cast<void**>(m.st), m.ns * sizeof(float) + s4_tile_pad_bytes());
        if (!st && e == hipSuccess)
            e = launch_retile_i4(ctx->stream, sb, ss, (int)E, m.n, m.k, (int)group, *m.bt, *m.st);
        hipStreamSynchronize(ctx->stream);
        if (!from_device) {
            hipFree(sb);
            hipFree(ss);
        }
        if (st || e != hipSuccess) {
            free_moe_i4(L.get());
            return st ? st : hip_fail(e, "moe_layer_i4_create retile");
        }
    }
    *out = L.release();
    return FOCR_HIP_OK;
}

int32_t focr_hip_moe_layer_i4_free(focr_hip_moe_layer_i4* L) {
    if (!L) return FOCR_HIP_OK;
    hipSetDevice(L->ctx->device);
    hipStreamSynchronize(L->ctx->stream);
    free_moe_i4(L);
    delete L;
    return FOCR_HIP_OK;
}

int32_t focr_hip_moe_prefill_i4(focr_hip_ctx* ctx, const focr_hip_moe_layer_i4* L, const float* x, size_t t,
                                size_t top_k, const uint32_t* idx, const float* gates, float* out,
                                int32_t check_idx) {
    ENGINE_CTX(ctx);
    if (!L) return fail(FOCR_HIP_E_BAD_HANDLE, "moe_prefill_i4: null moe layer");
    if (!x || !idx || !gates || !out) return fail(FOCR_HIP_E_ARG, "moe_prefill_i4: null pointer");
    if (top_k < 1 || top_k > 8) return fail(FOCR_HIP_E_SHAPE, fmt("moe_prefill_i4: top_k %zu outside 1..=8", top_k));
    if (t < 1 || t > 16384) return fail(FOCR_HIP_E_SHAPE, fmt("moe_prefill_i4: t %zu outside 1..=16384", t));
    const size_t H = L->hidden, I = L->inter, TK = t * top_k;
    MoeI4Scratch w;
    char* a = static_cast<char*>(ctx->scratch_get(kScrI4, TK * I * sizeof(float) + TK * H * sizeof(float)));
    char* b = static_cast<char*>(ctx->scratch_get(
        kScrI4b, t * H + 256 + t * 4 + 256 + TK * I + 256 + TK * 4 + 256 +
                     (moe_i4_plan_ints(static_cast<int>(TK), static_cast<int>(L->n_experts)) + 1) * sizeof(int)));
    if (!a || !b) return FOCR_HIP_E_OOM;
    auto take = [](char*& p, size_t bytes) {
        char* r = p;
        p += (bytes + 255) & ~static_cast<size_t>(255);
        return r;
    };
    w.act = reinterpret_cast<float*>(a);
    w.ybuf = reinterpret_cast<float*>(a + TK * I * sizeof(float));
    w.xq = reinterpret_cast<int8_t*>(take(b, t * H));
    w.xs = reinterpret_cast<float*>(take(b, t * 4));
    w.aq = reinterpret_cast<int8_t*>(take(b, TK * I));
    w.as = reinterpret_cast<float*>(take(b, TK * 4));
    w.plan = reinterpret_cast<int*>(b);
    w.err = w.plan + moe_i4_plan_ints(static_cast<int>(TK), static_cast<int>(L->n_experts));
    FOCR_HIP_TRY(launch_moe_prefill_i4(ctx->stream, L, x, static_cast<int>(t), static_cast<int>(top_k), idx, gates, out,
                                       w, ctx),
                 "moe_prefill_i4 launch");
    if (check_idx) {
        int err = 0;
        FOCR_HIP_TRY(hipMemcpyAsync(&err, w.err, sizeof(int), hipMemcpyDeviceToHost, ctx->stream), "D2H err");
        FOCR_HIP_TRY(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
        if (err)
            return fail(FOCR_HIP_E_SHAPE,
                        fmt("moe_prefill_i4: expert index out of range (n_experts %zu)", L->n_experts));
    }
    return FOCR_HIP_OK;
}

// ---- prefill: int8 linear and int8 MoE on the matrix cores ------------------------

}  // extern "C"

namespace {

// The fragment-ordered copy of n_mats [n][k] int8 matrices (launch_retile_i8),
// allocated and written on the context's stream the first time.
int32_t ensure_tiled(focr_hip_ctx* ctx, int8_t** dst, const int8_t* src, size_t n_mats, size_t n, size_t k,
                     const char* what) {
    if (*dst) return FOCR_HIP_OK;
    const size_t bytes = i8_tiled_bytes((int)n_mats, (int)n, (int)k);
    int8_t* p = nullptr;
    if (hipMalloc(&p, bytes) != hipSuccess)
        return fail(FOCR_HIP_E_OOM, fmt("%s: fragment-order copy of %zu bytes", what, bytes));
    hipError_t e = launch_retile_i8(ctx->stream, src, (int)n_mats, (int)n, (int)k, p);
    if (e != hipSuccess) {
        hipFree(p);
        return hip_fail(e, "retile launch");
    }
    *dst = p;
    return FOCR_HIP_OK;
}

}  // namespace

extern "C" {

// norm_w (nullable): x is first RMS-normalised with that weight and eps, in
// the quantize launch; only on the 256 x 128 tiled path (the caller checks
// linear_i8_norm_fusable)
static bool linear_i8_norm_fusable(const focr_hip_qint8* w, size_t m) {
    return w && !gemv_rows_preferred((int)w->n, (int)w->k, (int)m, false) &&
           i8_gemm256_supported((int)m, (int)w->n, (int)w->k) && w->k <= 4096;
}

// The activation layout linear_int8_dynamic quantizes x into (row-major, or
// the 256 x 128 GEMM's tiled order) and its bytes, in the kScrXq slot.
static bool linear_i8_act_tiled(const focr_hip_qint8* w, size_t m, const float* bias) {
    if (!bias && gemv_rows_preferred((int)w->n, (int)w->k, (int)m, false)) return false;
    return i8_gemm256_supported((int)m, (int)w->n, (int)w->k);
}
static size_t linear_i8_act_bytes(const focr_hip_qint8* w, size_t m, const float* bias) {
    return linear_i8_act_tiled(w, m, bias) ? i8_gemm256_a_bytes((int)m, (int)w->k) : m * w->k;
}

// prequant: the rows are already quantized by the dynamic rule in the
// kScrXq / kScrXs slots, in linear_i8_act_tiled's layout (x unused)
static int32_t linear_i8_dynamic_impl(focr_hip_ctx* ctx, const focr_hip_qint8* w, const float* x, size_t m,
                                   const float* bias, float* y, const float* norm_w = nullptr, float eps = 0.0f,
                                   bool prequant = false) {
    if (!w) return fail(FOCR_HIP_E_BAD_HANDLE, "linear_int8_dynamic: null weight handle");
    if ((!x && !prequant) || !y) return fail(FOCR_HIP_E_ARG, "linear_int8_dynamic: null device pointer");
    if (m < 1 || m > (1u << 20)) return fail(FOCR_HIP_E_SHAPE, fmt("linear_int8_dynamic: m %zu outside 1..=1048576", m));
    if (!i8_mfma_supported(static_cast<int>(w->k)))
        return fail(FOCR_HIP_E_SHAPE,
                    fmt("linear_int8_dynamic: k %zu is not a multiple of 64 (the matrix-core K stage)", w->k));
    // up to 256 rows without a bias, where it is the faster: the split-K GEMV
    // in 16-row groups on the upload layout (a prefill chunk's o_proj gets 10
    // blocks of the tiled GEMM at this size, (n / 16) x (m / 16) here)
    if (norm_w && !linear_i8_norm_fusable(w, m))
        return fail(FOCR_HIP_E_ARG, "linear_int8_dynamic: the fused norm needs the tiled path");
    if (!bias && gemv_rows_preferred((int)w->n, (int)w->k, (int)m, false)) {
        int8_t* xq = static_cast<int8_t*>(ctx->scratch_get(kScrXq, m * w->k));
        float* xs = static_cast<float*>(ctx->scratch_get(kScrXs, m * sizeof(float)));
        if (!xq || !xs) return FOCR_HIP_E_OOM;
        if (!prequant) {
            ProfScope ps(ctx, "quantize_rows_dyn");
            FOCR_HIP_TRY(launch_quantize_rows(ctx->stream, x, (int)m, (int)w->k, xq, xs, kQuantRuleDynamic),
                         "quantize launch");
        }
        ProfScope ps(ctx, "linear_i8");
        FOCR_HIP_TRY(launch_gemv_i8_rows(ctx->stream, w->w, w->scales, (int)w->n, (int)w->k, xq, xs, (int)m, y),
                     "linear_i8 launch");
        return FOCR_HIP_OK;
    }
    // 256 rows and up: 256 x 128 LDS-staged tiles on the tiled operands;
    // fewer: 64-row tiles on the fragment-order weight copy
    const bool big = i8_gemm256_supported((int)m, (int)w->n, (int)w->k);
    if (big) {
        if (!w->w_tiled) {
            const size_t bytes = i8_gemm256_b_bytes((int)w->n, (int)w->k);
            int8_t* p = nullptr;
            if (hipMalloc(&p, bytes) != hipSuccess)
                return fail(FOCR_HIP_E_OOM, fmt("linear_int8_dynamic: tiled weight copy of %zu bytes", bytes));
            hipError_t e = launch_i8_gemm256_retile_b(ctx->stream, w->w, (int)w->n, (int)w->k, p);
            if (e != hipSuccess) {
                hipFree(p);
                return hip_fail(e, "retile launch");
            }
            w->w_tiled = p;
        }
    } else {
        int32_t st = ensure_tiled(ctx, &w->w_mfma, w->w, 1, w->n, w->k, "linear_int8_dynamic");
        if (st) return st;
    }
    int8_t* xq = static_cast<int8_t*>(
        ctx->scratch_get(kScrXq, big ? i8_gemm256_a_bytes((int)m, (int)w->k) : m * w->k));
    float* xs = static_cast<float*>(ctx->scratch_get(kScrXs, m * sizeof(float)));
    if (!xq || !xs) return FOCR_HIP_E_OOM;
    if (!prequant) {
        ProfScope ps(ctx, "quantize_rows_dyn");
        if (big && norm_w)
            FOCR_HIP_TRY(launch_rms_norm_quantize_rows_tiled(ctx->stream, x, norm_w, eps, (int)m, (int)w->k, xq, xs,
                                                             kQuantRuleDynamic),
                         "norm + quantize launch");
        else if (big)
            FOCR_HIP_TRY(launch_quantize_rows_tiled(ctx->stream, x, (int)m, (int)w->k, xq, xs, kQuantRuleDynamic),
                         "quantize launch");
        else
            FOCR_HIP_TRY(launch_quantize_rows(ctx->stream, x, (int)m, (int)w->k, xq, xs, kQuantRuleDynamic),
                         "quantize launch");
    }
    ProfScope ps(ctx, "linear_i8");
    if (big)
        FOCR_HIP_TRY(launch_i8_gemm256(ctx->stream, xq, xs, (int)m, (int)w->k, w->w_tiled, w->scales, (int)w->n,
                                       bias, y),
                     "linear_i8 launch");
    else
        FOCR_HIP_TRY(launch_linear_i8(ctx->stream, xq, xs, (int)m, (int)w->k, w->w_mfma, w->scales, (int)w->n, bias,
                                      y),
                     "linear_i8 launch");
    return FOCR_HIP_OK;
}

int32_t focr_hip_linear_i8_dynamic(focr_hip_ctx* ctx, const focr_hip_qint8* w, const float* x, size_t m,
                                   const float* bias, float* y) {
    ENGINE_CTX(ctx);
    return linear_i8_dynamic_impl(ctx, w, x, m, bias, y);
}

// resid non-null: out = resid + the block's output (the decoder layer's
// residual, added in the combine)
static int32_t moe_prefill_i8_impl(focr_hip_ctx* ctx, const focr_hip_moe_layer* L, const float* x, size_t t,
                                const uint32_t* idx, const float* gates, int32_t with_shared, float* out,
                                int32_t check_idx, const float* resid = nullptr) {
    if (!L) return fail(FOCR_HIP_E_BAD_HANDLE, "moe_prefill_i8: null moe layer");
    if (!x || !idx || !gates || !out) return fail(FOCR_HIP_E_ARG, "moe_prefill_i8: null pointer");
    if (t < 1 || t > 16384) return fail(FOCR_HIP_E_SHAPE, fmt("moe_prefill_i8: t %zu outside 1..=16384", t));
    if (with_shared && !L->swg)
        return fail(FOCR_HIP_E_ARG, "moe_prefill_i8: with_shared set but no shared expert uploaded");
    const size_t H = L->hidden, I = L->inter, K = L->top_k, TK = t * K;
    if (!i8_mfma_supported((int)H) || !i8_mfma_supported((int)I) ||
        (with_shared && !i8_mfma_supported((int)L->shared_inter)))
        return fail(FOCR_HIP_E_SHAPE,
                    fmt("moe_prefill_i8: hidden %zu / inter %zu must be multiples of 64 (the matrix-core K stage)", H,
                        I));
    int32_t st;
    const size_t E = L->n_experts;
    if ((st = ensure_tiled(ctx, &L->wg_mfma, L->wg, E, I, H, "moe_prefill_i8")) ||
        (st = ensure_tiled(ctx, &L->wu_mfma, L->wu, E, I, H, "moe_prefill_i8")) ||
        (st = ensure_tiled(ctx, &L->wd_mfma, L->wd, E, H, I, "moe_prefill_i8")))
        return st;
    if (with_shared) {
        const size_t S = L->shared_inter;
        if ((st = ensure_tiled(ctx, &L->swg_mfma, L->swg, 1, S, H, "moe_prefill_i8")) ||
            (st = ensure_tiled(ctx, &L->swu_mfma, L->swu, 1, S, H, "moe_prefill_i8")) ||
            (st = ensure_tiled(ctx, &L->swd_mfma, L->swd, 1, H, S, "moe_prefill_i8")))
            return st;
    }
    auto take = [](char*& p, size_t bytes) {
        char* r = p;
        p += (bytes + 255) & ~static_cast<size_t>(255);
        return r;
    };
    MoeI8Scratch w{};
    char* a = static_cast<char*>(ctx->scratch_get(kScrI4, TK * I * sizeof(float) + 256 + TK * H * sizeof(float)));
    char* b = static_cast<char*>(ctx->scratch_get(
        kScrI4b, t * H + 256 + t * 4 + 256 + TK * I + 256 + TK * 4 + 256 +
                     (moe_i4_plan_ints(static_cast<int>(TK), static_cast<int>(L->n_experts)) + 1) * sizeof(int)));
    const size_t SI = with_shared ? L->shared_inter : 0;
    char* c = with_shared ? static_cast<char*>(ctx->scratch_get(
                                kScrShared, t * SI * 4 + 256 + t * SI + 256 + t * 4 + 256 + t * H * 4))
                          : nullptr;
    if (!a || !b || (with_shared && !c)) return FOCR_HIP_E_OOM;
    w.act = reinterpret_cast<float*>(take(a, TK * I * sizeof(float)));
    w.ybuf = reinterpret_cast<float*>(a);
    w.xq = reinterpret_cast<int8_t*>(take(b, t * H));
    w.xs = reinterpret_cast<float*>(take(b, t * 4));
    w.aq = reinterpret_cast<int8_t*>(take(b, TK * I));
    w.as = reinterpret_cast<float*>(take(b, TK * 4));
    w.plan = reinterpret_cast<int*>(b);
    w.err = w.plan + moe_i4_plan_ints(static_cast<int>(TK), static_cast<int>(L->n_experts));
    if (c) {
        w.shared_act = reinterpret_cast<float*>(take(c, t * SI * 4));
        w.shared_aq = reinterpret_cast<int8_t*>(take(c, t * SI));
        w.shared_as = reinterpret_cast<float*>(take(c, t * 4));
        w.shared_y = reinterpret_cast<float*>(c);
    }
    FOCR_HIP_TRY(launch_moe_prefill_i8(ctx->stream, L, x, static_cast<int>(t), static_cast<int>(K), idx, gates,
                                       with_shared, out, w, ctx, resid),
                 "moe_prefill_i8 launch");
    if (check_idx) {
        int err = 0;
        FOCR_HIP_TRY(hipMemcpyAsync(&err, w.err, sizeof(int), hipMemcpyDeviceToHost, ctx->stream), "D2H err");
        FOCR_HIP_TRY(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
        if (err)
            return fail(FOCR_HIP_E_SHAPE,
                        fmt("moe_prefill_i8: expert index out of range (n_experts %zu)", L->n_experts));
    }
    return FOCR_HIP_OK;
}

int32_t focr_hip_moe_prefill_i8(focr_hip_ctx* ctx, const focr_hip_moe_layer* L, const float* x, size_t t,
                                const uint32_t* idx, const float* gates, int32_t with_shared, float* out,
                                int32_t check_idx) {
    ENGINE_CTX(ctx);
    return moe_prefill_i8_impl(ctx, L, x, t, idx, gates, with_shared, out, check_idx);
}

// ---- R-SWA --------------------------------------------------------------------

int32_t focr_hip_rswa_create(focr_hip_ctx* ctx, size_t n_streams, size_t ref_capacity, focr_hip_rswa** out) {
    ENGINE_CTX(ctx);
    if (!out) return fail(FOCR_HIP_E_ARG, "rswa_create: null out");
    *out = nullptr;
    if (n_streams == 0) return fail(FOCR_HIP_E_SHAPE, "rswa: batched cache needs at least one stream");
    if (ref_capacity > (1u << 20)) return fail(FOCR_HIP_E_SHAPE, "rswa: ref_capacity exceeds the gfx950 tier limit");
    std::unique_ptr<focr_hip_rswa> c(new focr_hip_rswa());
    c->ctx = ctx;
    c->n_streams = n_streams;
    c->ref_capacity = ref_capacity;
    c->prefill_len.assign(n_streams, -1);
    c->ring_len.assign(n_streams, 0);
    c->ring_pos.assign(n_streams, 0);
    const size_t bytes = n_streams * c->stream_floats() * sizeof(float);
    FOCR_HIP_TRY(hipMalloc(reinterpret_cast<void**>(&c->base), bytes), "hipMalloc rswa");
    FOCR_HIP_TRY(hipMemsetAsync(c->base, 0, bytes, ctx->stream), "hipMemsetAsync rswa");
    FOCR_HIP_TRY(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
    *out = c.release();
    return FOCR_HIP_OK;
}

int32_t focr_hip_rswa_free(focr_hip_rswa* c) {
    if (!c) return FOCR_HIP_OK;
    hipSetDevice(c->ctx->device);
    hipStreamSynchronize(c->ctx->stream);
    hipFree(c->base);
    delete c;
    return FOCR_HIP_OK;
}

int32_t focr_hip_rswa_record_prefill(focr_hip_ctx* ctx, focr_hip_rswa* c, size_t stream, const float* k,
                                     const float* v, size_t seq) {
    ENGINE_CTX(ctx);
    if (!c) return fail(FOCR_HIP_E_BAD_HANDLE, "null rswa cache");
    if (stream >= c->n_streams) return fail(FOCR_HIP_E_SHAPE, fmt("rswa: stream %zu >= num_streams %zu", stream, c->n_streams));
    if (seq > c->ref_capacity)
        return fail(FOCR_HIP_E_STATE, fmt("rswa: prefill seq %zu exceeds ref_capacity %zu", seq, c->ref_capacity));
    if (seq && (!k || !v)) return fail(FOCR_HIP_E_ARG, "rswa_record_prefill: null device pointer");
    // head-major [10][seq][128] -> region rows [h][0..seq)
    const size_t row = static_cast<size_t>(kHeadDim) * sizeof(float);
    if (seq) {
        FOCR_HIP_TRY(hipMemcpy2DAsync(c->ref_k(stream), c->ref_capacity * row, k, seq * row, seq * row, kNumHeads,
                                      hipMemcpyDeviceToDevice, ctx->stream),
                     "copy prefill k");
        FOCR_HIP_TRY(hipMemcpy2DAsync(c->ref_v(stream), c->ref_capacity * row, v, seq * row, seq * row, kNumHeads,
                                      hipMemcpyDeviceToDevice, ctx->stream),
                     "copy prefill v");
    }
    c->prefill_len[stream] = static_cast<int64_t>(seq);
    c->ring_len[stream] = 0;
    c->ring_pos[stream] = 0;
    return FOCR_HIP_OK;
}

}  // extern "C"

namespace {

// rswa.rs:467-494: the slot one stream's next K/V row goes to, and the
// cursor update after it is written. Callers take the slots first and advance
// the cursors only once the launch that writes the rows has been accepted, so
// a failed step leaves the ring as it was.
uint32_t peek_slot(const focr_hip_rswa* c, size_t s) {
    return c->ring_len[s] < static_cast<uint32_t>(kRingWindow) ? c->ring_len[s] : c->ring_pos[s];
}

void advance_slot(focr_hip_rswa* c, size_t s) {
    if (c->ring_len[s] < static_cast<uint32_t>(kRingWindow)) {
        c->ring_len[s] += 1;
        c->ring_pos[s] = c->ring_len[s] % kRingWindow;
    } else {
        c->ring_pos[s] = (c->ring_pos[s] + 1) % kRingWindow;
    }
}

int32_t rswa_write_all(focr_hip_ctx* ctx, focr_hip_rswa* c, const float* k_steps, const float* v_steps,
                       uint32_t* slots) {
    for (size_t s = 0; s < c->n_streams; ++s)
        if (c->prefill_len[s] < 0) return fail(FOCR_HIP_E_STATE, "rswa: write_decode_step before record_prefill");
    if (!k_steps || !v_steps) return fail(FOCR_HIP_E_ARG, "rswa_write_decode_step: null device pointer");
    for (size_t s0 = 0; s0 < c->n_streams; s0 += RswaStepArgs::kMax) {
        RswaStepArgs a{};
        a.n = static_cast<uint32_t>(std::min<size_t>(RswaStepArgs::kMax, c->n_streams - s0));
        for (uint32_t i = 0; i < a.n; ++i) {
            a.slot[i] = peek_slot(c, s0 + i);
            if (slots) slots[s0 + i] = a.slot[i];
        }
        const size_t off = s0 * kNumHeads * kHeadDim;
        ProfScope ps(ctx, "rswa_write");
        FOCR_HIP_TRY(launch_rswa_write(ctx->stream, c, s0, a, k_steps + off, v_steps + off), "ring write launch");
        for (uint32_t i = 0; i < a.n; ++i) advance_slot(c, s0 + i);
    }
    return FOCR_HIP_OK;
}

int32_t rswa_attend_all(focr_hip_ctx* ctx, const focr_hip_rswa* c, const float* q, float* out) {
    for (size_t s = 0; s < c->n_streams; ++s) {
        if (c->prefill_len[s] < 0) return fail(FOCR_HIP_E_STATE, "rswa: decode_attention before record_prefill");
        if (c->prefill_len[s] + c->ring_len[s] == 0)
            return fail(FOCR_HIP_E_STATE, "rswa: empty attention key set (prefill_len=0, ring_len=0)");
    }
    if (!q || !out) return fail(FOCR_HIP_E_ARG, "rswa_decode_attention: null device pointer");
    const size_t chunk_streams = std::min<size_t>(RswaStepArgs::kMax, c->n_streams);
    float* partials = static_cast<float*>(
        ctx->scratch_get(kScrRswa, rswa_partials_bytes(chunk_streams, c->ref_capacity + kRingWindow)));
    if (!partials) return FOCR_HIP_E_OOM;
    for (size_t s0 = 0; s0 < c->n_streams; s0 += RswaStepArgs::kMax) {
        RswaStepArgs a{};
        a.n = static_cast<uint32_t>(std::min<size_t>(RswaStepArgs::kMax, c->n_streams - s0));
        for (uint32_t i = 0; i < a.n; ++i) {
            a.prefill_len[i] = static_cast<uint32_t>(c->prefill_len[s0 + i]);
            a.ring_len[i] = c->ring_len[s0 + i];
        }
        const size_t off = s0 * kNumHeads * kHeadDim;
        FOCR_HIP_TRY(launch_rswa_attention(ctx->stream, c, s0, a, q + off, out + off, partials, ctx->cu_count, ctx),
                     "attention launch");
    }
    return FOCR_HIP_OK;
}

}  // namespace

extern "C" {

int32_t focr_hip_rswa_write_decode_step(focr_hip_ctx* ctx, focr_hip_rswa* c, const float* k_steps,
                                        const float* v_steps, uint32_t* slots) {
    ENGINE_CTX(ctx);
    if (!c) return fail(FOCR_HIP_E_BAD_HANDLE, "null rswa cache");
    return rswa_write_all(ctx, c, k_steps, v_steps, slots);
}

int32_t focr_hip_rswa_decode_attention(focr_hip_ctx* ctx, const focr_hip_rswa* c, const float* q, float* out) {
    ENGINE_CTX(ctx);
    if (!c) return fail(FOCR_HIP_E_BAD_HANDLE, "null rswa cache");
    return rswa_attend_all(ctx, c, q, out);
}

int32_t focr_hip_rswa_step(focr_hip_ctx* ctx, focr_hip_rswa* c, const float* q, const float* k_steps,
                           const float* v_steps, float* out) {
    ENGINE_CTX(ctx);
    if (!c) return fail(FOCR_HIP_E_BAD_HANDLE, "null rswa cache");
    int32_t st = rswa_write_all(ctx, c, k_steps, v_steps, nullptr);
    if (st) return st;
    return rswa_attend_all(ctx, c, q, out);
}

// ---- one decoder layer's decode step (decoder.rs:2542-2627, :2812-2933) --------

int32_t focr_hip_rms_norm(focr_hip_ctx* ctx, const float* x, size_t rows, size_t n, const float* w, float eps,
                          float* y) {
    ENGINE_CTX(ctx);
    if (rows == 0) return FOCR_HIP_OK;
    if (!x || !y) return fail(FOCR_HIP_E_ARG, "rms_norm: null device pointer");
    if (n == 0 || n > 4096 || rows > (1u << 20)) return fail(FOCR_HIP_E_SHAPE, fmt("rms_norm: cols %zu outside 1..=4096", n));
    ProfScope ps(ctx, "rms_norm");
    FOCR_HIP_TRY(launch_rms_norm(ctx->stream, x, w, (int)rows, (int)n, eps, y), "rms_norm launch");
    return FOCR_HIP_OK;
}

int32_t focr_hip_decoder_layer_create(focr_hip_ctx* ctx, size_t hidden, size_t n_heads, size_t head_dim,
                                      const float* input_ln, const float* post_attn_ln, const focr_hip_qint8* qkv,
                                      const focr_hip_qint8* o_proj, const focr_hip_moe_layer* moe,
                                      const focr_hip_qint8* dense_gate, const focr_hip_qint8* dense_up,
                                      const focr_hip_qint8* dense_down, float rms_eps, float rope_theta,
                                      focr_hip_decoder_layer** out) {
    ENGINE_CTX(ctx);
    if (!out) return fail(FOCR_HIP_E_ARG, "decoder_layer_create: null out");
    *out = nullptr;
    if (!input_ln || !post_attn_ln || !qkv || !o_proj)
        return fail(FOCR_HIP_E_ARG, "decoder_layer_create: null norm weight or projection");
    const bool dense = dense_gate || dense_up || dense_down;
    if ((moe != nullptr) == dense || (dense && !(dense_gate && dense_up && dense_down)))
        return fail(FOCR_HIP_E_ARG, "decoder_layer_create: exactly one of moe or (dense_gate, dense_up, dense_down)");
    const size_t D = n_heads * head_dim;
    if (hidden == 0 || hidden > 4096 || hidden % 64 || head_dim % 2 || D == 0 || D % 16 ||
        qkv->n != 3 * D || qkv->k != hidden || o_proj->n != hidden || o_proj->k != D)
        return fail(FOCR_HIP_E_SHAPE, fmt("decoder_layer_create: qkv [%zu, %zu] / o_proj [%zu, %zu] do not match "
                                          "hidden %zu, heads %zu x %zu",
                                          qkv->n, qkv->k, o_proj->n, o_proj->k, hidden, n_heads, head_dim));
    if (moe && moe->hidden != hidden)
        return fail(FOCR_HIP_E_SHAPE, fmt("decoder_layer_create: moe hidden %zu != %zu", moe->hidden, hidden));
    if (dense && (dense_gate->k != hidden || dense_up->k != hidden || dense_up->n != dense_gate->n ||
                  dense_down->n != hidden || dense_down->k != dense_gate->n))
        return fail(FOCR_HIP_E_SHAPE, "decoder_layer_create: dense gate/up [i, hidden], down [hidden, i] expected");
    auto* L = new focr_hip_decoder_layer();
    L->ctx = ctx;
    L->hidden = hidden;
    L->n_heads = n_heads;
    L->head_dim = head_dim;
    L->eps = rms_eps;
    L->qkv = qkv;
    L->o_proj = o_proj;
    L->moe = moe;
    L->gate = dense_gate;
    L->up = dense_up;
    L->down = dense_down;
    // RopeTable::build's table (decoder.rs:197-205): f64 pow, narrowed to f32
    std::vector<float> inv(head_dim / 2);
    for (size_t i = 0; i < inv.size(); ++i)
        inv[i] = static_cast<float>(1.0 / std::pow(static_cast<double>(rope_theta),
                                                   static_cast<double>(2 * i) / static_cast<double>(head_dim)));
    hipError_t e = hipMalloc(&L->input_ln, hidden * sizeof(float));
    if (e == hipSuccess) e = hipMalloc(&L->post_ln, hidden * sizeof(float));
    if (e == hipSuccess) e = hipMalloc(&L->inv_freq, inv.size() * sizeof(float));
    if (e == hipSuccess) e = hipMemcpy(L->input_ln, input_ln, hidden * sizeof(float), hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(L->post_ln, post_attn_ln, hidden * sizeof(float), hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(L->inv_freq, inv.data(), inv.size() * sizeof(float), hipMemcpyHostToDevice);
    // the qkv weights in RoPE pair order for the GEMV with the RoPE epilogue
    const size_t qn = qkv->n, qk = qkv->k;
    if (e == hipSuccess) e = hipMalloc(&L->qkv_rope_w, qn * qk);
    if (e == hipSuccess) e = hipMalloc(&L->qkv_rope_s, qn * sizeof(float));
    if (e == hipSuccess)
        e = launch_permute_rows_i8(ctx->stream, qkv->w, qkv->scales, (int)qn, (int)qk, (int)(n_heads * head_dim),
                                   (int)head_dim, L->qkv_rope_w, L->qkv_rope_s);
    if (dense) {
        // gate rows then up rows, so one GEMV launch computes both
        const size_t gi = dense_gate->n, gh = dense_gate->k;
        if (e == hipSuccess) e = hipMalloc(&L->gate_up_w, 2 * gi * gh);
        if (e == hipSuccess) e = hipMalloc(&L->gate_up_s, 2 * gi * sizeof(float));
        if (e == hipSuccess)
            e = hipMemcpyAsync(L->gate_up_w, dense_gate->w, gi * gh, hipMemcpyDeviceToDevice, ctx->stream);
        if (e == hipSuccess)
            e = hipMemcpyAsync(L->gate_up_w + gi * gh, dense_up->w, gi * gh, hipMemcpyDeviceToDevice, ctx->stream);
        if (e == hipSuccess)
            e = hipMemcpyAsync(L->gate_up_s, dense_gate->scales, gi * sizeof(float), hipMemcpyDeviceToDevice,
                               ctx->stream);
        if (e == hipSuccess)
            e = hipMemcpyAsync(L->gate_up_s + gi, dense_up->scales, gi * sizeof(float), hipMemcpyDeviceToDevice,
                               ctx->stream);
    }
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) {
        hipFree(L->input_ln);
        hipFree(L->post_ln);
        hipFree(L->inv_freq);
        hipFree(L->qkv_rope_w);
        hipFree(L->qkv_rope_s);
        hipFree(L->gate_up_w);
        hipFree(L->gate_up_s);
        delete L;
        return hip_fail(e, "decoder_layer_create upload");
    }
    *out = L;
    return FOCR_HIP_OK;
}

int32_t focr_hip_decoder_layer_free(focr_hip_decoder_layer* L) {
    if (!L) return FOCR_HIP_OK;
    hipSetDevice(L->ctx->device);
    hipStreamSynchronize(L->ctx->stream);
    hipFree(L->input_ln);
    hipFree(L->post_ln);
    hipFree(L->inv_freq);
    hipFree(L->qkv_rope_w);
    hipFree(L->qkv_rope_s);
    hipFree(L->gate_up_w);
    hipFree(L->gate_up_s);
    delete L;
    return FOCR_HIP_OK;
}

static int32_t decoder_layer_step_impl(focr_hip_ctx* ctx, const focr_hip_decoder_layer* L, focr_hip_rswa* cache,
                                    const uint32_t* positions, float* x, uint32_t* route_idx, int32_t check_route) {
    if (!L) return fail(FOCR_HIP_E_BAD_HANDLE, "decoder_layer_step: null layer");
    if (!cache) return fail(FOCR_HIP_E_BAD_HANDLE, "decoder_layer_step: null rswa cache");
    if (!positions || !x) return fail(FOCR_HIP_E_ARG, "decoder_layer_step: null positions or x");
    const size_t B = cache->n_streams, H = L->hidden, D = L->n_heads * L->head_dim;
    if (L->n_heads != 10 || L->head_dim != 128)
        return fail(FOCR_HIP_E_SHAPE, "decoder_layer_step: the R-SWA cache holds 10 heads x 128");
    const size_t max_b = L->gate ? std::min<size_t>(32, 57344 / L->gate->n) : 32;
    if (B < 1) return fail(FOCR_HIP_E_SHAPE, "decoder_layer_step: no streams");
    if (B > max_b) {
        // more streams than one pass takes: groups of max_b streams, each
        // through a view of the cache that holds just its streams' regions
        // and cursors (every stream's step is independent of the others')
        for (size_t s0 = 0; s0 < B; s0 += max_b) {
            const size_t n = std::min(max_b, B - s0);
            focr_hip_rswa view;
            view.ctx = cache->ctx;
            view.n_streams = n;
            view.ref_capacity = cache->ref_capacity;
            view.base = cache->ref_k(s0);
            view.prefill_len.assign(cache->prefill_len.begin() + s0, cache->prefill_len.begin() + s0 + n);
            view.ring_len.assign(cache->ring_len.begin() + s0, cache->ring_len.begin() + s0 + n);
            view.ring_pos.assign(cache->ring_pos.begin() + s0, cache->ring_pos.begin() + s0 + n);
            const size_t K = L->moe ? L->moe->top_k : 0;
            int32_t st = decoder_layer_step_impl(ctx, L, &view, positions + s0, x + s0 * H,
                                                 route_idx ? route_idx + s0 * K : nullptr, check_route);
            // the cursors the group's launches were made with (the step's
            // launches are issued; the ring slots advance with them)
            std::copy(view.ring_len.begin(), view.ring_len.end(), cache->ring_len.begin() + s0);
            std::copy(view.ring_pos.begin(), view.ring_pos.end(), cache->ring_pos.begin() + s0);
            if (st) return st;
        }
        return FOCR_HIP_OK;
    }
    const size_t I = L->gate ? L->gate->n : 0;
    // one scratch slot carved into the step's intermediates
    const size_t fl = B * (3 * D + D + D + H + H + H) + (L->gate ? 3 * B * I : 0);
    char* base = static_cast<char*>(ctx->scratch_get(kScrLayer, fl * 4 + B * H + B * I + 16 * 256));
    if (!base) return FOCR_HIP_E_OOM;
    auto take = [&](size_t bytes) {
        char* r = base;
        base += (bytes + 255) & ~static_cast<size_t>(255);
        return r;
    };
    float* qkv = reinterpret_cast<float*>(take(B * 3 * D * 4));
    float* q = reinterpret_cast<float*>(take(B * D * 4));
    float* cx = reinterpret_cast<float*>(take(B * D * 4));
    float* attn = reinterpret_cast<float*>(take(B * H * 4));
    float* h = reinterpret_cast<float*>(take(B * H * 4));
    float* nrm = reinterpret_cast<float*>(take(B * H * 4));
    int8_t* xq = reinterpret_cast<int8_t*>(take(B * (H > D ? H : D)));
    float* xs = reinterpret_cast<float*>(take(B * 4));
    hipStream_t s = ctx->stream;
    // 1. input RMSNorm + quantize_row_i8, 2. the fused qkv GEMV, 3. RoPE at
    //    each stream's position and the ring write: k and v go straight to
    //    each stream's next ring slot (the cursors advance as
    //    rswa_write_all's do, once that launch is accepted). One launch (blocks norm and quantize the rows
    //    themselves, the epilogue rotates and scatters) where the shape
    //    allows, else the GEMV and the RoPE kernel.
    {
        RopePositions rp{};
        for (size_t i = 0; i < B; ++i) rp.p[i] = positions[i];
        for (size_t i = 0; i < B; ++i)
            if (cache->prefill_len[i] < 0) return fail(FOCR_HIP_E_STATE, "rswa: write_decode_step before record_prefill");
        RopeRing ring{};
        ring.head_stride = static_cast<size_t>(kRingWindow) * kHeadDim;
        for (size_t i = 0; i < B; ++i) {
            const uint32_t slot = peek_slot(cache, i);
            ring.k[i] = cache->ring_k(i) + static_cast<size_t>(slot) * kHeadDim;
            ring.v[i] = cache->ring_v(i) + static_cast<size_t>(slot) * kHeadDim;
        }
        hipError_t qe = hipErrorNotSupported;
        if (L->qkv_rope_w) {
            ProfScope ps(ctx, "layer_qkv_rope");
            const RopeEpi epi{L->inv_freq, rp, ring, q, (int)D, (int)L->head_dim, 0};
            qe = launch_qkv_rope_f32(s, L->qkv_rope_w, L->qkv_rope_s, (int)(3 * D), (int)H, x, L->input_ln, L->eps,
                                     (int)B, epi, ctx->cu_count);
            if (qe != hipErrorNotSupported) FOCR_HIP_TRY(qe, "qkv rope launch");
        }
        if (qe == hipErrorNotSupported) {
            {
                ProfScope ps(ctx, "layer_qkv");
                FOCR_HIP_TRY(launch_gemv_i8_f32(s, L->qkv->w, L->qkv->scales, (int)(3 * D), (int)H, x, L->input_ln,
                                                L->eps, (int)B, qkv, xq, xs, ctx->cu_count),
                             "qkv gemv launch");
            }
            ProfScope ps(ctx, "layer_rope");
            FOCR_HIP_TRY(launch_rope_split(s, qkv, rp, L->inv_freq, (int)B, (int)L->n_heads, (int)L->head_dim, q,
                                           nullptr, nullptr, &ring),
                         "rope launch");
        }
        for (size_t i = 0; i < B; ++i) advance_slot(cache, i);  // k and v are in their slots
    }
    int32_t st = rswa_attend_all(ctx, cache, q, cx);
    if (st) return st;
    // 4. quantize_row_i8 of the contexts + o_proj (one launch); 5. residual +
    //    post-attention RMSNorm
    {
        ProfScope ps(ctx, "layer_o_proj");
        FOCR_HIP_TRY(launch_gemv_i8_f32(s, L->o_proj->w, L->o_proj->scales, (int)H, (int)D, cx, nullptr, 0.0f, (int)B,
                                        attn, xq, xs, ctx->cu_count),
                     "o_proj gemv launch");
    }
    // 6. decode_mlp_i8 (decoder.rs:2199-2268) and the residual
    if (L->moe && H <= 1280) {
        // route_default (moe.rs:53-76: norm_topk_prob false, scaling 1.0) + the shared expert; the
        // route kernel computes h = x + attn and routes rms_norm(h) * post_ln itself
        const MoeRouteNorm rn{attn, L->post_ln, L->eps, h};
        return moe_decode_impl(ctx, L->moe, x, B, 0, 1.0f, L->moe->swg ? 1 : 0, x, route_idx, nullptr, check_route,
                               h, false, &rn);
    }
    // dense (layer 0) in three launches where the shapes allow: the residual,
    // the post-attention norm, quantize, the gate and up GEMVs and SiLU(g) * u
    // in one (h = x + attn stored by it); quantize_row_i8 of act; the down
    // GEMV with the residual add in its epilogue (x = h + down(act))
    const int cu = ctx->cu_count > 0 ? ctx->cu_count : 256;
    if (!L->moe && L->gate_up_w && B >= 2 && H % 64 == 0 && H <= 1280 && I % 64 == 0 && I <= 8192 &&
        (I + 15) / 16 < static_cast<size_t>(4 * cu) && (H + 15) / 16 < static_cast<size_t>(4 * cu)) {
        float* act = reinterpret_cast<float*>(take(B * I * 4));
        int8_t* aq = reinterpret_cast<int8_t*>(take(B * I));
        ProfScope ps(ctx, "layer_dense_mlp");
        FOCR_HIP_TRY(launch_swiglu_i8_f32_add(s, L->gate_up_w, L->gate_up_s, (int)I, (int)H, x, attn, h, L->post_ln,
                                              L->eps, (int)B, act, ctx->cu_count),
                     "dense residual + norm + gate/up + silu launch");
        FOCR_HIP_TRY(launch_quantize_rows(s, act, (int)B, (int)I, aq, xs, 0), "dense quantize launch");
        FOCR_HIP_TRY(launch_gemv_i8_resid(s, L->down->w, L->down->scales, (int)H, (int)I, aq, xs, (int)B, h, x,
                                          ctx->cu_count),
                     "dense down + residual launch");
        return FOCR_HIP_OK;
    }
    {
        ProfScope ps(ctx, "layer_residual_norm");
        FOCR_HIP_TRY(launch_residual_rms_norm(s, x, attn, L->post_ln, (int)B, (int)H, L->eps, h, nrm),
                     "residual rms_norm launch");
    }
    if (L->moe)
        return moe_decode_impl(ctx, L->moe, nrm, B, 0, 1.0f, L->moe->swg ? 1 : 0, x, route_idx, nullptr, check_route,
                               h);
    // dense (layer 0): expert_gemv_i8 (decoder.rs:1711-1720)
    float* g = reinterpret_cast<float*>(take(B * I * 4));
    float* u = reinterpret_cast<float*>(take(B * I * 4));
    float* act = reinterpret_cast<float*>(take(B * I * 4));
    int8_t* aq = reinterpret_cast<int8_t*>(take(B * I));
    ProfScope ps(ctx, "layer_dense_mlp");
    FOCR_HIP_TRY(launch_gemv_i8_f32(s, L->gate->w, L->gate->scales, (int)I, (int)H, nrm, nullptr, 0.0f, (int)B, g,
                                    xq, xs, ctx->cu_count),
                 "dense gate launch");
    FOCR_HIP_TRY(launch_gemv_i8_f32(s, L->up->w, L->up->scales, (int)I, (int)H, nrm, nullptr, 0.0f, (int)B, u, xq,
                                    xs, ctx->cu_count),
                 "dense up launch");
    FOCR_HIP_TRY(launch_silu_mul(s, g, u, act, B * I), "silu launch");
    FOCR_HIP_TRY(launch_gemv_i8_f32(s, L->down->w, L->down->scales, (int)H, (int)I, act, nullptr, 0.0f, (int)B, attn,
                                    aq, xs, ctx->cu_count),
                 "dense down launch");
    FOCR_HIP_TRY(launch_add_rows(s, h, attn, x, B * H), "residual launch");
    return FOCR_HIP_OK;
}

int32_t focr_hip_decoder_layer_step(focr_hip_ctx* ctx, const focr_hip_decoder_layer* L, focr_hip_rswa* cache,
                                    const uint32_t* positions, float* x, uint32_t* route_idx, int32_t check_route) {
    ENGINE_CTX(ctx);
    return decoder_layer_step_impl(ctx, L, cache, positions, x, route_idx, check_route);
}

// ---- prefill attention (decoder.rs:568-640, :1282-1340) ------------------------

}  // extern "C"

namespace {

// The shared body: causal attention of cs queries (positions c0 ..) over a
// c1-key prefix, geometry as AttnGeom, on the context's stream.
int32_t attn_run(focr_hip_ctx* ctx, const char* name, const AttnGeom& gm, const float* q, const float* k,
                 const float* v, float* out, size_t cs, size_t c0, size_t c1, size_t heads,
                 AttnQuantOut* qo = nullptr) {
    int split_len = 0;
    const int nsplit = attn_pick_splits((int)cs, (int)c1, (int)heads, ctx->cu_count, &split_len);
    float* part = nullptr;
    if (nsplit > 1) {
        part = static_cast<float*>(ctx->scratch_get(kScrAttn, attn_partials_bytes((int)cs, (int)heads, nsplit)));
        if (!part) return FOCR_HIP_E_OOM;
    }
    ProfScope ps(ctx, "attn_prefill");
    FOCR_HIP_TRY(launch_attn_prefill(ctx->stream, gm, q, k, v, out, (int)cs, (int)c0, (int)c1, (int)heads, kHeadDim,
                                     nsplit, split_len, part, qo),
                 name);
    return FOCR_HIP_OK;
}

int32_t attn_checks(const char* name, const void* q, const void* k, const void* v, const void* out, size_t cs,
                    size_t c1, size_t heads, size_t head_dim) {
    if (heads == 0 || head_dim == 0 || heads > (size_t(1) << 20) / head_dim)
        return fail(FOCR_HIP_E_SHAPE, fmt("%s: num_heads*head_dim overflow or zero (%zu x %zu)", name, heads, head_dim));
    if (head_dim != static_cast<size_t>(kHeadDim))
        return fail(FOCR_HIP_E_SHAPE, fmt("%s: head_dim %zu unsupported (the gfx950 kernel takes %d)", name, head_dim,
                                          kHeadDim));
    if (c1 > static_cast<size_t>(1) << 24 || cs > c1)
        return fail(FOCR_HIP_E_SHAPE, fmt("%s: %zu rows over a %zu-key prefix exceed the supported range", name, cs, c1));
    if (cs && (!q || !k || !v || !out)) return fail(FOCR_HIP_E_ARG, fmt("%s: null device pointer", name));
    return FOCR_HIP_OK;
}

}  // namespace

extern "C" {

int32_t focr_hip_chunk_prefill_attention(focr_hip_ctx* ctx, const float* q_chunk, size_t cs, const float* k_prefix,
                                         const float* v_prefix, size_t c1, size_t num_heads, size_t head_dim,
                                         size_t c0, float* out) {
    ENGINE_CTX(ctx);
    const char* name = "chunk_prefill_attention";
    if (c0 > c1 || c0 + cs != c1)  // decoder.rs:1320-1325
        return fail(FOCR_HIP_E_SHAPE, fmt("chunk_prefill_attention: chunk [%zu, %zu) of %zu rows does not fit prefix %zu",
                                          c0, c0 + cs, cs, c1));
    int32_t st = attn_checks(name, q_chunk, k_prefix, v_prefix, out, cs, c1, num_heads, head_dim);
    if (st || cs == 0) return st;
    const int dim = static_cast<int>(num_heads * head_dim);
    const AttnGeom gm{dim, kHeadDim, dim, kHeadDim, dim, kHeadDim, dim, kHeadDim};
    return attn_run(ctx, name, gm, q_chunk, k_prefix, v_prefix, out, cs, c0, c1, num_heads);
}

int32_t focr_hip_prefill_attention(focr_hip_ctx* ctx, const float* q, const float* k, const float* v, size_t seq,
                                   size_t num_heads, size_t head_dim, float* out) {
    ENGINE_CTX(ctx);
    const char* name = "prefill_attention";
    int32_t st = attn_checks(name, q, k, v, out, seq, seq, num_heads, head_dim);
    if (st || seq == 0) return st;
    const int dim = static_cast<int>(num_heads * head_dim);
    const AttnGeom gm{dim, kHeadDim, dim, kHeadDim, dim, kHeadDim, dim, kHeadDim};
    return attn_run(ctx, name, gm, q, k, v, out, seq, 0, seq, num_heads);
}

// kv_in_place: the chunk's K / V rows are in the reference block already
// (the prefill layer's RoPE writes them there); k_chunk / v_chunk unused.
static int32_t rswa_prefill_chunk_impl(focr_hip_ctx* ctx, focr_hip_rswa* c, size_t stream, const float* q_chunk,
                                    const float* k_chunk, const float* v_chunk, size_t cs, size_t c0, float* out,
                                    bool kv_in_place = false, AttnQuantOut* qo = nullptr) {
    const char* name = "rswa_prefill_chunk";
    if (!c) return fail(FOCR_HIP_E_BAD_HANDLE, "null rswa cache");
    if (stream >= c->n_streams)
        return fail(FOCR_HIP_E_SHAPE, fmt("rswa: stream %zu >= num_streams %zu", stream, c->n_streams));
    if (c0 != 0 && c->prefill_len[stream] != static_cast<int64_t>(c0))
        return fail(FOCR_HIP_E_STATE, fmt("rswa_prefill_chunk: chunk starts at %zu but the stream holds %lld prefill "
                                          "tokens",
                                          c0, static_cast<long long>(c->prefill_len[stream])));
    if (c0 + cs > c->ref_capacity)
        return fail(FOCR_HIP_E_STATE, fmt("rswa: prefill seq %zu exceeds ref_capacity %zu", c0 + cs, c->ref_capacity));
    int32_t st = attn_checks(name, q_chunk, kv_in_place ? q_chunk : k_chunk, kv_in_place ? q_chunk : v_chunk, out,
                             cs, c0 + cs, kNumHeads, kHeadDim);
    if (st) return st;
    if (cs) {
        if (!kv_in_place)
            FOCR_HIP_TRY(launch_attn_scatter_kv(ctx->stream, k_chunk, v_chunk, (int)cs, kNumHeads, c->ref_k(stream),
                                                c->ref_v(stream), (int)c->ref_capacity, (int)c0),
                         "rswa_prefill_chunk scatter");
        const int dim = kNumHeads * kHeadDim;
        const int hs = static_cast<int>(c->ref_capacity) * kHeadDim;
        const AttnGeom gm{dim, kHeadDim, kHeadDim, hs, kHeadDim, hs, dim, kHeadDim};
        if ((st = attn_run(ctx, name, gm, q_chunk, c->ref_k(stream), c->ref_v(stream), out, cs, c0, c0 + cs,
                           kNumHeads, qo)))
            return st;
    }
    // the reference seeds the ring once from the whole prefix (record_prefill,
    // decoder.rs:1438-1447): prefill_len = the prefix, ring empty
    c->prefill_len[stream] = static_cast<int64_t>(c0 + cs);
    c->ring_len[stream] = 0;
    c->ring_pos[stream] = 0;
    return FOCR_HIP_OK;
}

int32_t focr_hip_rswa_prefill_chunk(focr_hip_ctx* ctx, focr_hip_rswa* c, size_t stream, const float* q_chunk,
                                    const float* k_chunk, const float* v_chunk, size_t cs, size_t c0, float* out) {
    ENGINE_CTX(ctx);
    return rswa_prefill_chunk_impl(ctx, c, stream, q_chunk, k_chunk, v_chunk, cs, c0, out);
}

// ---- one decoder layer over a prefill chunk (decoder.rs:2428-2520) ---------------

// route_default (moe.rs:273-280: norm_topk_prob false, scaling 1.0) of a
// prefill chunk's t rows
static int32_t prefill_route_impl(focr_hip_ctx* ctx, const focr_hip_moe_layer* L, const float* x, size_t t,
                                  uint32_t* idx, float* gates, int* flag) {
    return route_rows_impl(ctx, L, x, t, 0, 1.0f, idx, gates, nullptr, flag);
}

static int32_t decoder_layer_prefill_impl(focr_hip_ctx* ctx, const focr_hip_decoder_layer* L, focr_hip_rswa* cache,
                                          size_t stream, float* x, size_t cs, size_t c0, uint32_t* route_idx,
                                          int32_t check_route) {
    if (!L) return fail(FOCR_HIP_E_BAD_HANDLE, "decoder_layer_prefill: null layer");
    if (!cache) return fail(FOCR_HIP_E_BAD_HANDLE, "decoder_layer_prefill: null rswa cache");
    if (!x) return fail(FOCR_HIP_E_ARG, "decoder_layer_prefill: null x");
    if (L->n_heads != 10 || L->head_dim != 128)
        return fail(FOCR_HIP_E_SHAPE, "decoder_layer_prefill: the R-SWA cache holds 10 heads x 128");
    if (cs < 1 || cs > static_cast<size_t>(kLayerPrefillMaxRows))
        return fail(FOCR_HIP_E_SHAPE,
                    fmt("decoder_layer_prefill: chunk of %zu rows outside 1..=%d", cs, kLayerPrefillMaxRows));
    if (stream >= cache->n_streams)
        return fail(FOCR_HIP_E_SHAPE, fmt("rswa: stream %zu >= num_streams %zu", stream, cache->n_streams));
    // the chunk order rswa_prefill_chunk requires, checked before any launch
    if (c0 != 0 && cache->prefill_len[stream] != static_cast<int64_t>(c0))
        return fail(FOCR_HIP_E_STATE, fmt("rswa_prefill_chunk: chunk starts at %zu but the stream holds %lld prefill "
                                          "tokens",
                                          c0, static_cast<long long>(cache->prefill_len[stream])));
    if (c0 + cs > cache->ref_capacity)
        return fail(FOCR_HIP_E_STATE,
                    fmt("rswa: prefill seq %zu exceeds ref_capacity %zu", c0 + cs, cache->ref_capacity));
    const size_t H = L->hidden, D = L->n_heads * L->head_dim;
    const size_t I = L->gate ? L->gate->n : 0, K = L->moe ? L->moe->top_k : 0;
    // one scratch slot carved into the chunk's intermediates
    const size_t fl = cs * (H + 3 * D + D + D + H + H + H) + (L->gate ? 2 * cs * I : 0) + cs * K * 2 + cs;
    char* base = static_cast<char*>(ctx->scratch_get(kScrLayer, fl * 4 + 20 * 256));
    if (!base) return FOCR_HIP_E_OOM;
    auto take = [&](size_t bytes) {
        char* r = base;
        base += (bytes + 255) & ~static_cast<size_t>(255);
        return r;
    };
    float* nrm = reinterpret_cast<float*>(take(cs * H * 4));
    float* qkv = reinterpret_cast<float*>(take(cs * 3 * D * 4));
    float* q = reinterpret_cast<float*>(take(cs * D * 4));
    float* cx = reinterpret_cast<float*>(take(cs * D * 4));
    float* attn = reinterpret_cast<float*>(take(cs * H * 4));
    float* h = reinterpret_cast<float*>(take(cs * H * 4));
    float* mlp = reinterpret_cast<float*>(take(cs * H * 4));
    hipStream_t s = ctx->stream;
    int32_t st;
    // 1. input RMSNorm; 2. q / k / v = linear_int8_dynamic (one fused [3 D, H]
    //    weight: the same quantized rows times each projection's rows); 3.
    //    RoPE at the chunk's positions c0 ..; 4. K / V into the stream's
    //    reference block and the chunk's causal attention over [0, c0 + cs)
    // the input norm inside qkv's quantize launch where qkv takes the tiled GEMM
    // (its float4 row loads need 16-byte aligned rows and norm weight)
    if (linear_i8_norm_fusable(L->qkv, cs) && reinterpret_cast<uintptr_t>(x) % 16 == 0 &&
        reinterpret_cast<uintptr_t>(L->input_ln) % 16 == 0 && H % 4 == 0) {
        if ((st = linear_i8_dynamic_impl(ctx, L->qkv, x, cs, nullptr, qkv, L->input_ln, L->eps))) return st;
    } else {
        {
            ProfScope ps(ctx, "layer_prefill_norm");
            FOCR_HIP_TRY(launch_rms_norm(s, x, L->input_ln, (int)cs, (int)H, L->eps, nrm), "rms_norm launch");
        }
        if ((st = linear_i8_dynamic_impl(ctx, L->qkv, nrm, cs, nullptr, qkv))) return st;
    }
    {
        ProfScope ps(ctx, "layer_prefill_rope");
        // k and v straight into the stream's head-major reference block at c0
        const size_t hs = cache->ref_capacity * L->head_dim;
        FOCR_HIP_TRY(launch_rope_rows(s, qkv, (int)cs, (int)c0, L->inv_freq, (int)L->n_heads, (int)L->head_dim, q,
                                      cache->ref_k(stream) + c0 * L->head_dim, cache->ref_v(stream) + c0 * L->head_dim,
                                      L->head_dim, hs),
                     "rope launch");
    }
    // the split merge writes the context rows quantized for o_proj, in the
    // layout and scratch o_proj's linear_int8_dynamic reads
    AttnQuantOut qo{};
    qo.tiled = linear_i8_act_tiled(L->o_proj, cs, nullptr);
    qo.xq = static_cast<int8_t*>(ctx->scratch_get(kScrXq, linear_i8_act_bytes(L->o_proj, cs, nullptr)));
    qo.xs = static_cast<float*>(ctx->scratch_get(kScrXs, cs * sizeof(float)));
    if (!qo.xq || !qo.xs) return FOCR_HIP_E_OOM;
    if ((st = rswa_prefill_chunk_impl(ctx, cache, stream, q, nullptr, nullptr, cs, c0, cx, true, &qo))) return st;
    // 5. o_proj; 6. residual + post-attention RMSNorm
    if ((st = linear_i8_dynamic_impl(ctx, L->o_proj, qo.done ? nullptr : cx, cs, nullptr, attn, nullptr, 0.0f,
                                     qo.done)))
        return st;
    {
        ProfScope ps(ctx, "layer_prefill_residual_norm");
        FOCR_HIP_TRY(launch_residual_rms_norm(s, x, attn, L->post_ln, (int)cs, (int)H, L->eps, h, nrm),
                     "residual rms_norm launch");
    }
    // 7. prefill_mlp_i8 (decoder.rs:2184-2195): moe_block_i8 (route_default,
    //    the routed experts and the shared one) or the dense expert_mlp_i8
    if (L->moe) {
        uint32_t* idx = reinterpret_cast<uint32_t*>(take(cs * K * 4));
        float* gates = reinterpret_cast<float*>(take(cs * K * 4));
        int* flag = reinterpret_cast<int*>(take(cs * 4));
        if ((st = prefill_route_impl(ctx, L->moe, nrm, cs, idx, gates, flag))) return st;
        if (check_route) {
            std::vector<int> flags(cs);
            FOCR_HIP_TRY(hipMemcpyAsync(flags.data(), flag, cs * sizeof(int), hipMemcpyDeviceToHost, s), "D2H route flag");
            FOCR_HIP_TRY(hipStreamSynchronize(s), "hipStreamSynchronize");
            for (size_t i = 0; i < cs; ++i)
                if (flags[i]) return fail(FOCR_HIP_E_ROUTE, fmt("moe::route: no finite router score for token %zu", i));
        }
        if (route_idx)
            FOCR_HIP_TRY(hipMemcpyAsync(route_idx, idx, cs * K * 4, hipMemcpyDeviceToDevice, s), "route idx copy");
        // 8. the second residual, x = h + mlp, in the MoE block's combine
        return moe_prefill_i8_impl(ctx, L->moe, nrm, cs, idx, gates, L->moe->swg ? 1 : 0, x, 0, h);
    } else {
        float* g = reinterpret_cast<float*>(take(cs * I * 4));
        float* u = reinterpret_cast<float*>(take(cs * I * 4));
        if ((st = linear_i8_dynamic_impl(ctx, L->gate, nrm, cs, nullptr, g)) ||
            (st = linear_i8_dynamic_impl(ctx, L->up, nrm, cs, nullptr, u)))
            return st;
        {
            ProfScope ps(ctx, "layer_prefill_silu");
            FOCR_HIP_TRY(launch_silu_mul(s, g, u, g, cs * I), "silu launch");
        }
        if ((st = linear_i8_dynamic_impl(ctx, L->down, g, cs, nullptr, mlp))) return st;
    }
    // 8. the second residual
    ProfScope ps(ctx, "layer_prefill_residual");
    FOCR_HIP_TRY(launch_add_rows(s, h, mlp, x, cs * H), "residual launch");
    return FOCR_HIP_OK;
}

int32_t focr_hip_decoder_layer_prefill(focr_hip_ctx* ctx, const focr_hip_decoder_layer* L, focr_hip_rswa* cache,
                                       size_t stream, float* x, size_t cs, size_t c0, uint32_t* route_idx,
                                       int32_t check_route) {
    ENGINE_CTX(ctx);
    return decoder_layer_prefill_impl(ctx, L, cache, stream, x, cs, c0, route_idx, check_route);
}

// ---- the whole batched decode step (decoder.rs:2812-2965) ------------------------

int32_t focr_hip_decoder_create(focr_hip_ctx* ctx, size_t n_layers, const focr_hip_decoder_layer* const* layers,
                                const float* final_norm, float rms_eps, const focr_hip_qint8* lm_head,
                                focr_hip_decoder** out) {
    ENGINE_CTX(ctx);
    if (!out) return fail(FOCR_HIP_E_ARG, "decoder_create: null out");
    *out = nullptr;
    if (!layers || !final_norm) return fail(FOCR_HIP_E_ARG, "decoder_create: null layers or final_norm");
    if (!lm_head) return fail(FOCR_HIP_E_BAD_HANDLE, "decoder_create: null lm_head");
    if (n_layers < 1 || n_layers > 256)
        return fail(FOCR_HIP_E_SHAPE, fmt("decoder_create: %zu layers outside 1..=256", n_layers));
    const size_t H = layers[0] ? layers[0]->hidden : 0;
    size_t top_k = 0;
    for (size_t l = 0; l < n_layers; ++l) {
        const focr_hip_decoder_layer* L = layers[l];
        if (!L) return fail(FOCR_HIP_E_BAD_HANDLE, fmt("decoder_create: null layer %zu", l));
        if (L->hidden != H)
            return fail(FOCR_HIP_E_SHAPE, fmt("decoder_create: layer %zu hidden %zu != %zu", l, L->hidden, H));
        if (L->moe) {
            if (top_k && L->moe->top_k != top_k)
                return fail(FOCR_HIP_E_SHAPE, fmt("decoder_create: layer %zu top_k %zu != %zu", l, L->moe->top_k,
                                                  top_k));
            top_k = L->moe->top_k;
        }
    }
    if (lm_head->k != H)
        return fail(FOCR_HIP_E_SHAPE, fmt("decoder_create: lm_head [%zu, %zu] does not take hidden %zu", lm_head->n,
                                          lm_head->k, H));
    auto* d = new focr_hip_decoder();
    d->ctx = ctx;
    d->hidden = H;
    d->top_k = top_k;
    d->eps = rms_eps;
    d->layers.assign(layers, layers + n_layers);
    d->lm_head = lm_head;
    hipError_t e = hipMalloc(&d->final_norm, H * sizeof(float));
    if (e == hipSuccess) e = hipMemcpy(d->final_norm, final_norm, H * sizeof(float), hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        hipFree(d->final_norm);
        delete d;
        return hip_fail(e, "decoder_create upload");
    }
    *out = d;
    return FOCR_HIP_OK;
}

int32_t focr_hip_decoder_free(focr_hip_decoder* d) {
    if (!d) return FOCR_HIP_OK;
    hipSetDevice(d->ctx->device);
    hipStreamSynchronize(d->ctx->stream);
    hipFree(d->final_norm);
    delete d;
    return FOCR_HIP_OK;
}

// every layer's decode step, then the final RMSNorm of each row into the
// returned buffer (the LM head's input)
static int32_t decoder_layers_impl(focr_hip_ctx* ctx, const focr_hip_decoder* d, focr_hip_rswa* const* caches,
                                   const uint32_t* positions, float* x, uint32_t* route_idx, int32_t check_route,
                                   float** normed, size_t* n_streams) {
    if (!d) return fail(FOCR_HIP_E_BAD_HANDLE, "decoder_step: null decoder");
    if (!caches || !positions || !x) return fail(FOCR_HIP_E_ARG, "decoder_step: null caches, positions or x");
    const size_t NL = d->layers.size();
    for (size_t l = 0; l < NL; ++l)
        if (!caches[l]) return fail(FOCR_HIP_E_BAD_HANDLE, fmt("decoder_step: null rswa cache for layer %zu", l));
    const size_t B = caches[0]->n_streams;
    for (size_t l = 1; l < NL; ++l)
        if (caches[l]->n_streams != B)
            return fail(FOCR_HIP_E_SHAPE, fmt("decoder_step: layer %zu cache holds %zu streams, layer 0's %zu", l,
                                              caches[l]->n_streams, B));
    for (size_t l = 0; l < NL; ++l) {
        const focr_hip_decoder_layer* L = d->layers[l];
        uint32_t* ri = (route_idx && L->moe) ? route_idx + l * B * d->top_k : nullptr;
        int32_t st = decoder_layer_step_impl(ctx, L, caches[l], positions, x, ri, check_route);
        if (st) return st;
    }
    float* xn = static_cast<float*>(ctx->scratch_get(kScrDec, B * d->hidden * sizeof(float)));
    if (!xn) return FOCR_HIP_E_OOM;
    {
        ProfScope ps(ctx, "rms_norm");
        FOCR_HIP_TRY(launch_rms_norm(ctx->stream, x, d->final_norm, (int)B, (int)d->hidden, d->eps, xn),
                     "final rms_norm launch");
    }
    *normed = xn;
    *n_streams = B;
    return FOCR_HIP_OK;
}

int32_t focr_hip_decoder_step(focr_hip_ctx* ctx, const focr_hip_decoder* d, focr_hip_rswa* const* caches,
                              const uint32_t* positions, float* x, float* logits, uint32_t* tokens,
                              uint32_t* route_idx, int32_t check_route) {
    ENGINE_CTX(ctx);
    if (!tokens) return fail(FOCR_HIP_E_ARG, "decoder_step: null tokens");
    float* xn = nullptr;
    size_t B = 0;
    int32_t st = decoder_layers_impl(ctx, d, caches, positions, x, route_idx, check_route, &xn, &B);
    if (st) return st;
    // the LM head takes up to 32 rows per pass
    const size_t H = d->hidden, V = d->lm_head->n;
    for (size_t r0 = 0; r0 < B; r0 += 32) {
        const size_t m = std::min<size_t>(32, B - r0);
        if ((st = lm_head_i8_impl(ctx, d->lm_head, xn + r0 * H, m, logits ? logits + r0 * V : nullptr, tokens + r0)))
            return st;
    }
    return FOCR_HIP_OK;
}

int32_t focr_hip_decoder_step_sample(focr_hip_ctx* ctx, const focr_hip_decoder* d, focr_hip_rswa* const* caches,
                                     const uint32_t* positions, float* x, uint32_t* history, size_t history_cap,
                                     uint32_t* history_len, size_t ngram_size, size_t window,
                                     const uint32_t* whitelist, size_t n_whitelist, float temperature,
                                     uint32_t eos_token_id, int32_t append, float* logits, uint32_t* tokens,
                                     uint8_t* is_eos, uint32_t* route_idx, int32_t check_route) {
    ENGINE_CTX(ctx);
    if (!tokens) return fail(FOCR_HIP_E_ARG, "decoder_step_sample: null tokens");
    if (temperature > 0.0f)  // refused before any layer runs (the sampler refuses it too)
        return fail(FOCR_HIP_E_NOT_IMPLEMENTED, "native_engine::sampler::decode_step_premasked — temperature>0 "
                                                "sampling is outside the greedy fp32 spine");
    float* xn = nullptr;
    size_t B = 0;
    int32_t st = decoder_layers_impl(ctx, d, caches, positions, x, route_idx, check_route, &xn, &B);
    if (st) return st;
    // the sampling LM head takes up to 32 rows per pass
    const size_t H = d->hidden, V = d->lm_head->n;
    for (size_t r0 = 0; r0 < B; r0 += 32) {
        const size_t m = std::min<size_t>(32, B - r0);
        if ((st = lm_head_sample_i8_impl(ctx, d->lm_head, xn + r0 * H, m, history ? history + r0 * history_cap : nullptr,
                                         history_cap, history_len ? history_len + r0 : nullptr, ngram_size, window,
                                         whitelist, n_whitelist, temperature, eos_token_id, append,
                                         logits ? logits + r0 * V : nullptr, tokens + r0,
                                         is_eos ? is_eos + r0 : nullptr, check_route)))
            return st;
    }
    return FOCR_HIP_OK;
}

// ---- the whole prefill of one stream (decoder.rs:2428-2520) ---------------------

int32_t focr_hip_decoder_prefill(focr_hip_ctx* ctx, const focr_hip_decoder* d, focr_hip_rswa* const* caches,
                                 size_t stream, float* x, size_t seq, size_t chunk, float* logits, uint32_t* token,
                                 uint32_t* route_idx, int32_t check_route) {
    ENGINE_CTX(ctx);
    if (!d) return fail(FOCR_HIP_E_BAD_HANDLE, "decoder_prefill: null decoder");
    if (!caches || !x) return fail(FOCR_HIP_E_ARG, "decoder_prefill: null caches or x");
    if (seq < 1) return fail(FOCR_HIP_E_SHAPE, "decoder_prefill: empty sequence");
    const size_t NL = d->layers.size();
    for (size_t l = 0; l < NL; ++l) {
        if (!caches[l]) return fail(FOCR_HIP_E_BAD_HANDLE, fmt("decoder_prefill: null rswa cache for layer %zu", l));
        if (stream >= caches[l]->n_streams)
            return fail(FOCR_HIP_E_SHAPE, fmt("rswa: stream %zu >= num_streams %zu", stream, caches[l]->n_streams));
        if (seq > caches[l]->ref_capacity)
            return fail(FOCR_HIP_E_STATE,
                        fmt("rswa: prefill seq %zu exceeds ref_capacity %zu", seq, caches[l]->ref_capacity));
    }
    // prefill_chunk_bounds(seq, chunk) with every layer per chunk, the chunk
    // loop outermost as in the reference; chunk 0: the monolithic schedule.
    // A chunk is at most the layer step's row limit.
    const size_t step = std::min<size_t>(chunk ? chunk : seq, static_cast<size_t>(kLayerPrefillMaxRows));
    const size_t H = d->hidden;
    int32_t st;
    for (size_t c0 = 0; c0 < seq; c0 += step) {
        const size_t cs = std::min(step, seq - c0);
        for (size_t l = 0; l < NL; ++l) {
            const focr_hip_decoder_layer* L = d->layers[l];
            uint32_t* ri = (route_idx && L->moe) ? route_idx + (l * seq + c0) * d->top_k : nullptr;
            if ((st = decoder_layer_prefill_impl(ctx, L, caches[l], stream, x + c0 * H, cs, c0, ri, check_route)))
                return st;
        }
    }
    if (!logits && !token) return FOCR_HIP_OK;
    // the first generated token: model.norm of the last position, the LM
    // head and argmax_row (decoder.rs:2943-2965, sampler.rs:168-186)
    float* xn = static_cast<float*>(ctx->scratch_get(kScrDec, H * sizeof(float) + 256));
    if (!xn) return FOCR_HIP_E_OOM;
    uint32_t* tok = token ? token : reinterpret_cast<uint32_t*>(xn + H);
    {
        ProfScope ps(ctx, "rms_norm");
        FOCR_HIP_TRY(launch_rms_norm(ctx->stream, x + (seq - 1) * H, d->final_norm, 1, (int)H, d->eps, xn),
                     "final rms_norm launch");
    }
    return lm_head_i8_impl(ctx, d->lm_head, xn, 1, logits, tok);
}

int32_t focr_hip_rswa_get_state(const focr_hip_rswa* c, size_t stream, uint32_t* prefill_len, uint32_t* ring_len,
                                uint32_t* ring_pos) {
    if (!c) return fail(FOCR_HIP_E_BAD_HANDLE, "null rswa cache");
    if (stream >= c->n_streams) return fail(FOCR_HIP_E_SHAPE, "rswa: stream out of range");
    if (c->prefill_len[stream] < 0) return fail(FOCR_HIP_E_STATE, "rswa: prefill never recorded");
    if (prefill_len) *prefill_len = static_cast<uint32_t>(c->prefill_len[stream]);
    if (ring_len) *ring_len = c->ring_len[stream];
    if (ring_pos) *ring_pos = c->ring_pos[stream];
    return FOCR_HIP_OK;
}

int32_t focr_hip_rswa_set_state(focr_hip_rswa* c, size_t stream, uint32_t ring_len, uint32_t ring_pos) {
    if (!c) return fail(FOCR_HIP_E_BAD_HANDLE, "null rswa cache");
    if (stream >= c->n_streams) return fail(FOCR_HIP_E_SHAPE, "rswa: stream out of range");
    if (c->prefill_len[stream] < 0) return fail(FOCR_HIP_E_STATE, "rswa: prefill never recorded");
    // A reachable cursor pair: warm-up has ring_pos == ring_len % W, steady
    // state has ring_len == W and any ring_pos < W (rswa.rs:467-494).
    if (ring_len > static_cast<uint32_t>(kRingWindow) || ring_pos >= static_cast<uint32_t>(kRingWindow) ||
        (ring_len < static_cast<uint32_t>(kRingWindow) && ring_pos != ring_len % kRingWindow))
        return fail(FOCR_HIP_E_STATE, fmt("rswa: unreachable ring state (ring_len=%u, ring_pos=%u)", ring_len, ring_pos));
    c->ring_len[stream] = ring_len;
    c->ring_pos[stream] = ring_pos;
    return FOCR_HIP_OK;
}

int32_t focr_hip_rswa_regions(const focr_hip_rswa* c, size_t stream, float** ref_k, float** ref_v, float** ring_k,
                              float** ring_v) {
    if (!c) return fail(FOCR_HIP_E_BAD_HANDLE, "null rswa cache");
    if (stream >= c->n_streams) return fail(FOCR_HIP_E_SHAPE, "rswa: stream out of range");
    if (ref_k) *ref_k = c->ref_k(stream);
    if (ref_v) *ref_v = c->ref_v(stream);
    if (ring_k) *ring_k = c->ring_k(stream);
    if (ring_v) *ring_v = c->ring_v(stream);
    return FOCR_HIP_OK;
}

// ---- profiling -------------------------------------------------------------------

int32_t focr_hip_prof_enable(focr_hip_ctx* ctx, int32_t on) {
    if (!ctx) return fail(FOCR_HIP_E_BAD_HANDLE, "null focr_hip_ctx");
    std::lock_guard<std::mutex> lk(ctx->mu);
    ctx->prof = on != 0;
    return FOCR_HIP_OK;
}

static void drain_prof(focr_hip_ctx* ctx) {
    hipStreamSynchronize(ctx->stream);
    for (auto& p : ctx->pending) {
        float ms = 0.0f;
        if (hipEventElapsedTime(&ms, p.start, p.stop) == hipSuccess) {
            auto& v = ctx->prof_samples[p.name];
            if (v.size() < kProfMaxSamples) v.push_back(ms);
        }
        // not recycled: an event reused for a later dispatch has read back
        // elapsed times several times the kernel's (same step throughput)
        hipEventDestroy(p.start);
        hipEventDestroy(p.stop);
    }
    ctx->pending.clear();
}

static void drop_marks(focr_hip_ctx* ctx) {
    for (hipEvent_t e : ctx->marks) hipEventDestroy(e);
    ctx->marks.clear();
}

int32_t focr_hip_prof_reset(focr_hip_ctx* ctx) {
    if (!ctx) return fail(FOCR_HIP_E_BAD_HANDLE, "null focr_hip_ctx");
    std::lock_guard<std::mutex> lk(ctx->mu);
    hipSetDevice(ctx->device);
    drain_prof(ctx);
    ctx->prof_samples.clear();
    return FOCR_HIP_OK;
}

// nearest rank: rank = ceil(q * n) clamped to [1, n], element rank - 1 of the
// ascending samples (the reference's bench statistics, perf_harness.rs:276-282)
static double nearest_rank(const std::vector<float>& sorted, double q) {
    const size_t n = sorted.size();
    size_t rank = static_cast<size_t>(std::ceil(q * static_cast<double>(n)));
    rank = std::min(std::max<size_t>(rank, 1), n);
    return sorted[rank - 1];
}

int32_t focr_hip_prof_read(focr_hip_ctx* ctx, char* json, size_t cap) {
    if (!ctx) return fail(FOCR_HIP_E_BAD_HANDLE, "null focr_hip_ctx");
    std::lock_guard<std::mutex> lk(ctx->mu);
    hipSetDevice(ctx->device);
    drain_prof(ctx);
    std::string j = "{";
    bool first = true;
    for (auto& kv : ctx->prof_samples) {
        if (kv.second.empty()) continue;
        std::vector<float> v = kv.second;
        double total = 0.0;
        for (float x : v) total += x;
        std::sort(v.begin(), v.end());
        char buf[384];
        snprintf(buf, sizeof(buf),
                 "%s\"%s\":{\"count\":%zu,\"ms\":%.6f,\"min_ms\":%.6f,\"p50_ms\":%.6f,\"p90_ms\":%.6f}",
                 first ? "" : ",", kv.first.c_str(), v.size(), total, static_cast<double>(v.front()),
                 nearest_rank(v, 0.5), nearest_rank(v, 0.9));
        j += buf;
        first = false;
    }
    j += "}";
    if (json && cap) snprintf(json, cap, "%s", j.c_str());
    return FOCR_HIP_OK;
}

int32_t focr_hip_mark(focr_hip_ctx* ctx) {
    if (!ctx) return fail(FOCR_HIP_E_BAD_HANDLE, "null focr_hip_ctx");
    std::lock_guard<std::mutex> lk(ctx->mu);
    FOCR_HIP_TRY(ctx->bind(), "mark: set device");
    if (ctx->marks.size() >= kMaxMarks) return fail(FOCR_HIP_E_SHAPE, fmt("mark: more than %zu marks", kMaxMarks));
    hipEvent_t e = nullptr;
    FOCR_HIP_TRY(hipEventCreate(&e), "mark: event create");
    hipError_t err = hipEventRecord(e, ctx->stream);
    if (err != hipSuccess) {
        hipEventDestroy(e);
        FOCR_HIP_TRY(err, "mark: event record");
    }
    ctx->marks.push_back(e);
    return FOCR_HIP_OK;
}

int32_t focr_hip_marks_read(focr_hip_ctx* ctx, float* ms, size_t cap, size_t* n_out) {
    if (!ctx) return fail(FOCR_HIP_E_BAD_HANDLE, "null focr_hip_ctx");
    std::lock_guard<std::mutex> lk(ctx->mu);
    FOCR_HIP_TRY(ctx->bind(), "marks_read: set device");
    hipError_t err = hipStreamSynchronize(ctx->stream);
    const size_t n = ctx->marks.size() < 2 ? 0 : ctx->marks.size() - 1;
    if (err == hipSuccess && n > cap) err = hipErrorInvalidValue;
    for (size_t i = 0; i < n && err == hipSuccess; ++i) err = hipEventElapsedTime(&ms[i], ctx->marks[i], ctx->marks[i + 1]);
    drop_marks(ctx);
    if (err == hipErrorInvalidValue && n > cap)
        return fail(FOCR_HIP_E_SHAPE, fmt("marks_read: %zu intervals, room for %zu", n, cap));
    FOCR_HIP_TRY(err, "marks_read");
    if (n_out) *n_out = n;
    return FOCR_HIP_OK;
}

}  // extern "C"
