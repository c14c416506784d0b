// focr_hip.cpp — the C ABI (include/focr_hip.h): context, status/errors,
// shape contracts with the reference's panic messages, device buffers, the
// drop-in tier, the uploaded-weight engine ops and profiling.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cinttypes>
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

namespace focr {

static thread_local std::string g_last_error;

void set_error(const std::string& msg) { g_last_error = msg; }
void clear_error() { g_last_error.clear(); }
int32_t fail(int32_t code, const std::string& msg) {
    set_error(msg);
    return code;
}
int32_t hip_fail(hipError_t e, const char* what) {
    std::string m = std::string(what) + ": " + hipGetErrorString(e);
    set_error(m);
    return e == hipErrorOutOfMemory ? FOCR_HIP_E_OOM : FOCR_HIP_E_HIP;
}

static std::string fmt(const char* f, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, f);
    vsnprintf(buf, sizeof(buf), f, ap);
    va_end(ap);
    return buf;
}

// checked_len (scalar.rs:63-67): "{context}: {expr} overflow ({lhs} * {rhs})"
static bool checked_len(const char* context, size_t lhs, size_t rhs, const char* expr, size_t* out,
                        int32_t* status) {
    if (lhs != 0 && rhs > std::numeric_limits<size_t>::max() / lhs) {
        *status = fail(FOCR_HIP_E_SHAPE, fmt("%s: %s overflow (%zu * %zu)", context, expr, lhs, rhs));
        return false;
    }
    *out = lhs * rhs;
    return true;
}

// The kernels index with 32-bit ints; larger extents are a GPU-tier limit.
static bool fits_i32(const char* context, size_t v, const char* what, int32_t* status) {
    if (v > static_cast<size_t>(std::numeric_limits<int32_t>::max())) {
        *status = fail(FOCR_HIP_E_SHAPE, fmt("%s: %s %zu exceeds the gfx950 tier limit", context, what, v));
        return false;
    }
    return true;
}

LaunchEvents& launch_events() {
    static thread_local LaunchEvents le;
    return le;
}

ProfScope::ProfScope(focr_hip_ctx* c, const char* n) : ctx(c), name(n) {
    if (ctx && ctx->prof) {
        start = ctx->take_event();
        stop = ctx->take_event();
        if (start && stop) launch_events() = LaunchEvents{start, stop, true, false};
    }
}

ProfScope::~ProfScope() {
    LaunchEvents& le = launch_events();
    const bool used = le.used && le.stop == stop;
    if (le.stop == stop) le = LaunchEvents{};
    if (!start || !stop) return;
    if (used) {
        ctx->pending.push_back({name, start, stop});
    } else {  // nothing launched (an error path)
        hipEventDestroy(start);
        hipEventDestroy(stop);
    }
}

}  // namespace focr

using namespace focr;

void* focr_hip_ctx::scratch_get(int slot, size_t bytes) {
    Buf& b = scratch[slot];
    if (bytes == 0) bytes = 16;
    if (b.cap >= bytes) return b.p;
    if (b.p) {
        hipStreamSynchronize(stream);
        hipFree(b.p);
        b.p = nullptr;
        b.cap = 0;
    }
    size_t cap = std::max(bytes, static_cast<size_t>(4096));
    cap = (cap + 255) & ~static_cast<size_t>(255);
    hipError_t e = hipMalloc(&b.p, cap);
    if (e != hipSuccess) {
        b.p = nullptr;
        hip_fail(e, "scratch hipMalloc");
        return nullptr;
    }
    b.cap = cap;
    return b.p;
}

// A fresh event per profiled scope, destroyed once read (drain_prof).
hipEvent_t focr_hip_ctx::take_event() {
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    return e;
}

size_t focr_hip_rswa::stream_floats() const {
    return 2 * static_cast<size_t>(kNumHeads) * ref_capacity * kHeadDim +
           2 * static_cast<size_t>(kNumHeads) * kRingWindow * kHeadDim;
}
float* focr_hip_rswa::ref_k(size_t s) const { return base + s * stream_floats(); }
float* focr_hip_rswa::ref_v(size_t s) const { return ref_k(s) + static_cast<size_t>(kNumHeads) * ref_capacity * kHeadDim; }
float* focr_hip_rswa::ring_k(size_t s) const { return ref_v(s) + static_cast<size_t>(kNumHeads) * ref_capacity * kHeadDim; }
float* focr_hip_rswa::ring_v(size_t s) const { return ring_k(s) + static_cast<size_t>(kNumHeads) * kRingWindow * kHeadDim; }

#define CTX_GUARD(ctx)                                                            \
    if (!(ctx)) return fail(FOCR_HIP_E_BAD_HANDLE, "null focr_hip_ctx");          \
    std::lock_guard<std::mutex> lock_((ctx)->mu);                                  \
    clear_error();                                                                 \
    FOCR_HIP_TRY((ctx)->bind(), "hipSetDevice")

extern "C" {

const char* focr_hip_last_error(void) { return g_last_error.c_str(); }

const char* focr_hip_version(void) { return "franken_ocr_amd 0.1.0 (gfx950)"; }

int32_t focr_hip_device_count(int32_t* count) {
    if (!count) return fail(FOCR_HIP_E_ARG, "focr_hip_device_count: null out");
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess) n = 0;
    *count = n;
    return FOCR_HIP_OK;
}

int32_t focr_hip_ctx_create(int32_t device, focr_hip_ctx** out) {
    clear_error();
    if (!out) return fail(FOCR_HIP_E_ARG, "focr_hip_ctx_create: null out");
    *out = nullptr;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0)
        return fail(FOCR_HIP_E_NO_DEVICE, "focr_hip_ctx_create: no HIP device visible");
    if (device < 0 || device >= n)
        return fail(FOCR_HIP_E_NO_DEVICE, fmt("focr_hip_ctx_create: device %d out of range (%d visible)", device, n));
    hipDeviceProp_t prop;
    FOCR_HIP_TRY(hipGetDeviceProperties(&prop, device), "hipGetDeviceProperties");
    std::string arch = prop.gcnArchName;
    if (arch.compare(0, 6, "gfx950") != 0)
        return fail(FOCR_HIP_E_NO_DEVICE,
                    fmt("focr_hip_ctx_create: device %d is %s; this library ships gfx950 code only", device, arch.c_str()));
    FOCR_HIP_TRY(hipSetDevice(device), "hipSetDevice");
    std::unique_ptr<focr_hip_ctx> c(new (std::nothrow) focr_hip_ctx());
    if (!c) return fail(FOCR_HIP_E_OOM, "focr_hip_ctx_create: host allocation failed");
    c->device = device;
    c->cu_count = prop.multiProcessorCount;
    c->arch = arch;
    // Default priority, non-blocking with respect to the legacy null stream.
    FOCR_HIP_TRY(hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking), "hipStreamCreate");
    // The allocation-free entry points' scratch: this device's address of the
    // static array, resolved once per device with the device current. A
    // failure here only disables those entry points (they report it).
    c->static_scratch_err = static_scratch_init(device, &c->static_scratch);
    *out = c.release();
    return FOCR_HIP_OK;
}

int32_t focr_hip_ctx_destroy(focr_hip_ctx* ctx) {
    if (!ctx) return FOCR_HIP_OK;
    hipSetDevice(ctx->device);
    hipStreamSynchronize(ctx->stream);
    for (auto& b : ctx->scratch)
        if (b.p) hipFree(b.p);
    for (auto& p : ctx->pending) {
        hipEventDestroy(p.start);
        hipEventDestroy(p.stop);
    }
    for (hipEvent_t e : ctx->marks) hipEventDestroy(e);
    hipStreamDestroy(ctx->stream);
    delete ctx;
    return FOCR_HIP_OK;
}

int32_t focr_hip_ctx_set_route_wait(focr_hip_ctx* ctx, uint32_t ticks) {
    if (!ctx) return fail(FOCR_HIP_E_BAD_HANDLE, "null focr_hip_ctx");
    std::lock_guard<std::mutex> lk(ctx->mu);
    ctx->route_wait_ticks = ticks;
    return FOCR_HIP_OK;
}

int32_t focr_hip_ctx_scratch_bytes(focr_hip_ctx* ctx, size_t* bytes) {
    if (!ctx) return fail(FOCR_HIP_E_BAD_HANDLE, "null focr_hip_ctx");
    if (!bytes) return fail(FOCR_HIP_E_ARG, "focr_hip_ctx_scratch_bytes: null out");
    std::lock_guard<std::mutex> lk(ctx->mu);
    size_t total = 0;
    for (auto& b : ctx->scratch) total += b.cap;
    *bytes = total;
    return FOCR_HIP_OK;
}

int32_t focr_hip_ctx_synchronize(focr_hip_ctx* ctx) {
    CTX_GUARD(ctx);
    FOCR_HIP_TRY(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
    return FOCR_HIP_OK;
}

int32_t focr_hip_device_synchronize(focr_hip_ctx* ctx) {
    CTX_GUARD(ctx);
    FOCR_HIP_TRY(hipDeviceSynchronize(), "hipDeviceSynchronize");
    return FOCR_HIP_OK;
}

int32_t focr_hip_ctx_stream(focr_hip_ctx* ctx, void** stream) {
    if (!ctx) return fail(FOCR_HIP_E_BAD_HANDLE, "null focr_hip_ctx");
    if (!stream) return fail(FOCR_HIP_E_ARG, "focr_hip_ctx_stream: null out");
    *stream = ctx->stream;
    return FOCR_HIP_OK;
}

int32_t focr_hip_ctx_device_info(focr_hip_ctx* ctx, char* arch, size_t arch_cap, int32_t* cu_count) {
    if (!ctx) return fail(FOCR_HIP_E_BAD_HANDLE, "null focr_hip_ctx");
    if (arch && arch_cap) snprintf(arch, arch_cap, "%s", ctx->arch.c_str());
    if (cu_count) *cu_count = ctx->cu_count;
    return FOCR_HIP_OK;
}

int32_t focr_hip_tier(char* tag, size_t tag_cap, char* feature, size_t feature_cap) {
    if (tag && tag_cap) snprintf(tag, tag_cap, "%s", "gfx950");
    if (feature && feature_cap) snprintf(feature, feature_cap, "%s", "gfx950+mfma-i8");
    return FOCR_HIP_OK;
}

// ---- device buffers --------------------------------------------------------

int32_t focr_hip_dmalloc(focr_hip_ctx* ctx, size_t bytes, void** out) {
    CTX_GUARD(ctx);
    if (!out) return fail(FOCR_HIP_E_ARG, "focr_hip_dmalloc: null out");
    *out = nullptr;
    FOCR_HIP_TRY(hipMalloc(out, bytes ? bytes : 16), "hipMalloc");
    return FOCR_HIP_OK;
}

int32_t focr_hip_dfree(focr_hip_ctx* ctx, void* ptr) {
    CTX_GUARD(ctx);
    if (!ptr) return FOCR_HIP_OK;
    FOCR_HIP_TRY(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
    FOCR_HIP_TRY(hipFree(ptr), "hipFree");
    return FOCR_HIP_OK;
}

int32_t focr_hip_h2d(focr_hip_ctx* ctx, void* dst, const void* src, size_t bytes) {
    CTX_GUARD(ctx);
    if (!bytes) return FOCR_HIP_OK;
    if (!dst || !src) return fail(FOCR_HIP_E_ARG, "focr_hip_h2d: null pointer");
    FOCR_HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx->stream), "hipMemcpyAsync H2D");
    FOCR_HIP_TRY(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
    return FOCR_HIP_OK;
}

int32_t focr_hip_d2h(focr_hip_ctx* ctx, void* dst, const void* src, size_t bytes) {
    CTX_GUARD(ctx);
    if (!bytes) return FOCR_HIP_OK;
    if (!dst || !src) return fail(FOCR_HIP_E_ARG, "focr_hip_d2h: null pointer");
    FOCR_HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx->stream), "hipMemcpyAsync D2H");
    FOCR_HIP_TRY(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
    return FOCR_HIP_OK;
}

int32_t focr_hip_d2d(focr_hip_ctx* ctx, void* dst, const void* src, size_t bytes) {
    CTX_GUARD(ctx);
    if (!bytes) return FOCR_HIP_OK;
    if (!dst || !src) return fail(FOCR_HIP_E_ARG, "focr_hip_d2d: null pointer");
    FOCR_HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, ctx->stream), "hipMemcpyAsync D2D");
    return FOCR_HIP_OK;
}

}  // extern "C"

// ---- drop-in tier ----------------------------------------------------------

namespace {

// scalar.rs:79-102 contract, with the entry's own message prefix.
int32_t igemm_contract(const char* ctxname, const void* a, size_t a_len, const void* b, size_t b_len,
                       size_t m, size_t k, size_t n, const void* out, size_t out_len) {
    int32_t st = FOCR_HIP_OK;
    size_t al, bl, ol;
    if (!checked_len(ctxname, m, k, "m*k", &al, &st)) return st;
    if (!checked_len(ctxname, n, k, "n*k", &bl, &st)) return st;
    if (!checked_len(ctxname, m, n, "m*n", &ol, &st)) return st;
    if (a_len != al) return fail(FOCR_HIP_E_SHAPE, fmt("%s: a.len %zu != m*k %zu", ctxname, a_len, al));
    if (b_len != bl) return fail(FOCR_HIP_E_SHAPE, fmt("%s: b.len %zu != n*k %zu", ctxname, b_len, bl));
    if (out_len != ol) return fail(FOCR_HIP_E_SHAPE, fmt("%s: out.len %zu != m*n %zu", ctxname, out_len, ol));
    if ((a_len && !a) || (b_len && !b) || (out_len && !out))
        return fail(FOCR_HIP_E_ARG, fmt("%s: null pointer with a non-zero length", ctxname));
    if (!fits_i32(ctxname, m, "m", &st) || !fits_i32(ctxname, k, "k", &st) || !fits_i32(ctxname, n, "n", &st))
        return st;
    return FOCR_HIP_OK;
}

int32_t igemm_host(focr_hip_ctx* ctx, const char* name, const void* a, size_t a_len, bool a_u8,
                   const int8_t* b, size_t b_len, size_t m, size_t k, size_t n, int32_t* out,
                   size_t out_len) {
    if (!ctx) return fail(FOCR_HIP_E_BAD_HANDLE, "null focr_hip_ctx");
    std::lock_guard<std::mutex> lock(ctx->mu);
    clear_error();
    int32_t st = igemm_contract(name, a, a_len, b, b_len, m, k, n, out, out_len);
    if (st) return st;
    if (out_len == 0) return FOCR_HIP_OK;
    FOCR_HIP_TRY(ctx->bind(), "hipSetDevice");
    void* da = ctx->scratch_get(kScrA, a_len);
    void* db = ctx->scratch_get(kScrB, b_len);
    void* dout = ctx->scratch_get(kScrOut, out_len * sizeof(int32_t));
    if (!da || !db || !dout) return FOCR_HIP_E_OOM;
    hipStream_t s = ctx->stream;
    if (a_len) FOCR_HIP_TRY(hipMemcpyAsync(da, a, a_len, hipMemcpyHostToDevice, s), "H2D a");
    if (b_len) FOCR_HIP_TRY(hipMemcpyAsync(db, b, b_len, hipMemcpyHostToDevice, s), "H2D b");
    FOCR_HIP_TRY(hipMemcpyAsync(dout, out, out_len * sizeof(int32_t), hipMemcpyHostToDevice, s), "H2D out");
    {
        ProfScope ps(ctx, "igemm_i8");
        FOCR_HIP_TRY(launch_igemm_i8(s, da, a_u8, static_cast<const int8_t*>(db), static_cast<int32_t*>(dout),
                                     static_cast<int>(m), static_cast<int>(k), static_cast<int>(n)),
                     "igemm kernel launch");
    }
    FOCR_HIP_TRY(hipMemcpyAsync(out, dout, out_len * sizeof(int32_t), hipMemcpyDeviceToHost, s), "D2H out");
    FOCR_HIP_TRY(hipStreamSynchronize(s), "hipStreamSynchronize");
    return FOCR_HIP_OK;
}

// int4.rs:350-402 assert_packed_shapes (and :180-221 for igemm_s4s8).
int32_t s4_contract(const char* name, const void* a, size_t a_len, const void* b, size_t b_len,
                    const void* sc, size_t s_len, size_t group, size_t m, size_t k, size_t n,
                    const void* out, size_t out_len, bool check_scales_out) {
    int32_t st = FOCR_HIP_OK;
    if (k % 2) return fail(FOCR_HIP_E_SHAPE, fmt("%s: k %zu must be even", name, k));
    if (group != 16 && group != 32) return fail(FOCR_HIP_E_SHAPE, fmt("%s: group %zu must be 16 or 32", name, group));
    if (k % group) return fail(FOCR_HIP_E_SHAPE, fmt("%s: group %zu must divide k %zu", name, group, k));
    const size_t groups = k / group;
    size_t al, bl, sl, ol;
    if (!checked_len(name, m, k, "m*k", &al, &st)) return st;
    if (!checked_len(name, n, k / 2, "n*k/2", &bl, &st)) return st;
    if (!checked_len(name, n, groups, "n*(k/group)", &sl, &st)) return st;
    if (!checked_len(name, m, n, "m*n", &ol, &st)) return st;
    if (a_len != al) return fail(FOCR_HIP_E_SHAPE, fmt("%s: a len %zu != m*k %zu", name, a_len, al));
    if (b_len != bl) return fail(FOCR_HIP_E_SHAPE, fmt("%s: b_packed len %zu != n*k/2 %zu", name, b_len, bl));
    if (check_scales_out) {
        if (s_len != sl) return fail(FOCR_HIP_E_SHAPE, fmt("%s: scales len %zu != n*(k/group) %zu", name, s_len, sl));
        if (out_len != ol) return fail(FOCR_HIP_E_SHAPE, fmt("%s: out len %zu != m*n %zu", name, out_len, ol));
    }
    if ((a_len && !a) || (b_len && !b) || (check_scales_out && ((s_len && !sc) || (out_len && !out))))
        return fail(FOCR_HIP_E_ARG, fmt("%s: null pointer with a non-zero length", name));
    if (!fits_i32(name, m, "m", &st) || !fits_i32(name, k, "k", &st) || !fits_i32(name, n, "n", &st)) return st;
    return FOCR_HIP_OK;
}

// The int4 packed GEMM on the matrix cores when the shape allows it (group
// 16/32, k a multiple of 32 up to 4096), else the per-lane kernel; both give
// the reference's f32 result bit for bit.
hipError_t launch_s4s8_any(focr_hip_ctx* ctx, const int8_t* a, const uint8_t* b, const float* scales, int group,
                           int m, int k, int n, float* out) {
    if (s4_mfma_supported(group, k)) {
        ProfScope ps(ctx, "s4s8_mfma");
        return launch_s4s8_mfma(ctx->stream, a, b, scales, group, m, k, n, out);
    }
    ProfScope ps(ctx, "s4s8_packed");
    return launch_s4s8_packed(ctx->stream, a, b, scales, group, m, k, n, out, nullptr);
}

int32_t s4s8_host(focr_hip_ctx* ctx, const char* name, const int8_t* a, size_t a_len, const uint8_t* b,
                  size_t b_len, const float* scales, size_t s_len, size_t group, size_t m, size_t k, size_t n,
                  float* out, size_t out_len, int32_t* partials, size_t partials_len) {
    if (!ctx) return fail(FOCR_HIP_E_BAD_HANDLE, "null focr_hip_ctx");
    std::lock_guard<std::mutex> lock(ctx->mu);
    clear_error();
    const size_t groups = (group == 16 || group == 32) ? k / group : 0;
    // The debug entry has no scales/out: validate it against a virtual shape.
    const bool debug = partials != nullptr;
    int32_t st = s4_contract(name, a, a_len, b, b_len, scales, s_len, group, m, k, n, out, out_len, !debug);
    if (st) return st;
    if (debug && partials_len != m * n * groups)
        return fail(FOCR_HIP_E_SHAPE, fmt("%s: partials len %zu != m*n*(k/group) %zu", name, partials_len, m * n * groups));
    if (m * n == 0) return FOCR_HIP_OK;
    FOCR_HIP_TRY(ctx->bind(), "hipSetDevice");
    // Row starts must be 4-byte aligned for the packed kernel: k % 8 == 0
    // holds because group in {16, 32} divides k.
    void* da = ctx->scratch_get(kScrA, a_len);
    void* db = ctx->scratch_get(kScrB, b_len);
    void* ds = ctx->scratch_get(kScrAux, std::max<size_t>(n * groups * sizeof(float), 16));
    void* dout = ctx->scratch_get(kScrOut, debug ? m * n * groups * sizeof(int32_t) + m * n * sizeof(float)
                                                 : out_len * sizeof(float));
    if (!da || !db || !ds || !dout) return FOCR_HIP_E_OOM;
    hipStream_t s = ctx->stream;
    FOCR_HIP_TRY(hipMemcpyAsync(da, a, a_len, hipMemcpyHostToDevice, s), "H2D a");
    FOCR_HIP_TRY(hipMemcpyAsync(db, b, b_len, hipMemcpyHostToDevice, s), "H2D b");
    if (!debug) FOCR_HIP_TRY(hipMemcpyAsync(ds, scales, s_len * sizeof(float), hipMemcpyHostToDevice, s), "H2D scales");
    else FOCR_HIP_TRY(hipMemsetAsync(ds, 0, n * groups * sizeof(float), s), "memset scales");
    float* fout = debug ? reinterpret_cast<float*>(static_cast<char*>(dout) + m * n * groups * sizeof(int32_t))
                        : static_cast<float*>(dout);
    int32_t* dpart = debug ? static_cast<int32_t*>(dout) : nullptr;
    if (debug) {
        ProfScope ps(ctx, "s4s8_packed");
        FOCR_HIP_TRY(launch_s4s8_packed(s, static_cast<const int8_t*>(da), static_cast<const uint8_t*>(db),
                                        static_cast<const float*>(ds), static_cast<int>(group), static_cast<int>(m),
                                        static_cast<int>(k), static_cast<int>(n), fout, dpart),
                     "s4s8 kernel launch");
    } else {
        FOCR_HIP_TRY(launch_s4s8_any(ctx, static_cast<const int8_t*>(da), static_cast<const uint8_t*>(db),
                                     static_cast<const float*>(ds), static_cast<int>(group), static_cast<int>(m),
                                     static_cast<int>(k), static_cast<int>(n), fout),
                     "s4s8 kernel launch");
    }
    if (debug)
        FOCR_HIP_TRY(hipMemcpyAsync(partials, dpart, partials_len * sizeof(int32_t), hipMemcpyDeviceToHost, s), "D2H");
    else
        FOCR_HIP_TRY(hipMemcpyAsync(out, fout, out_len * sizeof(float), hipMemcpyDeviceToHost, s), "D2H");
    FOCR_HIP_TRY(hipStreamSynchronize(s), "hipStreamSynchronize");
    return FOCR_HIP_OK;
}

}  // namespace

extern "C" {

int32_t focr_hip_igemm_s8s8(focr_hip_ctx* ctx, const int8_t* a, size_t a_len, const int8_t* b, size_t b_len,
                            size_t m, size_t k, size_t n, int32_t* out, size_t out_len) {
    return igemm_host(ctx, "igemm_s8s8", a, a_len, false, b, b_len, m, k, n, out, out_len);
}

int32_t focr_hip_igemm_u8s8(focr_hip_ctx* ctx, const uint8_t* a, size_t a_len, const int8_t* b, size_t b_len,
                            size_t m, size_t k, size_t n, int32_t* out, size_t out_len) {
    return igemm_host(ctx, "igemm_u8s8", a, a_len, true, b, b_len, m, k, n, out, out_len);
}

int32_t focr_hip_igemm_s4s8_packed(focr_hip_ctx* ctx, const int8_t* a, size_t a_len, const uint8_t* b_packed,
                                   size_t b_len, const float* scales, size_t scales_len, size_t group, size_t m,
                                   size_t k, size_t n, float* out, size_t out_len) {
    return s4s8_host(ctx, "igemm_s4s8_packed", a, a_len, b_packed, b_len, scales, scales_len, group, m, k, n, out,
                     out_len, nullptr, 0);
}

int32_t focr_hip_igemm_s4s8(focr_hip_ctx* ctx, const int8_t* a, size_t a_len, const uint8_t* b_packed,
                            size_t b_len, const float* scales, size_t scales_len, size_t group, size_t m, size_t k,
                            size_t n, float* out, size_t out_len) {
    return s4s8_host(ctx, "igemm_s4s8", a, a_len, b_packed, b_len, scales, scales_len, group, m, k, n, out,
                     out_len, nullptr, 0);
}

int32_t focr_hip_debug_s4s8_group_i32(focr_hip_ctx* ctx, const int8_t* a, size_t a_len, const uint8_t* b_packed,
                                      size_t b_len, size_t group, size_t m, size_t k, size_t n, int32_t* partials,
                                      size_t partials_len) {
    if (!partials && partials_len == 0 && m * n == 0) {
        // nothing to write; still validate the shape
        int32_t dummy = 0;
        return s4s8_host(ctx, "debug_s4s8_group_i32", a, a_len, b_packed, b_len, nullptr, 0, group, m, k, n,
                         nullptr, 0, &dummy, 0);
    }
    if (!partials) return fail(FOCR_HIP_E_ARG, "debug_s4s8_group_i32: null partials");
    return s4s8_host(ctx, "debug_s4s8_group_i32", a, a_len, b_packed, b_len, nullptr, 0, group, m, k, n, nullptr, 0,
                     partials, partials_len);
}

int32_t focr_hip_unpack_to_i8(focr_hip_ctx* ctx, const uint8_t* b_packed, size_t b_len, size_t n, size_t k,
                              int8_t* out, size_t out_len) {
    if (!ctx) return fail(FOCR_HIP_E_BAD_HANDLE, "null focr_hip_ctx");
    std::lock_guard<std::mutex> lock(ctx->mu);
    clear_error();
    int32_t st = FOCR_HIP_OK;
    if (k % 2) return fail(FOCR_HIP_E_SHAPE, fmt("unpack_to_i8: k %zu must be even (two nibbles/byte)", k));
    size_t pl, ol;
    if (!checked_len("unpack_to_i8", n, k / 2, "n*k/2", &pl, &st)) return st;
    if (!checked_len("unpack_to_i8", n, k, "n*k", &ol, &st)) return st;
    if (b_len != pl) return fail(FOCR_HIP_E_SHAPE, fmt("unpack_to_i8: packed len %zu != n*k/2 %zu", b_len, pl));
    if (out_len != ol) return fail(FOCR_HIP_E_SHAPE, fmt("unpack_to_i8: out len %zu != n*k %zu", out_len, ol));
    if (pl == 0) return FOCR_HIP_OK;
    if (!b_packed || !out) return fail(FOCR_HIP_E_ARG, "unpack_to_i8: null pointer");
    FOCR_HIP_TRY(ctx->bind(), "hipSetDevice");
    void* db = ctx->scratch_get(kScrB, pl);
    void* dout = ctx->scratch_get(kScrOut, ol);
    if (!db || !dout) return FOCR_HIP_E_OOM;
    hipStream_t s = ctx->stream;
    FOCR_HIP_TRY(hipMemcpyAsync(db, b_packed, pl, hipMemcpyHostToDevice, s), "H2D");
    FOCR_HIP_TRY(launch_unpack_i4(s, static_cast<const uint8_t*>(db), pl, static_cast<int8_t*>(dout)), "unpack launch");
    FOCR_HIP_TRY(hipMemcpyAsync(out, dout, ol, hipMemcpyDeviceToHost, s), "D2H");
    FOCR_HIP_TRY(hipStreamSynchronize(s), "hipStreamSynchronize");
    return FOCR_HIP_OK;
}

int32_t focr_hip_igemm_s8s8_dev(focr_hip_ctx* ctx, const int8_t* a, const int8_t* b, size_t m, size_t k, size_t n,
                                int32_t* out) {
    CTX_GUARD(ctx);
    int32_t st = FOCR_HIP_OK;
    if (!fits_i32("igemm_s8s8", m, "m", &st) || !fits_i32("igemm_s8s8", k, "k", &st) ||
        !fits_i32("igemm_s8s8", n, "n", &st))
        return st;
    if (m * n && (!a || !b || !out)) return fail(FOCR_HIP_E_ARG, "igemm_s8s8: null device pointer");
    ProfScope ps(ctx, "igemm_i8");
    FOCR_HIP_TRY(launch_igemm_i8(ctx->stream, a, false, b, out, (int)m, (int)k, (int)n), "igemm kernel launch");
    return FOCR_HIP_OK;
}

int32_t focr_hip_igemm_u8s8_dev(focr_hip_ctx* ctx, const uint8_t* a, const int8_t* b, size_t m, size_t k, size_t n,
                                int32_t* out) {
    CTX_GUARD(ctx);
    int32_t st = FOCR_HIP_OK;
    if (!fits_i32("igemm_u8s8", m, "m", &st) || !fits_i32("igemm_u8s8", k, "k", &st) ||
        !fits_i32("igemm_u8s8", n, "n", &st))
        return st;
    if (m * n && (!a || !b || !out)) return fail(FOCR_HIP_E_ARG, "igemm_u8s8: null device pointer");
    ProfScope ps(ctx, "igemm_i8");
    FOCR_HIP_TRY(launch_igemm_i8(ctx->stream, a, true, b, out, (int)m, (int)k, (int)n), "igemm kernel launch");
    return FOCR_HIP_OK;
}

int32_t focr_hip_igemm_s8s8_batched_dev(focr_hip_ctx* ctx, const int8_t* a, const int8_t* b, size_t batch,
                                        size_t m, size_t k, size_t n, int32_t* out) {
    CTX_GUARD(ctx);
    int32_t st = FOCR_HIP_OK;
    if (!fits_i32("igemm_s8s8_batched", m, "m", &st) || !fits_i32("igemm_s8s8_batched", k, "k", &st) ||
        !fits_i32("igemm_s8s8_batched", n, "n", &st))
        return st;
    if (batch > 65535)
        return fail(FOCR_HIP_E_SHAPE, fmt("igemm_s8s8_batched: batch %zu exceeds 65535", batch));
    if (batch * m * n == 0) return FOCR_HIP_OK;
    if (k == 0 || k % 16 || k > 65536)
        return fail(FOCR_HIP_E_SHAPE,
                    fmt("igemm_s8s8_batched: k %zu must be a positive multiple of 16, at most 65536", k));
    if (!a || !b || !out) return fail(FOCR_HIP_E_ARG, "igemm_s8s8_batched: null device pointer");
    if (reinterpret_cast<uintptr_t>(a) % 16 || reinterpret_cast<uintptr_t>(b) % 16)
        return fail(FOCR_HIP_E_ARG, "igemm_s8s8_batched: a and b must be 16-byte aligned");
    ProfScope ps(ctx, "igemm_i8_batched");
    FOCR_HIP_TRY(launch_igemm_i8_batched(ctx->stream, a, b, out, (int)batch, (int)m, (int)k, (int)n),
                 "igemm kernel launch");
    return FOCR_HIP_OK;
}

int32_t focr_hip_igemm_s4s8_packed_dev(focr_hip_ctx* ctx, const int8_t* a, const uint8_t* b_packed,
                                       const float* scales, size_t group, size_t m, size_t k, size_t n, float* out) {
    CTX_GUARD(ctx);
    int32_t st = s4_contract("igemm_s4s8_packed", a, m * k, b_packed, n * (k / 2), scales,
                             (group == 16 || group == 32) ? n * (k / group) : 0, group, m, k, n, out, m * n, true);
    if (st) return st;
    if (m * n == 0) return FOCR_HIP_OK;
    FOCR_HIP_TRY(launch_s4s8_any(ctx, a, b_packed, scales, (int)group, (int)m, (int)k, (int)n, out),
                 "s4s8 kernel launch");
    return FOCR_HIP_OK;
}

// ---- self-test (dispatch.rs:376-429) ----------------------------------------

int32_t focr_hip_selftest(focr_hip_ctx* ctx, char* json, size_t cap, int32_t* all_ok);

}  // extern "C"
