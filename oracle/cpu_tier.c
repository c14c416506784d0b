/*
 * cpu_tier.c — the reference's x86 int8 tier and its threading model,
 * restated in C (CPU baseline only; see cpu_tier.h).
 */
#define _GNU_SOURCE
#include "cpu_tier.h"

#include <immintrin.h>
#include <pthread.h>
#include <stdatomic.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

#include "focr_oracle.h"

/* ---- tier detection (dispatch.rs:179-200) --------------------------------- */
int cpu_detect_tier(void) {
    __builtin_cpu_init();
    if (__builtin_cpu_supports("avx512vnni") && __builtin_cpu_supports("avx512bw") &&
        __builtin_cpu_supports("avx512f"))
        return CPU_TIER_AVX512VNNI;
#if defined(__clang__) || (defined(__GNUC__) && (__GNUC__ >= 11))
    if (__builtin_cpu_supports("avxvnni")) return CPU_TIER_AVXVNNI;
#endif
    if (__builtin_cpu_supports("avx2")) return CPU_TIER_AVX2;
    return CPU_TIER_SCALAR;
}

/* 1 if this host can run the given tier's kernels (each tier needs its own
 * ISA extensions; a lower tier is not implied by a higher one for avxvnni). */
int cpu_tier_available(int tier) {
    __builtin_cpu_init();
    switch (tier) {
    case CPU_TIER_SCALAR: return 1;
    case CPU_TIER_AVX2: return __builtin_cpu_supports("avx2") != 0;
#if defined(__clang__) || (defined(__GNUC__) && (__GNUC__ >= 11))
    case CPU_TIER_AVXVNNI: return __builtin_cpu_supports("avxvnni") != 0;
#endif
    case CPU_TIER_AVX512VNNI:
        return __builtin_cpu_supports("avx512vnni") && __builtin_cpu_supports("avx512bw") &&
               __builtin_cpu_supports("avx512f");
    default: return 0;
    }
}

const char* cpu_tier_tag(int tier) {
    static const char* t[] = {"scalar", "avx2", "avxvnni", "avx512vnni"};
    return (tier >= 0 && tier <= 3) ? t[tier] : "scalar";
}

/* dispatch.rs:72-81 feature_string */
const char* cpu_tier_feature(int tier) {
    static const char* t[] = {"scalar", "x86_64+avx2", "x86_64+avx2+avxvnni", "x86_64+avx512vnni"};
    return (tier >= 0 && tier <= 3) ? t[tier] : "scalar";
}

/* ---- kernels (x86.rs) --------------------------------------------------------- */
static void scalar_s8s8(const int8_t* a, const int8_t* b, size_t m, size_t k, size_t n, int32_t* out) {
    oracle_igemm_s8s8(a, b, m, k, n, out);
}

#define MR 2
#define NR 2

/* x86.rs:327-385: AVX2, i8 -> i16 widening, non-saturating vpmaddwd. */
__attribute__((target("avx2"))) static int32_t hsum256(__m256i v) {
    __m128i s = _mm_add_epi32(_mm256_castsi256_si128(v), _mm256_extracti128_si256(v, 1));
    s = _mm_hadd_epi32(s, s);
    s = _mm_hadd_epi32(s, s);
    return _mm_cvtsi128_si32(s);
}

__attribute__((target("avx2"))) static void avx2_s8s8(const int8_t* a, const int8_t* b, size_t m,
                                                      size_t k, size_t n, int32_t* out) {
    size_t k16 = k - (k % 16);
    for (size_t r0 = 0; r0 < m; r0 += MR) {
        size_t mr = (m - r0) < MR ? (m - r0) : MR;
        for (size_t c0 = 0; c0 < n; c0 += NR) {
            size_t nr = (n - c0) < NR ? (n - c0) : NR;
            __m256i acc[MR][NR];
            for (size_t i = 0; i < MR; ++i)
                for (size_t j = 0; j < NR; ++j) acc[i][j] = _mm256_setzero_si256();
            for (size_t t = 0; t < k16; t += 16) {
                __m256i av[MR], bv[NR];
                for (size_t i = 0; i < mr; ++i)
                    av[i] = _mm256_cvtepi8_epi16(_mm_loadu_si128((const __m128i*)(a + (r0 + i) * k + t)));
                for (size_t j = 0; j < nr; ++j)
                    bv[j] = _mm256_cvtepi8_epi16(_mm_loadu_si128((const __m128i*)(b + (c0 + j) * k + t)));
                for (size_t i = 0; i < mr; ++i)
                    for (size_t j = 0; j < nr; ++j)
                        acc[i][j] = _mm256_add_epi32(acc[i][j], _mm256_madd_epi16(av[i], bv[j]));
            }
            for (size_t i = 0; i < mr; ++i)
                for (size_t j = 0; j < nr; ++j) {
                    int32_t s = hsum256(acc[i][j]);
                    for (size_t tt = k16; tt < k; ++tt)
                        s += (int32_t)a[(r0 + i) * k + tt] * (int32_t)b[(c0 + j) * k + tt];
                    out[(r0 + i) * n + c0 + j] += s;
                }
        }
    }
}

/* x86.rs:549-616: AVX-VNNI dpbusd((a+128), b) - 128*sum(b). */
__attribute__((target("avx2,avxvnni"))) static void avxvnni_s8s8(const int8_t* a, const int8_t* b,
                                                                 size_t m, size_t k, size_t n,
                                                                 int32_t* out) {
    size_t k32 = k - (k % 32);
    const __m256i bias = _mm256_set1_epi8((char)-128);
    for (size_t r0 = 0; r0 < m; r0 += MR) {
        size_t mr = (m - r0) < MR ? (m - r0) : MR;
        for (size_t c0 = 0; c0 < n; c0 += NR) {
            size_t nr = (n - c0) < NR ? (n - c0) : NR;
            __m256i acc[MR][NR];
            for (size_t i = 0; i < MR; ++i)
                for (size_t j = 0; j < NR; ++j) acc[i][j] = _mm256_setzero_si256();
            for (size_t t = 0; t < k32; t += 32) {
                __m256i av[MR], bv[NR];
                for (size_t i = 0; i < mr; ++i)
                    av[i] = _mm256_add_epi8(_mm256_loadu_si256((const __m256i*)(a + (r0 + i) * k + t)), bias);
                for (size_t j = 0; j < nr; ++j) bv[j] = _mm256_loadu_si256((const __m256i*)(b + (c0 + j) * k + t));
                for (size_t i = 0; i < mr; ++i)
                    for (size_t j = 0; j < nr; ++j) acc[i][j] = _mm256_dpbusd_avx_epi32(acc[i][j], av[i], bv[j]);
            }
            for (size_t i = 0; i < mr; ++i)
                for (size_t j = 0; j < nr; ++j) {
                    int32_t s = hsum256(acc[i][j]);
                    int32_t bsum = 0;
                    for (size_t tt = 0; tt < k32; ++tt) bsum += b[(c0 + j) * k + tt];
                    s -= 128 * bsum;
                    for (size_t tt = k32; tt < k; ++tt)
                        s += (int32_t)a[(r0 + i) * k + tt] * (int32_t)b[(c0 + j) * k + tt];
                    out[(r0 + i) * n + c0 + j] += s;
                }
        }
    }
}

/* x86.rs:709-768: AVX-512-VNNI, zmm dpbusd with the +128 correction. */
__attribute__((target("avx512f,avx512bw,avx512vnni"))) static void avx512vnni_s8s8(
    const int8_t* a, const int8_t* b, size_t m, size_t k, size_t n, int32_t* out) {
    size_t k64 = k - (k % 64);
    const __m512i bias = _mm512_set1_epi8((char)-128);
    for (size_t r0 = 0; r0 < m; r0 += MR) {
        size_t mr = (m - r0) < MR ? (m - r0) : MR;
        for (size_t c0 = 0; c0 < n; c0 += NR) {
            size_t nr = (n - c0) < NR ? (n - c0) : NR;
            __m512i acc[MR][NR];
            for (size_t i = 0; i < MR; ++i)
                for (size_t j = 0; j < NR; ++j) acc[i][j] = _mm512_setzero_si512();
            for (size_t t = 0; t < k64; t += 64) {
                __m512i av[MR], bv[NR];
                for (size_t i = 0; i < mr; ++i)
                    av[i] = _mm512_add_epi8(_mm512_loadu_si512((const void*)(a + (r0 + i) * k + t)), bias);
                for (size_t j = 0; j < nr; ++j) bv[j] = _mm512_loadu_si512((const void*)(b + (c0 + j) * k + t));
                for (size_t i = 0; i < mr; ++i)
                    for (size_t j = 0; j < nr; ++j) acc[i][j] = _mm512_dpbusd_epi32(acc[i][j], av[i], bv[j]);
            }
            for (size_t i = 0; i < mr; ++i)
                for (size_t j = 0; j < nr; ++j) {
                    int32_t s = _mm512_reduce_add_epi32(acc[i][j]);
                    int32_t bsum = 0;
                    for (size_t tt = 0; tt < k64; ++tt) bsum += b[(c0 + j) * k + tt];
                    s -= 128 * bsum;
                    for (size_t tt = k64; tt < k; ++tt)
                        s += (int32_t)a[(r0 + i) * k + tt] * (int32_t)b[(c0 + j) * k + tt];
                    out[(r0 + i) * n + c0 + j] += s;
                }
        }
    }
}

void cpu_igemm_s8s8(int tier, const int8_t* a, const int8_t* b, size_t m, size_t k, size_t n, int32_t* out) {
    switch (tier) {
        case CPU_TIER_AVX512VNNI: avx512vnni_s8s8(a, b, m, k, n, out); break;
        case CPU_TIER_AVXVNNI: avxvnni_s8s8(a, b, m, k, n, out); break;
        case CPU_TIER_AVX2: avx2_s8s8(a, b, m, k, n, out); break;
        default: scalar_s8s8(a, b, m, k, n, out); break;
    }
}

/* ---- a small persistent pool (rayon's global pool stand-in) ------------------ */
typedef void (*task_fn)(void* ctx, size_t item);

static struct {
    pthread_mutex_t mu;
    pthread_cond_t cv_work, cv_done;
    int nthreads;
    int started;
    unsigned long gen;
    task_fn fn;
    void* ctx;
    size_t nitems;
    atomic_size_t next;
    int active;
} g_pool = {PTHREAD_MUTEX_INITIALIZER, PTHREAD_COND_INITIALIZER, PTHREAD_COND_INITIALIZER, 0, 0, 0, 0, 0, 0, 0, 0};

static void pool_drain(void) {
    for (;;) {
        size_t i = atomic_fetch_add(&g_pool.next, 1);
        if (i >= g_pool.nitems) break;
        g_pool.fn(g_pool.ctx, i);
    }
}

static void* pool_worker(void* arg) {
    (void)arg;
    unsigned long seen = 0;
    pthread_mutex_lock(&g_pool.mu);
    for (;;) {
        while (g_pool.gen == seen) pthread_cond_wait(&g_pool.cv_work, &g_pool.mu);
        seen = g_pool.gen;
        pthread_mutex_unlock(&g_pool.mu);
        pool_drain();
        pthread_mutex_lock(&g_pool.mu);
        if (--g_pool.active == 0) pthread_cond_signal(&g_pool.cv_done);
    }
    return NULL;
}

int cpu_set_threads(int n) {
    pthread_mutex_lock(&g_pool.mu);
    if (!g_pool.started) g_pool.nthreads = n > 0 ? n : (int)sysconf(_SC_NPROCESSORS_ONLN);
    pthread_mutex_unlock(&g_pool.mu);
    return g_pool.nthreads;
}

int cpu_threads(void) { return g_pool.nthreads ? g_pool.nthreads : cpu_set_threads(0); }

static void pool_start(void) {
    if (g_pool.started) return;
    if (!g_pool.nthreads) g_pool.nthreads = (int)sysconf(_SC_NPROCESSORS_ONLN);
    if (g_pool.nthreads < 1) g_pool.nthreads = 1;
    for (int i = 1; i < g_pool.nthreads; ++i) {
        pthread_t t;
        pthread_create(&t, NULL, pool_worker, NULL);
        pthread_detach(t);
    }
    g_pool.started = 1;
}

/* Run fn(ctx, 0..nitems) over the pool (the caller participates). */
static void pool_for(size_t nitems, task_fn fn, void* ctx) {
    pthread_mutex_lock(&g_pool.mu);
    pool_start();
    g_pool.fn = fn;
    g_pool.ctx = ctx;
    g_pool.nitems = nitems;
    atomic_store(&g_pool.next, 0);
    g_pool.active = g_pool.nthreads - 1;
    g_pool.gen++;
    pthread_cond_broadcast(&g_pool.cv_work);
    pthread_mutex_unlock(&g_pool.mu);
    pool_drain();
    pthread_mutex_lock(&g_pool.mu);
    while (g_pool.active > 0) pthread_cond_wait(&g_pool.cv_done, &g_pool.mu);
    pthread_mutex_unlock(&g_pool.mu);
}

/* ---- GEMV (decoder.rs:1582, :1621-1640, :2703-2747) --------------------------- */
#define GEMV_BLOCK 64

typedef struct {
    int tier;
    const int8_t* xq;
    const float* as;
    size_t m;
    const int8_t* w;
    const float* scales;
    size_t n, k;
    float* y;
} gemv_job;

static void gemv_block(void* p, size_t blk) {
    gemv_job* j = (gemv_job*)p;
    size_t base = blk * GEMV_BLOCK;
    size_t cnt = j->n - base < GEMV_BLOCK ? j->n - base : GEMV_BLOCK;
    int32_t acc[GEMV_BLOCK * 32];
    memset(acc, 0, sizeof(int32_t) * cnt * j->m);
    cpu_igemm_s8s8(j->tier, j->xq, j->w + base * j->k, j->m, j->k, cnt, acc);
    for (size_t r = 0; r < j->m; ++r)
        for (size_t o = 0; o < cnt; ++o) {
            float t = (float)acc[r * cnt + o] * j->as[r];
            j->y[r * j->n + base + o] = t * j->scales[base + o];
        }
}

void cpu_gemv_i8(int tier, const float* x, size_t m, const int8_t* w, const float* scales, size_t n, size_t k,
                 float* y) {
    if (m == 0 || m > 32) return;
    int8_t* xq = (int8_t*)malloc(m * k);
    float as[32];
    for (size_t r = 0; r < m; ++r) as[r] = oracle_quantize_row_i8(x + r * k, k, xq + r * k);
    gemv_job j = {tier, xq, as, m, w, scales, n, k, y};
    pool_for((n + GEMV_BLOCK - 1) / GEMV_BLOCK, gemv_block, &j);
    free(xq);
}

void cpu_lm_head_i8(int tier, const float* x, size_t m, const int8_t* w, const float* scales, size_t n, size_t k,
                    float* logits, uint32_t* argmax) {
    cpu_gemv_i8(tier, x, m, w, scales, n, k, logits);
    for (size_t r = 0; r < m; ++r) oracle_argmax_row(logits + r * n, n, argmax + r);
}

/* ---- MoE decode (decoder.rs:2199-2268 per token) ------------------------------ */
typedef struct {
    int tier;
    const float* x;
    size_t h, inter;
    const uint32_t* idx;
    const float* gates;
    const int8_t *wg, *wu, *wd;
    const float *sg, *su, *sd;
    float* partial; /* [top_k][h] */
} moe_job;

/* decoder.rs:1729-1755: one serial expert on the tier. */
static void expert_serial(int tier, const float* x, size_t h, size_t inter, const int8_t* wg, const float* sg,
                          const int8_t* wu, const float* su, const int8_t* wd, const float* sd, float* y) {
    int8_t* xq = (int8_t*)malloc(h);
    int32_t* acc = (int32_t*)malloc((inter > h ? inter : h) * sizeof(int32_t));
    float* g = (float*)malloc(inter * sizeof(float));
    float* u = (float*)malloc(inter * sizeof(float));
    int8_t* aq = (int8_t*)malloc(inter);
    float as = oracle_quantize_row_i8(x, h, xq);
    memset(acc, 0, inter * sizeof(int32_t));
    cpu_igemm_s8s8(tier, xq, wg, 1, h, inter, acc);
    for (size_t o = 0; o < inter; ++o) g[o] = ((float)acc[o] * as) * sg[o];
    memset(acc, 0, inter * sizeof(int32_t));
    cpu_igemm_s8s8(tier, xq, wu, 1, h, inter, acc);
    for (size_t o = 0; o < inter; ++o) u[o] = ((float)acc[o] * as) * su[o];
    for (size_t i = 0; i < inter; ++i) g[i] = oracle_silu(g[i]) * u[i];
    float as2 = oracle_quantize_row_i8(g, inter, aq);
    memset(acc, 0, h * sizeof(int32_t));
    cpu_igemm_s8s8(tier, aq, wd, 1, inter, h, acc);
    for (size_t o = 0; o < h; ++o) y[o] = ((float)acc[o] * as2) * sd[o];
    free(xq);
    free(acc);
    free(g);
    free(u);
    free(aq);
}

static void moe_slot(void* p, size_t j) {
    moe_job* m = (moe_job*)p;
    size_t e = m->idx[j];
    float* y = m->partial + j * m->h;
    expert_serial(m->tier, m->x, m->h, m->inter, m->wg + e * m->inter * m->h, m->sg + e * m->inter,
                  m->wu + e * m->inter * m->h, m->su + e * m->inter, m->wd + e * m->h * m->inter, m->sd + e * m->h, y);
    for (size_t c = 0; c < m->h; ++c) y[c] *= m->gates[j];
}

int cpu_moe_decode(int tier, const float* hidden, size_t t, size_t h, size_t inter, size_t n_experts, size_t top_k,
                   const float* router, const int8_t* wg, const float* sg, const int8_t* wu, const float* su,
                   const int8_t* wd, const float* sd, int norm_topk, float routed_scale, float* out, uint32_t* idx,
                   float* gates) {
    int st = oracle_route(hidden, t, h, router, n_experts, top_k, norm_topk, routed_scale, idx, gates, NULL);
    if (st) return st;
    float* partial = (float*)malloc(top_k * h * sizeof(float));
    for (size_t tok = 0; tok < t; ++tok) {
        moe_job j = {tier, hidden + tok * h, h, inter, idx + tok * top_k, gates + tok * top_k, wg, wu, wd, sg, su, sd,
                     partial};
        pool_for(top_k, moe_slot, &j);
        float* o = out + tok * h;
        for (size_t c = 0; c < h; ++c) o[c] = 0.0f;
        for (size_t s = 0; s < top_k; ++s)
            for (size_t c = 0; c < h; ++c) o[c] += partial[s * h + c];
    }
    free(partial);
    return 0;
}

/* ---- cfg1 batched: independent products, one task per instance ------------- */
typedef struct {
    int tier;
    const int8_t *a, *b;
    size_t m, k, n;
    int32_t* out;
} batched_job;

static void batched_item(void* p, size_t i) {
    batched_job* j = (batched_job*)p;
    cpu_igemm_s8s8(j->tier, j->a + i * j->m * j->k, j->b + i * j->n * j->k, j->m, j->k, j->n,
                   j->out + i * j->m * j->n);
}

void cpu_igemm_s8s8_batched(int tier, const int8_t* a, const int8_t* b, size_t batch, size_t m, size_t k, size_t n,
                            int32_t* out) {
    batched_job j = {tier, a, b, m, k, n, out};
    pool_for(batch, batched_item, &j);
}

/* ---- nn::linear_int8_dynamic (nn.rs:151-173) on the tier -------------------- */
typedef struct {
    int tier;
    const int8_t* xq;
    const float* xs;
    size_t m, k, n;
    const int8_t* w;
    const float* ws;
    float* y;
} linear_job;

static void linear_block(void* p, size_t blk) {
    linear_job* j = (linear_job*)p;
    size_t base = blk * GEMV_BLOCK;
    size_t cnt = j->n - base < GEMV_BLOCK ? j->n - base : GEMV_BLOCK;
    int32_t* acc = (int32_t*)calloc(j->m * cnt, sizeof(int32_t));
    cpu_igemm_s8s8(j->tier, j->xq, j->w + base * j->k, j->m, j->k, cnt, acc);
    for (size_t r = 0; r < j->m; ++r)
        for (size_t o = 0; o < cnt; ++o) {
            float v = (float)acc[r * cnt + o] * j->xs[r];
            j->y[r * j->n + base + o] = v * j->ws[base + o];
        }
    free(acc);
}

void cpu_linear_i8_dynamic(int tier, const float* x, size_t m, size_t k, const int8_t* w, const float* ws, size_t n,
                           float* y) {
    int8_t* xq = (int8_t*)malloc(m * k);
    float* xs = (float*)malloc(m * sizeof(float));
    for (size_t r = 0; r < m; ++r) xs[r] = oracle_quantize_row_dynamic(x + r * k, k, xq + r * k);
    linear_job j = {tier, xq, xs, m, k, n, w, ws, y};
    pool_for((n + GEMV_BLOCK - 1) / GEMV_BLOCK, linear_block, &j);
    free(xq);
    free(xs);
}

/* ---- decode_mlp_i8 with the shared expert (decoder.rs:2199-2268) -------------
 * Per token: the top-k routed experts and the shared expert as concurrent
 * serial tasks (decoder.rs:2231-2252); the routed outputs scaled by their
 * gates and summed in slot order, the shared output added last. */
typedef struct {
    moe_job routed;
    size_t shared_inter;
    const int8_t *swg, *swu, *swd;
    const float *ssg, *ssu, *ssd;
} moe_shared_job;

typedef struct {
    moe_shared_job* job;
    size_t top_k;
} moe_shared_ctx;

/* task j < top_k: routed slot j; task top_k: the shared expert */
static void moe_shared_task(void* p, size_t j) {
    moe_shared_ctx* c = (moe_shared_ctx*)p;
    moe_shared_job* m = c->job;
    if (j < c->top_k) {
        moe_slot(&m->routed, j);
        return;
    }
    expert_serial(m->routed.tier, m->routed.x, m->routed.h, m->shared_inter, m->swg, m->ssg, m->swu, m->ssu, m->swd,
                  m->ssd, m->routed.partial + c->top_k * m->routed.h);
}

int cpu_moe_decode_shared(int tier, const float* hidden, size_t t, size_t h, size_t inter, size_t n_experts,
                          size_t top_k, const float* router, const int8_t* wg, const float* sg, const int8_t* wu,
                          const float* su, const int8_t* wd, const float* sd, int norm_topk, float routed_scale,
                          const int8_t* swg, const float* ssg, const int8_t* swu, const float* ssu,
                          const int8_t* swd, const float* ssd, size_t shared_inter, float* out, uint32_t* idx,
                          float* gates) {
    int st = oracle_route(hidden, t, h, router, n_experts, top_k, norm_topk, routed_scale, idx, gates, NULL);
    if (st) return st;
    float* partial = (float*)malloc((top_k + 1) * h * sizeof(float));
    for (size_t tok = 0; tok < t; ++tok) {
        moe_shared_job j = {{tier, hidden + tok * h, h, inter, idx + tok * top_k, gates + tok * top_k, wg, wu, wd,
                             sg, su, sd, partial},
                            shared_inter, swg, swu, swd, ssg, ssu, ssd};
        moe_shared_ctx c = {&j, top_k};
        pool_for(top_k + (swg ? 1 : 0), moe_shared_task, &c);
        float* o = out + tok * h;
        for (size_t col = 0; col < h; ++col) o[col] = 0.0f;
        for (size_t s = 0; s < top_k; ++s)
            for (size_t col = 0; col < h; ++col) o[col] += partial[s * h + col];
        if (swg)
            for (size_t col = 0; col < h; ++col) o[col] += partial[top_k * h + col];
    }
    free(partial);
    return 0;
}

/* ---- one decoder layer's batched decode step (decoder.rs:2812-2933) ---------
 * Per-stream RMSNorm; one M = B qkv GEMV over the pool; per stream RoPE at
 * its position, ring write and R-SWA decode attention (single thread, streams
 * one after another, rswa.rs:894-939); one M = B o_proj GEMV; per stream the
 * residual, post-attention RMSNorm, decode_mlp_i8 (MoE + shared) and the
 * second residual. x [b][h] is updated in place. */
int cpu_decoder_layer_step(int tier, float* x, size_t b, const uint32_t* positions, float* const* ref_k,
                           float* const* ref_v, size_t ref_cap, const uint32_t* prefill_len, float* const* ring_k,
                           float* const* ring_v, uint32_t* ring_len, uint32_t* ring_pos, const float* input_ln,
                           const float* post_ln, float eps, float theta, const int8_t* wqkv, const float* sqkv,
                           const int8_t* wo, const float* so, const float* router, size_t n_experts, size_t top_k,
                           size_t inter, const int8_t* wg, const float* sg, const int8_t* wu, const float* su,
                           const int8_t* wd, const float* sd, const int8_t* swg, const float* ssg,
                           const int8_t* swu, const float* ssu, const int8_t* swd, const float* ssd,
                           size_t shared_inter) {
    const size_t h = 1280, nh = 10, hd = 128, dim = nh * hd;
    if (b == 0 || b > 32) return ORACLE_E_SHAPE;
    float* normed = (float*)malloc(b * h * sizeof(float));
    float* qkv = (float*)malloc(b * 3 * dim * sizeof(float));
    float* ctx = (float*)malloc(b * dim * sizeof(float));
    float* attn = (float*)malloc(b * h * sizeof(float));
    float* mlp = (float*)malloc(h * sizeof(float));
    uint32_t idx[64];
    float gates[64];
    int st = ORACLE_OK;
    for (size_t s = 0; s < b; ++s) oracle_rms_norm(x + s * h, h, input_ln, eps, normed + s * h);
    cpu_gemv_i8(tier, normed, b, wqkv, sqkv, 3 * dim, h, qkv);
    for (size_t s = 0; s < b && st == ORACLE_OK; ++s) {
        float* q = qkv + s * 3 * dim;
        uint32_t slot;
        st = oracle_rope(q, nh, hd, positions[s], theta);
        if (st == ORACLE_OK) st = oracle_rope(q + dim, nh, hd, positions[s], theta);
        if (st == ORACLE_OK)
            st = oracle_ring_write(ring_k[s], ring_v[s], &ring_len[s], &ring_pos[s], q + dim, q + 2 * dim, &slot);
        if (st == ORACLE_OK)
            st = oracle_decode_attention(ref_k[s], ref_v[s], ref_cap, prefill_len[s], ring_k[s], ring_v[s],
                                         ring_len[s], q, ctx + s * dim);
    }
    if (st == ORACLE_OK) cpu_gemv_i8(tier, ctx, b, wo, so, h, dim, attn);
    for (size_t s = 0; s < b && st == ORACLE_OK; ++s) {
        float* xs = x + s * h;
        for (size_t c = 0; c < h; ++c) xs[c] = xs[c] + attn[s * h + c];
        oracle_rms_norm(xs, h, post_ln, eps, normed + s * h);
        st = cpu_moe_decode_shared(tier, normed + s * h, 1, h, inter, n_experts, top_k, router, wg, sg, wu, su, wd,
                                   sd, 0, 1.0f, swg, ssg, swu, ssu, swd, ssd, shared_inter, mlp, idx, gates);
        for (size_t c = 0; c < h && st == ORACLE_OK; ++c) xs[c] = xs[c] + mlp[c];
    }
    free(normed);
    free(qkv);
    free(ctx);
    free(attn);
    free(mlp);
    return st;
}
