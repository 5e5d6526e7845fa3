/*
 * attn_oracle.c -- CPU restatement of vantablack's KV-cache attention path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the parity oracle and the CPU
 * baseline.  Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg may load it, and only as the checker (or as the timed CPU baseline),
 * never as the product path.  The product path is the HIP library under
 * vantablack_amd/; it has no CPU fallback.
 *
 * Every function restates one piece of the reference (Zig 0.16, not compiled
 * here: no Zig toolchain exists in this image) with the same loop order, the
 * same f32 arithmetic and no fast-math.  Build flags (oracle/Makefile):
 * -O3 -ffp-contract=off -fno-fast-math, so a*b+c is never fused, matching
 * Zig's default strict float mode.
 *
 * Pinning (what checks each function; tests/test_oracle.py):
 *   vtb_oracle_softmax         math.zig:224-230 KAT, shift invariance, f64 twin
 *   vtb_oracle_argmax          math.zig:252-254 KAT, first-max-wins tie case
 *   vtb_oracle_f16_to_f32      exhaustive 65536-pattern check vs IEEE binary16
 *   vtb_oracle_bf16_to_f32     exhaustive check vs bits<<16 closed form
 *   vtb_oracle_kv_*            kv_cache.zig:198-282 KATs (round trip, shrink)
 *   vtb_oracle_window_start    forward.zig:297-364 KAT + hand cases
 *   vtb_oracle_cpu_attention   forward.zig:297-364 KAT, closed forms (L=1,
 *                              constant K, one-hot score), GQA/window
 *                              invariants, independent numpy f64 formula
 *   vtb_oracle_attention_causal  row b == decode at pos b (bit-exact), f64
 *                              formula, window invariants
 *   vtb_oracle_attention_f64   independent numpy f64 formula
 *   vtb_oracle_pool_*          pool.zig:196-259 "sums chunks" KAT
 *   vtb_oracle_rmsnorm         constant-row closed form, scale invariance,
 *                              f64 formula (tests/test_layer_oracle.py)
 *   vtb_oracle_swiglu / _geglu_approx  f(0) = 0, f(z) - f(-z) = z (odd
 *                              sigmoid / tanh parts), f64 formula
 * The one thing no check pins is the ULP-level rounding of Zig's @exp
 * lowering versus glibc expf; the parity tolerances (1e-5 / 2e-3) absorb it.
 */
#define _GNU_SOURCE
#include <math.h>
#include <pthread.h>
#include <sched.h>
#include <stdatomic.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define VTB_NO_WINDOW SIZE_MAX /* maxInt(usize): sliding window disabled */

/* ---------------------------------------------------------------------- */
/* Upcasts                                                                 */
/* ---------------------------------------------------------------------- */

/* simd.zig:123-126 -- bf16 -> f32 is the 16 bits placed in the high half. */
float vtb_oracle_bf16_to_f32(uint16_t bits) {
    uint32_t w = (uint32_t)bits << 16;
    float f;
    memcpy(&f, &w, 4);
    return f;
}

/* simd.zig:64 / forward.zig:661-666 -- @floatCast(f16 -> f32), exact.
 * Written out from the IEEE-754 binary16 definition (sign, 5-bit exponent,
 * 10-bit fraction; exponent 0 = subnormal, 31 = inf/nan). */
float vtb_oracle_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) << 31;
    uint32_t exp = (h >> 10) & 0x1f;
    uint32_t frac = h & 0x3ff;
    uint32_t w;
    if (exp == 0) {
        if (frac == 0) {
            w = sign;
        } else {
            /* subnormal: value = frac * 2^-24; renormalise */
            int e = -1;
            do {
                frac <<= 1;
                e++;
            } while ((frac & 0x400) == 0);
            frac &= 0x3ff;
            w = sign | ((uint32_t)(127 - 15 - e) << 23) | (frac << 13);
        }
    } else if (exp == 31) {
        w = sign | 0x7f800000u | (frac << 13); /* inf / nan (payload kept) */
    } else {
        w = sign | ((exp + 127 - 15) << 23) | (frac << 13);
    }
    float f;
    memcpy(&f, &w, 4);
    return f;
}

void vtb_oracle_upcast_f16(const uint16_t *src, float *dst, size_t n) {
    for (size_t i = 0; i < n; i++) dst[i] = vtb_oracle_f16_to_f32(src[i]);
}

void vtb_oracle_upcast_bf16(const uint16_t *src, float *dst, size_t n) {
    for (size_t i = 0; i < n; i++) dst[i] = vtb_oracle_bf16_to_f32(src[i]);
}

/* ---------------------------------------------------------------------- */
/* math.zig                                                                */
/* ---------------------------------------------------------------------- */

/* math.zig:85-107 -- math.rope: in-place RoPE of one head (x has head_dim
 * elements) at absolute position pos.  Interleaved pairs (x[i], x[i+1]),
 * i even, rotated by theta = pos * inv_freq with inv_freq = 1 / base^(i/d),
 * all in f32; the exponent i/d is an f32 quotient (:94). */
void vtb_oracle_rope(float *x, size_t head_dim, size_t pos, float base) {
    const float pos_f = (float)pos;
    for (size_t i = 0; i + 1 < head_dim; i += 2) {
        const float e = (float)i / (float)head_dim;
        const float inv_freq = 1.0f / powf(base, e);
        const float theta = pos_f * inv_freq;
        const float c = cosf(theta);
        const float s = sinf(theta);
        const float x0 = x[i];
        const float x1 = x[i + 1];
        x[i] = x0 * c - x1 * s;
        x[i + 1] = x0 * s + x1 * c;
    }
}

/* math.zig:109-133 -- math.ropeHalf: element i pairs with i + d/2, both
 * rotated by theta_i = pos / base^(2i/d), i < d/2. */
void vtb_oracle_rope_half(float *x, size_t head_dim, size_t pos, float base) {
    const size_t half = head_dim / 2;
    const float pos_f = (float)pos;
    for (size_t i = 0; i < half; i++) {
        const float e = (float)(2 * i) / (float)head_dim;
        const float inv_freq = 1.0f / powf(base, e);
        const float theta = pos_f * inv_freq;
        const float c = cosf(theta);
        const float s = sinf(theta);
        const float x0 = x[i];
        const float x1 = x[i + half];
        x[i] = x0 * c - x1 * s;
        x[i + half] = x0 * s + x1 * c;
    }
}

/* The per-pair inverse frequencies both forms use, inv_freq[j] =
 * 1 / base^(2j/d) for j < d/2 (math.zig:95-96 with i = 2j, :124-125). */
void vtb_oracle_rope_inv_freq(float *out, size_t head_dim, float base) {
    for (size_t j = 0; j < head_dim / 2; j++)
        out[j] = 1.0f / powf(base, (float)(2 * j) / (float)head_dim);
}

/* math.zig:11-32 -- math.rmsNorm, in place: the sum of squares in 8 lane
 * accumulators (Vec) reduced in lane order, then the scalar tail; inv =
 * 1/sqrt(ss/n + eps); the vector part scales as v*w*inv, the tail as
 * x*inv*w.  Lane width 8 stands for std.simd.suggestVectorLength(f32) on an
 * AVX2 host; other widths change only the summation order. */
void vtb_oracle_rmsnorm(float *x, const float *w, size_t n, float eps) {
    enum { LANE = 8 };
    float acc[LANE] = {0};
    size_t i = 0;
    for (; i + LANE <= n; i += LANE)
        for (int l = 0; l < LANE; l++) acc[l] += x[i + l] * x[i + l];
    float ss = 0.0f;
    for (int l = 0; l < LANE; l++) ss += acc[l];
    for (; i < n; i++) ss += x[i] * x[i];
    const float inv = 1.0f / sqrtf(ss / (float)n + eps);
    i = 0;
    for (; i + LANE <= n; i += LANE)
        for (int l = 0; l < LANE; l++) x[i + l] = x[i + l] * w[i + l] * inv;
    for (; i < n; i++) x[i] = x[i] * inv * w[i];
}

/* math.zig:154-161 -- math.swiglu: gate = z / (1 + exp(-z)) * up. */
void vtb_oracle_swiglu(float *gate, const float *up, size_t n) {
    for (size_t i = 0; i < n; i++) {
        const float z = gate[i];
        const float silu = z / (1.0f + expf(-z));
        gate[i] = silu * up[i];
    }
}

/* math.zig:166-175 -- math.gegluApprox (tanh-approximate GELU). */
void vtb_oracle_geglu_approx(float *gate, const float *up, size_t n) {
    const float sqrt_2_over_pi = 0.7978845608028654f;
    for (size_t i = 0; i < n; i++) {
        const float z = gate[i];
        const float inner = sqrt_2_over_pi * (z + 0.044715f * z * z * z);
        const float gelu = 0.5f * z * (1.0f + tanhf(inner));
        gate[i] = gelu * up[i];
    }
}

/* math.zig:136-150 -- in-place softmax: max, exp(x-max) with a sequential
 * sum, then multiply by inv = 1/sum (a reciprocal multiply, not a divide). */
void vtb_oracle_softmax(float *x, size_t n) {
    if (n == 0) return;
    float max_v = x[0];
    for (size_t i = 1; i < n; i++)
        if (x[i] > max_v) max_v = x[i];
    float sum = 0.0f;
    for (size_t i = 0; i < n; i++) {
        float e = expf(x[i] - max_v);
        x[i] = e;
        sum += e;
    }
    float inv = 1.0f / sum;
    for (size_t i = 0; i < n; i++) x[i] *= inv;
}

/* math.zig:190-201 -- first maximum wins; 0 for empty input. */
size_t vtb_oracle_argmax(const float *x, size_t n) {
    if (n == 0) return 0;
    size_t best_i = 0;
    float best_v = x[0];
    for (size_t i = 1; i < n; i++) {
        if (x[i] > best_v) {
            best_v = x[i];
            best_i = i;
        }
    }
    return best_i;
}

/* ---------------------------------------------------------------------- */
/* kv_cache.zig                                                            */
/* ---------------------------------------------------------------------- */

/* kv_cache.zig:20-31.  k/v are [n_layers * max_seq * n_kv_heads * head_dim]
 * f32, layer-major; row t of layer l starts at l*max_seq*kv_dim + t*kv_dim
 * (layout doc kv_cache.zig:7-8, perLayer/rowSize :87-93). */
typedef struct {
    size_t n_layers, n_kv_heads, head_dim, max_seq;
    float *k, *v;
    size_t pos;
} vtb_oracle_kv_cache;

static size_t kv_per_layer(const vtb_oracle_kv_cache *c) {
    return c->max_seq * c->n_kv_heads * c->head_dim;
}
static size_t kv_row(const vtb_oracle_kv_cache *c) { return c->n_kv_heads * c->head_dim; }

/* kv_cache.zig:97-111 -- element offset of the slot at `pos` for `layer`.
 * Returns SIZE_MAX where the reference's debug asserts would fire. */
size_t vtb_oracle_kv_slot_offset(const vtb_oracle_kv_cache *c, size_t layer) {
    if (layer >= c->n_layers || c->pos >= c->max_seq) return SIZE_MAX;
    return layer * kv_per_layer(c) + c->pos * kv_row(c);
}

/* kv_cache.zig:116-128 -- element offset of layer `layer`'s prefix. */
size_t vtb_oracle_kv_layer_offset(const vtb_oracle_kv_cache *c, size_t layer) {
    if (layer >= c->n_layers) return SIZE_MAX;
    return layer * kv_per_layer(c);
}

/* kv_cache.zig:130-133 -- returns 0, or 1 where the assert would fire. */
int vtb_oracle_kv_advance(vtb_oracle_kv_cache *c) {
    if (c->pos >= c->max_seq) return 1;
    c->pos += 1;
    return 0;
}

/* kv_cache.zig:147-195 -- compact every layer's live prefix to the smaller
 * per-layer stride (forward copy; destination precedes source).  Returns 0,
 * or 4 (NewMaxSeqBelowPos).  The caller's arrays keep their capacity. */
int vtb_oracle_kv_shrink_to_fit(vtb_oracle_kv_cache *c, size_t new_max_seq) {
    if (new_max_seq >= c->max_seq) return 0;
    if (new_max_seq < c->pos) return 4;
    size_t old_per_layer = kv_per_layer(c);
    size_t new_per_layer = new_max_seq * kv_row(c);
    size_t live = c->pos * kv_row(c);
    for (size_t layer = 1; layer < c->n_layers; layer++) {
        size_t old_off = layer * old_per_layer, new_off = layer * new_per_layer;
        if (live > 0) {
            memmove(c->k + new_off, c->k + old_off, live * sizeof(float));
            memmove(c->v + new_off, c->v + old_off, live * sizeof(float));
        }
    }
    c->max_seq = new_max_seq;
    return 0;
}

/* ---------------------------------------------------------------------- */
/* Attention                                                               */
/* ---------------------------------------------------------------------- */

/* forward.zig:195-203 / prefill.zig:252-258 / forward.zig:475-480. */
size_t vtb_oracle_window_start(size_t pos, size_t sliding_window) {
    if (sliding_window == VTB_NO_WINDOW || pos < sliding_window) return 0;
    return pos - sliding_window + 1;
}

/* The attention fields of LlamaConfig the path reads (model.zig:40-70). */
typedef struct {
    size_t n_heads, n_kv_heads, head_dim, max_seq, sliding_window;
} vtb_oracle_config;

/* Body shared by decode and prefill: one query vector `q` (n_heads*head_dim)
 * at absolute position `cur_pos`, attending rows [window_start, cur_pos] of
 * layer `l`.  `scores` holds n_heads rows of stride `scores_stride`.
 * This is forward.zig:187-228 and prefill.zig:237-287 verbatim in structure:
 * dot in sequential f32, scale applied after the dot, softmax, then the
 * weighted V sum accumulated sequentially over i. */
static void attend_one(const float *q, const vtb_oracle_kv_cache *cache,
                       const vtb_oracle_config *c, size_t l, size_t cur_pos,
                       float *scores_base, size_t scores_stride, float *out) {
    float head_dim_f = (float)c->head_dim;
    float inv_sqrt_hd = 1.0f / sqrtf(head_dim_f);
    size_t seq_len = cur_pos + 1;
    size_t kvr = c->n_kv_heads * c->head_dim;
    const float *k_buf = cache->k + vtb_oracle_kv_layer_offset(cache, l);
    const float *v_buf = cache->v + vtb_oracle_kv_layer_offset(cache, l);
    size_t window_start = vtb_oracle_window_start(cur_pos, c->sliding_window);
    size_t attended_len = seq_len - window_start;

    memset(out, 0, c->n_heads * c->head_dim * sizeof(float));
    for (size_t h = 0; h < c->n_heads; h++) {
        size_t kv_h = (h * c->n_kv_heads) / c->n_heads; /* GQA fan-in */
        const float *q_h = q + h * c->head_dim;
        float *scores = scores_base + h * scores_stride;
        for (size_t i = 0; i < attended_len; i++) {
            size_t t = window_start + i;
            const float *k_th = k_buf + t * kvr + kv_h * c->head_dim;
            float s = 0.0f;
            for (size_t d = 0; d < c->head_dim; d++) s += q_h[d] * k_th[d];
            scores[i] = s * inv_sqrt_hd;
        }
        vtb_oracle_softmax(scores, attended_len);
        float *out_h = out + h * c->head_dim;
        for (size_t i = 0; i < attended_len; i++) {
            size_t t = window_start + i;
            const float *v_th = v_buf + t * kvr + kv_h * c->head_dim;
            float w = scores[i];
            for (size_t d = 0; d < c->head_dim; d++) out_h[d] += w * v_th[d];
        }
    }
}

/* forward.zig:187-228 cpuAttention.  q: [n_heads*head_dim]; the query sits at
 * cache->pos, whose K/V row the caller has already written (forward.zig:
 * 267-270).  scores: [n_heads * c->max_seq] scratch (State.attn_scores,
 * stride max_seq as at forward.zig:209).  attn_out: [n_heads*head_dim]. */
int vtb_oracle_cpu_attention(const float *q, const vtb_oracle_kv_cache *cache,
                             const vtb_oracle_config *c, size_t l, float *scores,
                             float *attn_out) {
    if (l >= cache->n_layers || cache->pos >= cache->max_seq) return 1;
    attend_one(q, cache, c, l, cache->pos, scores, c->max_seq, attn_out);
    return 0;
}

/* prefill.zig:237-287 attentionCausal for batch position b: the query is
 * q_all[b*(n_heads*head_dim)], at cur_pos = cache->pos + b, writing
 * attn_out_all[b*dim] with dim = n_heads*head_dim.  The caller has written
 * all B rows into the cache first (prefill.zig:175-191).  `scores` is one
 * [n_heads * max_seq] row (the reference's [B, n_heads*max_seq] scratch of
 * prefill.zig:87 is only ever used one b at a time). */
int vtb_oracle_attention_causal(const float *q_all, const vtb_oracle_kv_cache *cache,
                                const vtb_oracle_config *c, size_t l, size_t b,
                                float *scores, float *attn_out_all) {
    size_t cur_pos = cache->pos + b;
    if (l >= cache->n_layers || cur_pos >= cache->max_seq) return 1;
    size_t qd = c->n_heads * c->head_dim;
    attend_one(q_all + b * qd, cache, c, l, cur_pos, scores, c->max_seq,
               attn_out_all + b * qd);
    return 0;
}

/* f64 twin of attend_one (same indexing, double accumulation, libm exp) used
 * for error analysis of the f32 restatement and of the GPU kernels. */
int vtb_oracle_attention_f64(const float *q, const vtb_oracle_kv_cache *cache,
                             const vtb_oracle_config *c, size_t l, size_t cur_pos,
                             double *out) {
    if (l >= cache->n_layers || cur_pos >= cache->max_seq) return 1;
    size_t kvr = c->n_kv_heads * c->head_dim;
    const float *k_buf = cache->k + vtb_oracle_kv_layer_offset(cache, l);
    const float *v_buf = cache->v + vtb_oracle_kv_layer_offset(cache, l);
    size_t ws = vtb_oracle_window_start(cur_pos, c->sliding_window);
    size_t L = cur_pos + 1 - ws;
    double scale = 1.0 / sqrt((double)c->head_dim);
    double *s = (double *)malloc(L * sizeof(double));
    if (!s) return 2;
    memset(out, 0, c->n_heads * c->head_dim * sizeof(double));
    for (size_t h = 0; h < c->n_heads; h++) {
        size_t kv_h = (h * c->n_kv_heads) / c->n_heads;
        const float *q_h = q + h * c->head_dim;
        double mx = -INFINITY, sum = 0.0;
        for (size_t i = 0; i < L; i++) {
            const float *k_th = k_buf + (ws + i) * kvr + kv_h * c->head_dim;
            double acc = 0.0;
            for (size_t d = 0; d < c->head_dim; d++) acc += (double)q_h[d] * (double)k_th[d];
            s[i] = acc * scale;
            if (s[i] > mx) mx = s[i];
        }
        for (size_t i = 0; i < L; i++) {
            s[i] = exp(s[i] - mx);
            sum += s[i];
        }
        double *o = out + h * c->head_dim;
        for (size_t i = 0; i < L; i++) {
            const float *v_th = v_buf + (ws + i) * kvr + kv_h * c->head_dim;
            double w = s[i] / sum;
            for (size_t d = 0; d < c->head_dim; d++) o[d] += w * (double)v_th[d];
        }
    }
    free(s);
    return 0;
}

/* ---------------------------------------------------------------------- */
/* pool.zig -- persistent spin/yield pool, used only for the CPU baseline  */
/* ---------------------------------------------------------------------- */

typedef void (*vtb_oracle_job_fn)(size_t worker_id, size_t n_workers, void *ctx);

typedef struct vtb_oracle_pool {
    pthread_t *threads;
    size_t n_workers; /* includes the caller as worker 0 */
    _Atomic size_t n_active;
    _Atomic uint64_t epoch;
    _Atomic uint64_t completed;
    _Atomic(vtb_oracle_job_fn) job_fn;
    _Atomic(void *) job_ctx;
    _Atomic int shutdown;
} vtb_oracle_pool;

typedef struct {
    vtb_oracle_pool *pool;
    size_t worker_id;
} pool_arg;

/* pool.zig:145: spin this many times before yielding. */
#define IDLE_SPIN_THRESHOLD 1024u

/* pool.zig:147-177 workerLoop. */
static void *pool_worker(void *p) {
    pool_arg *a = (pool_arg *)p;
    vtb_oracle_pool *pool = a->pool;
    size_t worker_id = a->worker_id;
    free(a);
    uint64_t seen = 0;
    for (;;) {
        unsigned spins = 0;
        for (;;) {
            uint64_t e = atomic_load_explicit(&pool->epoch, memory_order_acquire);
            if (e != seen) {
                seen = e;
                break;
            }
            if (atomic_load_explicit(&pool->shutdown, memory_order_acquire)) return NULL;
            if (spins < IDLE_SPIN_THRESHOLD) {
                __builtin_ia32_pause();
                spins++;
            } else {
                sched_yield();
            }
        }
        if (atomic_load_explicit(&pool->shutdown, memory_order_acquire)) return NULL;
        vtb_oracle_job_fn fn = atomic_load_explicit(&pool->job_fn, memory_order_acquire);
        if (fn) {
            size_t active = atomic_load_explicit(&pool->n_active, memory_order_acquire);
            if (worker_id < active)
                fn(worker_id, active, atomic_load_explicit(&pool->job_ctx, memory_order_acquire));
            atomic_fetch_add_explicit(&pool->completed, 1, memory_order_release);
        }
    }
}

/* pool.zig:44-76 init; requested==0 -> (ncpu+1)/2 as at pool.zig:53. */
vtb_oracle_pool *vtb_oracle_pool_init(size_t requested, size_t ncpu) {
    size_t n = requested ? requested : ((ncpu + 1) / 2 > 0 ? (ncpu + 1) / 2 : 1);
    vtb_oracle_pool *pool = (vtb_oracle_pool *)calloc(1, sizeof(*pool));
    if (!pool) return NULL;
    pool->n_workers = n;
    atomic_store(&pool->n_active, n);
    if (n > 1) {
        pool->threads = (pthread_t *)calloc(n - 1, sizeof(pthread_t));
        for (size_t i = 1; i < n; i++) {
            pool_arg *a = (pool_arg *)malloc(sizeof(pool_arg));
            a->pool = pool;
            a->worker_id = i;
            pthread_create(&pool->threads[i - 1], NULL, pool_worker, a);
        }
    }
    return pool;
}

void vtb_oracle_pool_deinit(vtb_oracle_pool *pool) {
    if (!pool) return;
    atomic_store_explicit(&pool->shutdown, 1, memory_order_release);
    atomic_fetch_add_explicit(&pool->epoch, 1, memory_order_release);
    for (size_t i = 1; i < pool->n_workers; i++) pthread_join(pool->threads[i - 1], NULL);
    free(pool->threads);
    free(pool);
}

size_t vtb_oracle_pool_workers(const vtb_oracle_pool *pool) { return pool->n_workers; }

/* pool.zig:127-130. */
void vtb_oracle_pool_set_active(vtb_oracle_pool *pool, size_t target) {
    size_t t = target < 1 ? 1 : (target > pool->n_workers ? pool->n_workers : target);
    atomic_store_explicit(&pool->n_active, t, memory_order_release);
}

/* pool.zig:92-114 dispatch: bump the epoch, run worker 0 inline, spin until
 * every spawned worker has acknowledged the epoch. */
void vtb_oracle_pool_dispatch(vtb_oracle_pool *pool, vtb_oracle_job_fn fn, void *ctx) {
    size_t active = atomic_load_explicit(&pool->n_active, memory_order_acquire);
    if (pool->n_workers == 1 || active == 1) {
        fn(0, 1, ctx);
        return;
    }
    atomic_store_explicit(&pool->job_ctx, ctx, memory_order_release);
    atomic_store_explicit(&pool->job_fn, fn, memory_order_release);
    atomic_store_explicit(&pool->completed, 0, memory_order_release);
    atomic_fetch_add_explicit(&pool->epoch, 1, memory_order_release);
    fn(0, active, ctx);
    uint64_t target = pool->n_workers - 1;
    while (atomic_load_explicit(&pool->completed, memory_order_acquire) < target)
        __builtin_ia32_pause();
    atomic_store_explicit(&pool->job_fn, NULL, memory_order_release);
}

/* pool.zig:196-221 "ThreadPool sums chunks" job, exported for its KAT. */
typedef struct {
    const uint32_t *inputs;
    size_t n;
    uint64_t *partials;
} sum_ctx;

static void sum_worker(size_t wid, size_t nw, void *p) {
    sum_ctx *s = (sum_ctx *)p;
    size_t chunk = (s->n + nw - 1) / nw;
    size_t start = wid * chunk, end = start + chunk < s->n ? start + chunk : s->n;
    uint64_t acc = 0;
    for (size_t i = start; i < end; i++) acc += s->inputs[i];
    s->partials[wid] = acc;
}

uint64_t vtb_oracle_pool_sum(vtb_oracle_pool *pool, const uint32_t *inputs, size_t n) {
    uint64_t partials[256] = {0};
    if (pool->n_workers > 256) return 0;
    sum_ctx s = {inputs, n, partials};
    vtb_oracle_pool_dispatch(pool, sum_worker, &s);
    uint64_t total = 0;
    for (size_t i = 0; i < pool->n_workers; i++) total += partials[i];
    return total;
}

/* ---------------------------------------------------------------------- */
/* Pooled attention: the CPU baseline's parallel line.  vantablack itself  */
/* runs attention single-threaded (cpuAttention never calls the pool); this */
/* splits the same per-head loop over pool workers, each head's score row  */
/* being disjoint (stride max_seq), so results are bit-identical.          */
/* ---------------------------------------------------------------------- */

typedef struct {
    const float *q;
    const vtb_oracle_kv_cache *cache;
    const vtb_oracle_config *c;
    size_t l, cur_pos;
    float *scores, *out;
} attn_job;

static void attn_worker(size_t wid, size_t nw, void *p) {
    attn_job *j = (attn_job *)p;
    size_t H = j->c->n_heads;
    size_t chunk = (H + nw - 1) / nw;
    size_t h0 = wid * chunk, h1 = h0 + chunk < H ? h0 + chunk : H;
    if (h0 >= h1) return;
    /* attend_one restricted to heads [h0, h1): run it on a sub-config whose
     * head range is shifted, keeping the GQA map of the full config. */
    float head_dim_f = (float)j->c->head_dim;
    float inv_sqrt_hd = 1.0f / sqrtf(head_dim_f);
    const vtb_oracle_config *c = j->c;
    size_t kvr = c->n_kv_heads * c->head_dim;
    const float *k_buf = j->cache->k + vtb_oracle_kv_layer_offset(j->cache, j->l);
    const float *v_buf = j->cache->v + vtb_oracle_kv_layer_offset(j->cache, j->l);
    size_t ws = vtb_oracle_window_start(j->cur_pos, c->sliding_window);
    size_t L = j->cur_pos + 1 - ws;
    for (size_t h = h0; h < h1; h++) {
        size_t kv_h = (h * c->n_kv_heads) / c->n_heads;
        const float *q_h = j->q + h * c->head_dim;
        float *scores = j->scores + h * c->max_seq;
        for (size_t i = 0; i < L; i++) {
            const float *k_th = k_buf + (ws + i) * kvr + kv_h * c->head_dim;
            float s = 0.0f;
            for (size_t d = 0; d < c->head_dim; d++) s += q_h[d] * k_th[d];
            scores[i] = s * inv_sqrt_hd;
        }
        vtb_oracle_softmax(scores, L);
        float *out_h = j->out + h * c->head_dim;
        memset(out_h, 0, c->head_dim * sizeof(float));
        for (size_t i = 0; i < L; i++) {
            const float *v_th = v_buf + (ws + i) * kvr + kv_h * c->head_dim;
            float w = scores[i];
            for (size_t d = 0; d < c->head_dim; d++) out_h[d] += w * v_th[d];
        }
    }
}

int vtb_oracle_cpu_attention_pooled(vtb_oracle_pool *pool, const float *q,
                                    const vtb_oracle_kv_cache *cache,
                                    const vtb_oracle_config *c, size_t l, size_t cur_pos,
                                    float *scores, float *attn_out) {
    if (l >= cache->n_layers || cur_pos >= cache->max_seq) return 1;
    attn_job j = {q, cache, c, l, cur_pos, scores, attn_out};
    vtb_oracle_pool_dispatch(pool, attn_worker, &j);
    return 0;
}
