/*
 * fnkv CPU oracle — TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the reference's 8-bit KV path, used only by tests/, by __graft_entry__.smoke() and by
 * bench.py's cpu_baseline leg, always as the checker (or the timed CPU baseline), never as the product. The product is
 * the HIP library under fnfl-v100_amd/; nothing there links or calls this file.
 *
 * What each function restates (paths relative to the reference checkout):
 *   or_f32_to_f16 / or_f16_to_f32   ggml/src/ggml-impl.h:391-438 (fp32 <-> fp16, round to nearest even, subnormals,
 *                                   NaN -> 0x7e00 | sign); fn/quant/kv_q8_ref.cpp:10-43 is the same rounding.
 *   or_q8_0_quantize                ggml/src/ggml-quants.c:274-297 quantize_row_q8_0_ref (blocks of 32:
 *                                   d = amax / 127, id = d ? 1 / d : 0, qs = roundf(x * id), stored fp16(d)).
 *   or_q8_0_dequantize              ggml/src/ggml-quants.c:551-565 dequantize_row_q8_0 (y = qs * fp32(d)).
 *   or_kv8_quantize                 fn/quant/kv_q8_ref.cpp:72-93 (FNFL's group-64 rule: s = fp16(amax / 127),
 *                                   code = clamp(nearbyint(x / s), -127, 127)).
 *   or_pages_*                      fn/model/kv_pool.cpp:85-144 kv_pages (pages_for, take, give, physical).
 *   or_reclaim_victim               fn/model/kv_pool.cpp:146-158 kv_reclaim_victim.
 *   or_attn_f64, or_attn_f64_mt     fn/kernels/qsa/qa2_test.cpp:532-583, the FP64 attention form (scores q.k / 16,
 *                                   max-subtracted exp, sum, normalise) over the DECODED cache, made dense and causal;
 *                                   _mt spreads the (row, KV head) pairs over threads, the same bits.
 *   or_attn_ggml                    ggml-cpu's flash attention over Q8_0 K/V as the pinned llama.cpp runs it (source
 *                                   not in the checkout; restated from its published algorithm): F32 online softmax
 *                                   per query row over keys in order, K rows dequantized (or Q quantized to Q8_0 and
 *                                   dotted block by block when q_as_q8 is set), V rows dequantized to F32 and
 *                                   accumulated, output normalised and rounded to FP16. Threads over (token, head).
 *
 * Which checks pin each function is listed in tests/test_oracle.py.
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define OR_QK 32

static inline uint32_t f2u(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}
static inline float u2f(uint32_t u) {
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* fp32 -> fp16 bits, round to nearest even, by integer arithmetic on the fields */
uint16_t or_f32_to_f16(float f) {
    const uint32_t x = f2u(f);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t e8 = (x >> 23) & 0xffu;
    uint32_t m = x & 0x7fffffu;
    if (e8 == 0xffu) {
        return (uint16_t)(m ? (sign | 0x7e00u) : (sign | 0x7c00u));
    }
    const int32_t e = (int32_t)e8 - 127; /* unbiased */
    if (e > 15) {
        return (uint16_t)(sign | 0x7c00u);
    }
    if (e >= -14) {
        /* normal half: 10 mantissa bits kept, 13 dropped */
        uint32_t h = ((uint32_t)(e + 15) << 10) | (m >> 13);
        const uint32_t rem = m & 0x1fffu;
        if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) {
            h += 1; /* may carry into the exponent, up to inf: correct */
        }
        return (uint16_t)(sign | h);
    }
    /* subnormal half: value = mant * 2^-24 */
    if (e < -25) {
        return (uint16_t)sign; /* below half of the smallest subnormal */
    }
    m |= (e8 ? 0x800000u : 0u); /* an f32 subnormal is far below the range and handled above */
    const uint32_t shift = (uint32_t)(-e - 14 + 13); /* 14 .. 24 */
    uint32_t h = m >> shift;
    const uint32_t rem = m & ((1u << shift) - 1u);
    const uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (h & 1u))) {
        h += 1;
    }
    return (uint16_t)(sign | h);
}

float or_f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1fu;
    const uint32_t m = h & 0x3ffu;
    if (e == 0x1fu) {
        return u2f(sign | 0x7f800000u | (m ? 0x400000u : 0u) | (m << 13)); /* a NaN comes back quiet */
    }
    if (e == 0) {
        /* exact: m * 2^-24 */
        const float v = (float)m * 5.9604644775390625e-08f;
        return sign ? -v : v;
    }
    return u2f(sign | ((e + 112u) << 23) | (m << 13));
}

void or_f32_to_f16_n(const float * x, int64_t n, uint16_t * y) {
    for (int64_t i = 0; i < n; ++i) y[i] = or_f32_to_f16(x[i]);
}
void or_f16_to_f32_n(const uint16_t * x, int64_t n, float * y) {
    for (int64_t i = 0; i < n; ++i) y[i] = or_f16_to_f32(x[i]);
}

/* quantize_row_q8_0_ref, structure-of-arrays output: codes qs[k], scales d[k / 32] */
void or_q8_0_quantize(const float * x, int64_t k, int8_t * qs, uint16_t * d) {
    const int64_t nb = k / OR_QK;
    for (int64_t i = 0; i < nb; ++i) {
        float amax = 0.0f;
        for (int j = 0; j < OR_QK; ++j) {
            const float a = fabsf(x[i * OR_QK + j]);
            amax = amax > a ? amax : a;
        }
        const float dd = amax / 127.0f;
        const float id = dd != 0.0f ? 1.0f / dd : 0.0f;
        d[i] = or_f32_to_f16(dd);
        for (int j = 0; j < OR_QK; ++j) {
            const float v = x[i * OR_QK + j] * id;
            qs[i * OR_QK + j] = (int8_t)roundf(v);
        }
    }
}

void or_q8_0_dequantize(const int8_t * qs, const uint16_t * d, int64_t k, float * y) {
    for (int64_t i = 0; i < k / OR_QK; ++i) {
        const float s = or_f16_to_f32(d[i]);
        for (int j = 0; j < OR_QK; ++j) y[i * OR_QK + j] = (float)qs[i * OR_QK + j] * s;
    }
}

/* FNFL's KV8 rule (groups of 64) */
void or_kv8_quantize(const float * x, int64_t n, int8_t * codes, uint16_t * scales) {
    for (int64_t g = 0; g < n / 64; ++g) {
        float amax = 0.0f;
        for (int i = 0; i < 64; ++i) amax = fmaxf(amax, fabsf(x[g * 64 + i]));
        scales[g] = or_f32_to_f16(amax / 127.0f);
        const float s = or_f16_to_f32(scales[g]);
        for (int i = 0; i < 64; ++i) {
            int q = 0;
            if (s > 0.0f) {
                const float r = nearbyintf(x[g * 64 + i] / s);
                q = r < -127.0f ? -127 : r > 127.0f ? 127 : (int)r;
            }
            codes[g * 64 + i] = (int8_t)q;
        }
    }
}

/* ---- the page book (kv_pages) ---- */

typedef struct {
    int32_t n_slots, n_pages;
    int32_t * map;    /* [n_slots][n_pages] physical page of each logical page */
    int32_t * mapped; /* [n_slots] */
    int32_t * freel;  /* ascending */
    int32_t n_free;
} or_pages;

or_pages * or_pages_new(int32_t n_slots, int32_t n_pages) {
    or_pages * p = (or_pages *)calloc(1, sizeof(or_pages));
    p->n_slots = n_slots < 0 ? 0 : n_slots;
    p->n_pages = n_pages < 0 ? 0 : n_pages;
    p->map = (int32_t *)calloc((size_t)p->n_slots * (size_t)(p->n_pages ? p->n_pages : 1), 4);
    p->mapped = (int32_t *)calloc((size_t)(p->n_slots ? p->n_slots : 1), 4);
    p->freel = (int32_t *)calloc((size_t)(p->n_pages ? p->n_pages : 1), 4);
    for (int32_t i = 0; i < p->n_pages; ++i) p->freel[i] = i;
    p->n_free = p->n_pages;
    return p;
}
void or_pages_free(or_pages * p) {
    if (!p) return;
    free(p->map);
    free(p->mapped);
    free(p->freel);
    free(p);
}
int32_t or_pages_free_count(const or_pages * p) { return p->n_free; }
int32_t or_pages_mapped(const or_pages * p, int32_t slot) {
    return (slot < 0 || slot >= p->n_slots) ? 0 : p->mapped[slot];
}
int32_t or_pages_physical(const or_pages * p, int32_t slot, int32_t logical) {
    if (slot < 0 || slot >= p->n_slots || logical < 0 || logical >= p->mapped[slot]) return -1;
    return p->map[(int64_t)slot * p->n_pages + logical];
}
int32_t or_pages_for(int64_t cells, int32_t page_cells, int32_t n_pages) {
    if (cells <= 0 || page_cells <= 0) return 0;
    const int64_t n = (cells + page_cells - 1) / page_cells;
    return (int32_t)(n < n_pages ? n : n_pages);
}
/* 1 on success; the physical pages taken written to taken[*n_taken] */
int32_t or_pages_take(or_pages * p, int32_t slot, int32_t want, int32_t * taken, int32_t * n_taken) {
    *n_taken = 0;
    if (slot < 0 || slot >= p->n_slots || want > p->n_pages) return 0;
    const int32_t need = want - p->mapped[slot];
    if (need <= 0) return 1;
    if (need > p->n_free) return 0;
    for (int32_t i = 0; i < need; ++i) {
        taken[i] = p->freel[i];
        p->map[(int64_t)slot * p->n_pages + p->mapped[slot] + i] = p->freel[i];
    }
    memmove(p->freel, p->freel + need, (size_t)(p->n_free - need) * 4);
    p->n_free -= need;
    p->mapped[slot] += need;
    *n_taken = need;
    return 1;
}
static int cmp_i32(const void * a, const void * b) {
    const int32_t x = *(const int32_t *)a, y = *(const int32_t *)b;
    return (x > y) - (x < y);
}
/* the slot's logical pages keep .. mapped - 1, last first, into out[*n_out]; the free list re-sorted ascending */
void or_pages_give(or_pages * p, int32_t slot, int32_t keep, int32_t * out, int32_t * n_out) {
    *n_out = 0;
    if (slot < 0 || slot >= p->n_slots) return;
    if (keep < 0) keep = 0;
    while (p->mapped[slot] > keep) {
        const int32_t ph = p->map[(int64_t)slot * p->n_pages + p->mapped[slot] - 1];
        out[(*n_out)++] = ph;
        p->freel[p->n_free++] = ph;
        p->mapped[slot] -= 1;
    }
    qsort(p->freel, (size_t)p->n_free, 4, cmp_i32);
}

int32_t or_reclaim_victim(const uint8_t * active, const int32_t * pages, const uint64_t * released, int32_t n,
                          int32_t for_slot) {
    int32_t victim = -1;
    for (int32_t i = 0; i < n; ++i) {
        if (i == for_slot || active[i] || pages[i] == 0) continue;
        if (victim < 0 || released[i] < released[victim]) victim = i;
    }
    return victim;
}

/* ---- attention ---- */

/*
 * FP64 dense causal attention over the decoded cache.
 *   q     fp16 bits [T][hq][d]; query t sits at position n_ctx - T + t and sees keys 0 .. n_ctx - T + t
 *   k, v  decoded f32 [n_ctx][hkv][d]
 *   rows  query tokens to evaluate (n_rows of them; NULL: all T)
 *   out   f64 [n_rows][hq][d]
 */
/* One (row, KV head) of or_attn_f64: the group's query heads side by side (each head's dot products, maxima, sums and
 * accumulators in the same order as one head alone, so the result is the same bits), s: [n_ctx][grp] scratch. */
static void attn_f64_row_group(const uint16_t * q, const float * k, const float * v, int32_t n_ctx, int32_t T,
                               int32_t hq, int32_t hkv, int32_t d, double scale, int32_t t, int32_t kh, double * s,
                               double * qd, double * out_row) {
    const int32_t grp = hq / hkv;
    const int32_t last = n_ctx - T + t;
    for (int32_t g = 0; g < grp; ++g) {
        const int32_t h = kh * grp + g;
        for (int32_t e = 0; e < d; ++e) qd[(int64_t)e * grp + g] = (double)or_f16_to_f32(q[((int64_t)t * hq + h) * d + e]);
    }
    double m[64], l[64];
    for (int32_t g = 0; g < grp; ++g) {
        m[g] = -INFINITY;
        l[g] = 0.0;
    }
    for (int32_t c = 0; c <= last; ++c) {
        const float * kr = k + ((int64_t)c * hkv + kh) * d;
        double acc[64];
        for (int32_t g = 0; g < grp; ++g) acc[g] = 0.0;
        for (int32_t e = 0; e < d; ++e) { /* each head's sum in the order e = 0, 1, ...; the heads side by side */
            const double ke = (double)kr[e];
            for (int32_t g = 0; g < grp; ++g) acc[g] += qd[(int64_t)e * grp + g] * ke;
        }
        for (int32_t g = 0; g < grp; ++g) {
            const double sc = acc[g] * scale;
            s[(int64_t)c * grp + g] = sc;
            if (sc > m[g]) m[g] = sc;
        }
    }
    for (int32_t g = 0; g < grp; ++g) {
        double * o = out_row + (int64_t)(kh * grp + g) * d;
        for (int32_t e = 0; e < d; ++e) o[e] = 0.0;
    }
    for (int32_t c = 0; c <= last; ++c) {
        const float * vr = v + ((int64_t)c * hkv + kh) * d;
        for (int32_t g = 0; g < grp; ++g) {
            const double p = exp(s[(int64_t)c * grp + g] - m[g]);
            l[g] += p;
            double * o = out_row + (int64_t)(kh * grp + g) * d;
            for (int32_t e = 0; e < d; ++e) o[e] += p * (double)vr[e];
        }
    }
    for (int32_t g = 0; g < grp; ++g) {
        double * o = out_row + (int64_t)(kh * grp + g) * d;
        for (int32_t e = 0; e < d; ++e) o[e] /= l[g];
    }
}

typedef struct {
    const uint16_t * q;
    const float * k;
    const float * v;
    int32_t n_ctx, T, hq, hkv, d;
    double scale;
    const int32_t * rows;
    int32_t n_rows;
    double * out;
    int32_t next; /* the next (row, KV head) job */
    pthread_mutex_t mu;
} attn_f64_job;

static void * attn_f64_worker(void * arg) {
    attn_f64_job * j = (attn_f64_job *)arg;
    const int32_t grp = j->hq / j->hkv;
    double * s = (double *)malloc(sizeof(double) * (size_t)(j->n_ctx > 0 ? j->n_ctx : 1) * (size_t)grp);
    double * qd = (double *)malloc(sizeof(double) * (size_t)j->d * (size_t)grp);
    const int32_t jobs = j->n_rows * j->hkv;
    for (;;) {
        pthread_mutex_lock(&j->mu);
        const int32_t i = j->next++;
        pthread_mutex_unlock(&j->mu);
        if (i >= jobs) break;
        const int32_t ri = i / j->hkv, kh = i % j->hkv;
        const int32_t t = j->rows ? j->rows[ri] : ri;
        attn_f64_row_group(j->q, j->k, j->v, j->n_ctx, j->T, j->hq, j->hkv, j->d, j->scale, t, kh, s, qd,
                           j->out + (int64_t)ri * j->hq * j->d);
    }
    free(s);
    free(qd);
    return NULL;
}

/* or_attn_f64 over `threads` threads, one (row, KV head) a job: the same bits as one thread */
void or_attn_f64_mt(const uint16_t * q, const float * k, const float * v, int32_t n_ctx, int32_t T, int32_t hq,
                    int32_t hkv, int32_t d, double scale, const int32_t * rows, int32_t n_rows, double * out,
                    int32_t threads) {
    if (hkv <= 0 || hq % hkv != 0 || hq / hkv > 64) { /* the group's statistics are held in arrays of 64 */
        const int32_t nr = rows ? n_rows : T;
        for (int64_t i = 0; i < (int64_t)nr * hq * d; ++i) out[i] = NAN;
        return;
    }
    attn_f64_job j;
    j.q = q;
    j.k = k;
    j.v = v;
    j.n_ctx = n_ctx;
    j.T = T;
    j.hq = hq;
    j.hkv = hkv;
    j.d = d;
    j.scale = scale;
    j.rows = rows;
    j.n_rows = rows ? n_rows : T;
    j.out = out;
    j.next = 0;
    pthread_mutex_init(&j.mu, NULL);
    if (threads < 1) threads = 1;
    if (threads == 1) {
        attn_f64_worker(&j);
    } else {
        pthread_t * th = (pthread_t *)malloc(sizeof(pthread_t) * (size_t)threads);
        for (int32_t i = 0; i < threads; ++i) pthread_create(&th[i], NULL, attn_f64_worker, &j);
        for (int32_t i = 0; i < threads; ++i) pthread_join(th[i], NULL);
        free(th);
    }
    pthread_mutex_destroy(&j.mu);
}

void or_attn_f64(const uint16_t * q, const float * k, const float * v, int32_t n_ctx, int32_t T, int32_t hq,
                 int32_t hkv, int32_t d, double scale, const int32_t * rows, int32_t n_rows, double * out) {
    or_attn_f64_mt(q, k, v, n_ctx, T, hq, hkv, d, scale, rows, n_rows, out, 1);
}

/* ggml block_q8_0 as it lies in memory: fp16 d, then 32 int8 codes (34 bytes, no padding) */
typedef struct {
    uint16_t d;
    int8_t qs[OR_QK];
} or_block_q8_0;

typedef struct {
    const uint16_t * q;
    const or_block_q8_0 * k;
    const or_block_q8_0 * v;
    int32_t n_ctx, T, hq, hkv, d, q_as_q8;
    float scale;
    uint16_t * out;
    int32_t next; /* shared work counter */
    pthread_mutex_t mu;
} fa_job;

static void fa_row(const fa_job * j, int32_t t, int32_t h, float * qf, int8_t * qq, float * qdq, float * acc,
                   float * vrow) {
    const int32_t d = j->d, nb = d / OR_QK, kh = h / (j->hq / j->hkv);
    const int32_t last = j->n_ctx - j->T + t;
    for (int32_t e = 0; e < d; ++e) qf[e] = or_f16_to_f32(j->q[((int64_t)t * j->hq + h) * d + e]);
    if (j->q_as_q8) {
        uint16_t qd16[64];
        or_q8_0_quantize(qf, d, qq, qd16);
        for (int32_t b = 0; b < nb; ++b) qdq[b] = or_f16_to_f32(qd16[b]);
    }
    float m = -INFINITY, l = 0.0f;
    for (int32_t e = 0; e < d; ++e) acc[e] = 0.0f;
    for (int32_t c = 0; c <= last; ++c) {
        const or_block_q8_0 * kb = j->k + ((int64_t)c * j->hkv + kh) * nb;
        float sc = 0.0f;
        if (j->q_as_q8) {
            for (int32_t b = 0; b < nb; ++b) {
                int32_t isum = 0;
                for (int32_t e = 0; e < OR_QK; ++e) isum += (int32_t)qq[b * OR_QK + e] * (int32_t)kb[b].qs[e];
                sc += (float)isum * (or_f16_to_f32(kb[b].d) * qdq[b]);
            }
        } else {
            for (int32_t b = 0; b < nb; ++b) {
                const float s = or_f16_to_f32(kb[b].d);
                for (int32_t e = 0; e < OR_QK; ++e) sc += qf[b * OR_QK + e] * ((float)kb[b].qs[e] * s);
            }
        }
        sc *= j->scale;
        const or_block_q8_0 * vb = j->v + ((int64_t)c * j->hkv + kh) * nb;
        for (int32_t b = 0; b < nb; ++b) {
            const float s = or_f16_to_f32(vb[b].d);
            for (int32_t e = 0; e < OR_QK; ++e) vrow[b * OR_QK + e] = (float)vb[b].qs[e] * s;
        }
        if (sc > m) {
            const float f = expf(m - sc); /* 0 on the first key */
            for (int32_t e = 0; e < d; ++e) acc[e] = acc[e] * f + vrow[e];
            l = l * f + 1.0f;
            m = sc;
        } else {
            const float p = expf(sc - m);
            for (int32_t e = 0; e < d; ++e) acc[e] += p * vrow[e];
            l += p;
        }
    }
    uint16_t * o = j->out + ((int64_t)t * j->hq + h) * d;
    for (int32_t e = 0; e < d; ++e) o[e] = or_f32_to_f16(acc[e] / l);
}

static void * fa_worker(void * arg) {
    fa_job * j = (fa_job *)arg;
    const int32_t d = j->d;
    float * qf = (float *)malloc(sizeof(float) * (size_t)d);
    int8_t * qq = (int8_t *)malloc((size_t)d);
    float * qdq = (float *)malloc(sizeof(float) * (size_t)(d / OR_QK));
    float * acc = (float *)malloc(sizeof(float) * (size_t)d);
    float * vrow = (float *)malloc(sizeof(float) * (size_t)d);
    const int32_t total = j->T * j->hq;
    for (;;) {
        pthread_mutex_lock(&j->mu);
        const int32_t w = j->next++;
        pthread_mutex_unlock(&j->mu);
        if (w >= total) break;
        fa_row(j, w / j->hq, w % j->hq, qf, qq, qdq, acc, vrow);
    }
    free(qf);
    free(qq);
    free(qdq);
    free(acc);
    free(vrow);
    return NULL;
}

/*
 * ggml-semantics CPU flash attention over contiguous Q8_0 K/V (ggml's cache layout: [n_ctx][hkv][d / 32] blocks).
 *   q fp16 [T][hq][d]; out fp16 [T][hq][d]; threads >= 1
 */
void or_attn_ggml(const uint16_t * q, const void * k_blocks, const void * v_blocks, int32_t n_ctx, int32_t T,
                  int32_t hq, int32_t hkv, int32_t d, float scale, int32_t q_as_q8, int32_t threads, uint16_t * out) {
    fa_job j;
    j.q = q;
    j.k = (const or_block_q8_0 *)k_blocks;
    j.v = (const or_block_q8_0 *)v_blocks;
    j.n_ctx = n_ctx;
    j.T = T;
    j.hq = hq;
    j.hkv = hkv;
    j.d = d;
    j.q_as_q8 = q_as_q8;
    j.scale = scale;
    j.out = out;
    j.next = 0;
    pthread_mutex_init(&j.mu, NULL);
    if (threads < 1) threads = 1;
    pthread_t * th = (pthread_t *)malloc(sizeof(pthread_t) * (size_t)threads);
    for (int32_t i = 0; i < threads; ++i) pthread_create(&th[i], NULL, fa_worker, &j);
    for (int32_t i = 0; i < threads; ++i) pthread_join(th[i], NULL);
    free(th);
    pthread_mutex_destroy(&j.mu);
}

int32_t or_block_q8_0_size(void) { return (int32_t)sizeof(or_block_q8_0); }
