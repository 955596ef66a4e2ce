/*
 * attn_oracle.c -- CPU oracle for the FlashAttention-2 forward path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the shipped library links, loads or
 * calls this file; only tests/, __graft_entry__.smoke() and bench.py's CPU
 * baseline use it, and only to check results against.  It restates, in plain C, the
 * semantics of the reference's attention path (dmonkman/RDNAttention):
 *
 *   - masking        src/rdna/fa2_forward_f16.hip:297-348 (kvBlockRange, isMasked),
 *                    tests/hip_forward_gate.hip:88-111, docs/api.md:150-165
 *   - RoPE           src/rdna/fa2_forward_f16.hip:63-77 (applyRope), :703, :256
 *   - GQA head map   src/rdna/fa2_forward_f16.hip:643-645 (kv = h / (Hq/Hkv))
 *   - empty rows     src/rdna/fa2_forward_f16.hip:733 (l == 0 -> output 0)
 *   - INT8 scheme    src/rdna/fa2_forward_int8qk.hip:281-382 (running max per
 *                    64-key block, P = min(127, lround(p*127)), l from unquantised p)
 *   - INT8 gate      tests/hip_forward_int8qk_gate.hip:62-120 (global max, fp64)
 *   - quantisers     rdnattention/__init__.py:313-343 (amax/127, 0 -> 1,
 *                    round-half-even, clamp +-127)
 *
 * How each function is pinned (closed forms, library routines, invariants) is
 * recorded in tests/test_oracle.py.  Build: oracle/Makefile (gcc, -O2,
 * -ffp-contract=off so float arithmetic is plain IEEE single/double).
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define ORACLE_API __attribute__((visibility("default")))

/* ------------------------------------------------------------------------ */
/* fp16 <-> fp32 (IEEE binary16, round-to-nearest-even).  gcc 11 on x86-64    */
/* has no _Float16, so the conversion is written out.                         */
/* ------------------------------------------------------------------------ */

ORACLE_API float oracle_half_to_float(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu;
    uint32_t man = h & 0x3ffu;
    uint32_t bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else { /* subnormal: value = man * 2^-24 */
            float f = (float)man * 5.9604644775390625e-08f;
            memcpy(&bits, &f, 4);
            bits |= sign;
        }
    } else if (exp == 31) {
        bits = sign | 0x7f800000u | (man << 13);
    } else {
        bits = sign | ((exp + 112u) << 23) | (man << 13);
    }
    float out;
    memcpy(&out, &bits, 4);
    return out;
}

ORACLE_API uint16_t oracle_float_to_half(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) { /* inf or nan */
        return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u : 0u));
    }
    if (ax >= 0x477ff000u) { /* rounds to >= 65520 -> inf */
        return (uint16_t)(sign | 0x7c00u);
    }
    if (ax < 0x38800000u) { /* below the smallest normal half (2^-14) */
        /* value in units of 2^-24, rounded to nearest even */
        float a;
        memcpy(&a, &ax, 4);
        double units = (double)a * 16777216.0; /* exact: a < 2^-14 */
        double r = nearbyint(units);           /* default mode: ties to even */
        return (uint16_t)(sign | (uint16_t)r); /* r <= 1024 -> may carry into exponent: correct */
    }
    uint32_t e = (ax >> 23) - 112u; /* half exponent, 1..30 */
    uint32_t m = ax & 0x7fffffu;
    uint32_t hm = m >> 13;
    uint32_t rest = m & 0x1fffu;
    uint32_t h = (e << 10) | hm;
    if (rest > 0x1000u || (rest == 0x1000u && (hm & 1u))) {
        h += 1u; /* carry may roll into the exponent: that is the correct result */
    }
    return (uint16_t)(sign | h);
}

ORACLE_API float oracle_round_f16(float f) {
    return oracle_half_to_float(oracle_float_to_half(f));
}

/* ------------------------------------------------------------------------ */
/* Masking: is key `k` visible to query row `i`?                             */
/* Follows fa2_forward_f16.hip:325-348 and tests/hip_forward_gate.hip:92-100 */
/* ------------------------------------------------------------------------ */
static int visible(int64_t i, int64_t k, int64_t sk, int64_t delta, int causal, int window) {
    if (k < 0 || k >= sk) {
        return 0;
    }
    if (causal && k > i + delta) {
        return 0;
    }
    if (window > 0) {
        if (causal) {
            if (i + delta - k >= window) {
                return 0;
            }
        } else {
            int64_t d = i + delta - k;
            if (d < 0) {
                d = -d;
            }
            if (d > window / 2) {
                return 0;
            }
        }
    }
    return 1;
}

ORACLE_API int32_t oracle_visible(int64_t i, int64_t k, int64_t sq, int64_t sk, int32_t causal, int32_t window) {
    return visible(i, k, sk, sk - sq, causal, window);
}

/* Exact number of visible (query, key) pairs for one (b, h): the FLOP-count */
/* convention of tests/benchmark.py:77-88, extended to windows.              */
ORACLE_API int64_t oracle_valid_pairs(int64_t sq, int64_t sk, int32_t causal, int32_t window) {
    int64_t delta = sk - sq;
    int64_t total = 0;
    for (int64_t i = 0; i < sq; i++) {
        int64_t lo = 0, hi = sk - 1; /* inclusive visible interval */
        if (causal && i + delta < hi) {
            hi = i + delta;
        }
        if (window > 0) {
            if (causal) {
                int64_t l2 = i + delta - window + 1;
                if (l2 > lo) {
                    lo = l2;
                }
            } else {
                int64_t hw = window / 2;
                if (i + delta - hw > lo) {
                    lo = i + delta - hw;
                }
                if (i + delta + hw < hi) {
                    hi = i + delta + hw;
                }
            }
        }
        if (hi >= lo) {
            total += hi - lo + 1;
        }
    }
    return total;
}

/* ------------------------------------------------------------------------ */
/* RoPE: interleaved pairs (2i, 2i+1) rotated by table column i of row s.    */
/* fa2_forward_f16.hip:63-77 computes (a*c - b*s, a*s + b*c) in fp32 and     */
/* rounds to fp16; round_f16 = 0 keeps fp32 (the gate's oracle,              */
/* tests/hip_forward_gate.hip:59-73).                                         */
/* x: [bh, seq, d] contiguous fp32; tables: [>= seq, d/2] fp32.              */
/* ------------------------------------------------------------------------ */
ORACLE_API void oracle_rope(float* x, int64_t bh, int64_t seq, int64_t d, const float* cos_t, const float* sin_t,
                            int32_t round_f16) {
    int64_t half = d / 2;
    for (int64_t h = 0; h < bh; h++) {
        for (int64_t s = 0; s < seq; s++) {
            float* row = x + (h * seq + s) * d;
            const float* c = cos_t + s * half;
            const float* sn = sin_t + s * half;
            for (int64_t p = 0; p < half; p++) {
                float a = row[2 * p], b = row[2 * p + 1];
                float r0 = a * c[p] - b * sn[p];
                float r1 = a * sn[p] + b * c[p];
                if (round_f16) {
                    r0 = oracle_round_f16(r0);
                    r1 = oracle_round_f16(r1);
                }
                row[2 * p] = r0;
                row[2 * p + 1] = r1;
            }
        }
    }
}

/* ------------------------------------------------------------------------ */
/* Threading helper: parallel-for over (b, h) pairs with a shared counter.   */
/* ------------------------------------------------------------------------ */
typedef void (*task_fn)(void* ctx, int64_t task);
typedef struct {
    task_fn fn;
    void* ctx;
    int64_t ntasks;
    int64_t next;
    pthread_mutex_t mu;
} pool_t;

static void* pool_worker(void* arg) {
    pool_t* p = (pool_t*)arg;
    for (;;) {
        pthread_mutex_lock(&p->mu);
        int64_t t = p->next++;
        pthread_mutex_unlock(&p->mu);
        if (t >= p->ntasks) {
            break;
        }
        p->fn(p->ctx, t);
    }
    return NULL;
}

static void run_tasks(task_fn fn, void* ctx, int64_t ntasks, int nthreads) {
    if (nthreads <= 1 || ntasks <= 1) {
        for (int64_t t = 0; t < ntasks; t++) {
            fn(ctx, t);
        }
        return;
    }
    if (nthreads > 64) {
        nthreads = 64;
    }
    pool_t p;
    p.fn = fn;
    p.ctx = ctx;
    p.ntasks = ntasks;
    p.next = 0;
    pthread_mutex_init(&p.mu, NULL);
    pthread_t th[64];
    int started = 0;
    for (int i = 0; i < nthreads; i++) {
        if (pthread_create(&th[i], NULL, pool_worker, &p) == 0) {
            started++;
        } else {
            break;
        }
    }
    if (started == 0) {
        pool_worker(&p);
    }
    for (int i = 0; i < started; i++) {
        pthread_join(th[i], NULL);
    }
    pthread_mutex_destroy(&p.mu);
}

/* ------------------------------------------------------------------------ */
/* FP attention: softmax(scale * Q K^T + mask) V in fp64, output fp32.       */
/* Follows tests/hip_forward_gate.hip:75-129 (refAttention) with the masking */
/* above; a row with no visible key outputs 0 (fa2_forward_f16.hip:733).      */
/* q: [B,Hq,Sq,D], k/v: [B,Hkv,Sk,D], out: [B,Hq,Sq,D]; all contiguous fp32.  */
/* ------------------------------------------------------------------------ */
typedef struct {
    const float *q, *k, *v;
    float* out;
    float* lse; /* optional [B,Hq,Sq] natural-log sum-exp of scaled scores */
    int64_t B, Hq, Hkv, Sq, Sk, D;
    double scale;
    int causal, window;
} attn_ctx;

#define ATTN_ROW_CHUNK 64

static void attn_task(void* vctx, int64_t task) {
    attn_ctx* c = (attn_ctx*)vctx;
    int64_t nchunk = (c->Sq + ATTN_ROW_CHUNK - 1) / ATTN_ROW_CHUNK;
    int64_t chunk = task % nchunk;
    task /= nchunk;
    int64_t b = task / c->Hq, h = task % c->Hq;
    int64_t ratio = c->Hq / c->Hkv;
    int64_t kvh = h / ratio;
    int64_t delta = c->Sk - c->Sq;
    const float* qb = c->q + (b * c->Hq + h) * c->Sq * c->D;
    const float* kb = c->k + (b * c->Hkv + kvh) * c->Sk * c->D;
    const float* vb = c->v + (b * c->Hkv + kvh) * c->Sk * c->D;
    float* ob = c->out + (b * c->Hq + h) * c->Sq * c->D;
    double* pr = (double*)malloc(sizeof(double) * (size_t)(c->Sk > 0 ? c->Sk : 1));
    double* acc = (double*)malloc(sizeof(double) * (size_t)c->D);
    int64_t i_end = (chunk + 1) * ATTN_ROW_CHUNK < c->Sq ? (chunk + 1) * ATTN_ROW_CHUNK : c->Sq;
    for (int64_t i = chunk * ATTN_ROW_CHUNK; i < i_end; i++) {
        double mx = -INFINITY;
        int64_t cnt = 0;
        for (int64_t j = 0; j < c->Sk; j++) {
            if (!visible(i, j, c->Sk, delta, c->causal, c->window)) {
                pr[j] = -INFINITY;
                continue;
            }
            double s = 0.0;
            for (int64_t d = 0; d < c->D; d++) {
                s += (double)qb[i * c->D + d] * (double)kb[j * c->D + d];
            }
            s *= c->scale;
            pr[j] = s;
            if (s > mx) {
                mx = s;
            }
            cnt++;
        }
        double sum = 0.0;
        for (int64_t d = 0; d < c->D; d++) {
            acc[d] = 0.0;
        }
        if (cnt > 0) {
            for (int64_t j = 0; j < c->Sk; j++) {
                if (pr[j] == -INFINITY) {
                    continue;
                }
                double p = exp(pr[j] - mx);
                sum += p;
                const float* vr = vb + j * c->D;
                for (int64_t d = 0; d < c->D; d++) {
                    acc[d] += p * (double)vr[d];
                }
            }
        }
        for (int64_t d = 0; d < c->D; d++) {
            ob[i * c->D + d] = cnt > 0 ? (float)(acc[d] / sum) : 0.0f;
        }
        if (c->lse) {
            c->lse[(b * c->Hq + h) * c->Sq + i] = cnt > 0 ? (float)(mx + log(sum)) : -INFINITY;
        }
    }
    free(pr);
    free(acc);
}

static int check_dims(int64_t B, int64_t Hq, int64_t Hkv, int64_t Sq, int64_t Sk, int64_t D) {
    if (B < 0 || Hq <= 0 || Hkv <= 0 || Sq < 0 || Sk < 0 || D <= 0) {
        return -1;
    }
    if (Hq % Hkv != 0) {
        return -2;
    }
    return 0;
}

ORACLE_API int32_t oracle_attention(const float* q, const float* k, const float* v, float* out, float* lse, int64_t B,
                                    int64_t Hq, int64_t Hkv, int64_t Sq, int64_t Sk, int64_t D, double scale,
                                    int32_t causal, int32_t window, int32_t nthreads) {
    int rc = check_dims(B, Hq, Hkv, Sq, Sk, D);
    if (rc) {
        return rc;
    }
    attn_ctx c = {q, k, v, out, lse, B, Hq, Hkv, Sq, Sk, D, scale, causal != 0, window};
    run_tasks(attn_task, &c, B * Hq * ((Sq + ATTN_ROW_CHUNK - 1) / ATTN_ROW_CHUNK), nthreads);
    return 0;
}

/* ------------------------------------------------------------------------ */
/* INT8: exact int32 scores S = Q_i8 K_i8^T, [B,Hq,Sq,Sk].                   */
/* The value both the reference's sdot4 loop (fa2_forward_int8qk.hip:254-278) */
/* and an int8 MFMA compute exactly.                                          */
/* ------------------------------------------------------------------------ */
ORACLE_API int32_t oracle_int8_scores(const int8_t* q, const int8_t* k, int32_t* s, int64_t B, int64_t Hq,
                                      int64_t Hkv, int64_t Sq, int64_t Sk, int64_t D) {
    int rc = check_dims(B, Hq, Hkv, Sq, Sk, D);
    if (rc) {
        return rc;
    }
    int64_t ratio = Hq / Hkv;
    for (int64_t b = 0; b < B; b++) {
        for (int64_t h = 0; h < Hq; h++) {
            const int8_t* qb = q + (b * Hq + h) * Sq * D;
            const int8_t* kb = k + (b * Hkv + h / ratio) * Sk * D;
            int32_t* sb = s + (b * Hq + h) * Sq * Sk;
            for (int64_t i = 0; i < Sq; i++) {
                for (int64_t j = 0; j < Sk; j++) {
                    int32_t acc = 0;
                    for (int64_t d = 0; d < D; d++) {
                        acc += (int32_t)qb[i * D + d] * (int32_t)kb[j * D + d];
                    }
                    sb[i * Sk + j] = acc;
                }
            }
        }
    }
    return 0;
}

/* ------------------------------------------------------------------------ */
/* INT8 attention, kernel-exact emulation (fa2_forward_int8qk.hip:281-382).  */
/* Keys are processed in blocks of `block_n` aligned to multiples of block_n */
/* (the reference uses 64).  Per block, in the log2 domain:                   */
/*   s_j  = (float)S_ij * qs_i * ks_j * (scale * log2e)          [fp32, :301] */
/*   m'   = max(m, max_j s_j); corr = exp2(m - m'); l *= corr; O *= corr      */
/*   p_j  = exp2(s_j - m');  l += sum_j p_j                 [unquantised]     */
/*   pq_j = min(127, lround(p_j * 127))                               [:335]  */
/*   O   += (float)(sum_j pq_j v_j) * ((1/127) * v_scale)          [:375-382] */
/* out = O / l (0 when no key is visible).  A block with no visible key for   */
/* row i leaves the row untouched, which is what the reference's sentinel    */
/* arithmetic gives (masked p = 0, max unchanged).                             */
/* q_scale_vec: [B,Hq,Sq] or NULL (use q_scale); k_scale_vec: [B,Hkv,Sk] or   */
/* NULL (use k_scale) -- the contiguous indexing of :410 and :287.           */
/* v_token_vec ([B,Hkv,Sk], the library's per-token V extension; no          */
/* reference counterpart): V row j becomes v'_j = fp16(sat(v_j * vs_j)),     */
/* the product in fp32 saturated to +-65504 and rounded once to fp16, and    */
/* O += (sum_j pq_j v'_j) * ((1/127) * v_scale), the sum in double.          */
/* ------------------------------------------------------------------------ */
typedef struct {
    const int8_t *q, *k, *v;
    const float *qsv, *ksv, *vtv;
    float qs, ks, vs;
    float* out;
    int64_t B, Hq, Hkv, Sq, Sk, D;
    float scale;
    int causal, window, block_n;
} i8_ctx;

static void i8_task(void* vctx, int64_t task) {
    i8_ctx* c = (i8_ctx*)vctx;
    int64_t b = task / c->Hq, h = task % c->Hq;
    int64_t ratio = c->Hq / c->Hkv, kvh = h / ratio;
    int64_t delta = c->Sk - c->Sq;
    const int8_t* qb = c->q + (b * c->Hq + h) * c->Sq * c->D;
    const int8_t* kb = c->k + (b * c->Hkv + kvh) * c->Sk * c->D;
    const int8_t* vb = c->v + (b * c->Hkv + kvh) * c->Sk * c->D;
    float* ob = c->out + (b * c->Hq + h) * c->Sq * c->D;
    const float kLog2E = 1.442695041f;
    const float scaleLog2e = c->scale * kLog2E;
    const float pvScale = (1.0f / 127.0f) * c->vs;
    int64_t bn = c->block_n;
    float* o = (float*)malloc(sizeof(float) * (size_t)c->D);
    float* sj = (float*)malloc(sizeof(float) * (size_t)bn);
    int32_t* pq = (int32_t*)malloc(sizeof(int32_t) * (size_t)bn);
    int32_t* pv = (int32_t*)malloc(sizeof(int32_t) * (size_t)c->D);
    double* pvd = (double*)malloc(sizeof(double) * (size_t)c->D);
    const float* vtb = c->vtv ? c->vtv + (b * c->Hkv + kvh) * c->Sk : NULL;
    for (int64_t i = 0; i < c->Sq; i++) {
        float qs = c->qsv ? c->qsv[(b * c->Hq + h) * c->Sq + i] : c->qs;
        float m = -INFINITY, l = 0.0f;
        for (int64_t d = 0; d < c->D; d++) {
            o[d] = 0.0f;
        }
        for (int64_t k0 = 0; k0 < c->Sk; k0 += bn) {
            int any = 0;
            float bmax = -INFINITY;
            for (int64_t jj = 0; jj < bn; jj++) {
                int64_t j = k0 + jj;
                if (!visible(i, j, c->Sk, delta, c->causal, c->window)) {
                    sj[jj] = -INFINITY;
                    continue;
                }
                any = 1;
                int32_t acc = 0;
                for (int64_t d = 0; d < c->D; d++) {
                    acc += (int32_t)qb[i * c->D + d] * (int32_t)kb[j * c->D + d];
                }
                float ks = c->ksv ? c->ksv[(b * c->Hkv + kvh) * c->Sk + j] : c->ks;
                float s = (float)acc * qs;
                s = s * ks;
                s = s * scaleLog2e;
                sj[jj] = s;
                if (s > bmax) {
                    bmax = s;
                }
            }
            if (!any) {
                continue;
            }
            float mnew = m > bmax ? m : bmax;
            if (mnew > m) {
                float corr = exp2f(m - mnew); /* m = -inf -> 0 */
                l *= corr;
                for (int64_t d = 0; d < c->D; d++) {
                    o[d] *= corr;
                }
            }
            float lsum = 0.0f;
            for (int64_t jj = 0; jj < bn; jj++) {
                if (sj[jj] == -INFINITY) {
                    pq[jj] = 0;
                    continue;
                }
                float p = exp2f(sj[jj] - mnew);
                lsum += p;
                long r = lroundf(p * 127.0f);
                pq[jj] = (int32_t)(r < 127 ? r : 127);
            }
            l += lsum;
            m = mnew;
            for (int64_t d = 0; d < c->D; d++) {
                pv[d] = 0;
                pvd[d] = 0.0;
            }
            for (int64_t jj = 0; jj < bn; jj++) {
                int64_t j = k0 + jj;
                if (pq[jj] == 0) {
                    continue;
                }
                const int8_t* vr = vb + j * c->D;
                if (vtb) {
                    const float vs = vtb[j];
                    for (int64_t d = 0; d < c->D; d++) {
                        float x = (float)vr[d] * vs;
                        x = x > 65504.0f ? 65504.0f : (x < -65504.0f ? -65504.0f : x);
                        pvd[d] += (double)pq[jj] * (double)oracle_round_f16(x);
                    }
                } else {
                    for (int64_t d = 0; d < c->D; d++) {
                        pv[d] += pq[jj] * (int32_t)vr[d];
                    }
                }
            }
            for (int64_t d = 0; d < c->D; d++) {
                o[d] += (vtb ? (float)pvd[d] : (float)pv[d]) * pvScale;
            }
        }
        float inv = l > 0.0f ? 1.0f / l : 0.0f;
        for (int64_t d = 0; d < c->D; d++) {
            ob[i * c->D + d] = o[d] * inv;
        }
    }
    free(o);
    free(sj);
    free(pq);
    free(pv);
    free(pvd);
}

ORACLE_API int32_t oracle_attention_int8(const int8_t* q, const int8_t* k, const int8_t* v, const float* q_scale_vec,
                                         const float* k_scale_vec, float q_scale, float k_scale, float v_scale,
                                         float* out, int64_t B, int64_t Hq, int64_t Hkv, int64_t Sq, int64_t Sk,
                                         int64_t D, float scale, int32_t causal, int32_t window, int32_t block_n,
                                         int32_t nthreads) {
    int rc = check_dims(B, Hq, Hkv, Sq, Sk, D);
    if (rc) {
        return rc;
    }
    if (block_n <= 0) {
        return -3;
    }
    i8_ctx c = {q,  k,  v,  q_scale_vec, k_scale_vec, NULL,   q_scale, k_scale, v_scale, out,
                B,  Hq, Hkv, Sq,         Sk,          D,      scale,   causal != 0, window, block_n};
    run_tasks(i8_task, &c, B * Hq, nthreads);
    return 0;
}

/* oracle_attention_int8 with a per-token V scale v_token_vec [B,Hkv,Sk]. */
ORACLE_API int32_t oracle_attention_int8_vtoken(const int8_t* q, const int8_t* k, const int8_t* v,
                                                const float* q_scale_vec, const float* k_scale_vec,
                                                const float* v_token_vec, float q_scale, float k_scale, float v_scale,
                                                float* out, int64_t B, int64_t Hq, int64_t Hkv, int64_t Sq, int64_t Sk,
                                                int64_t D, float scale, int32_t causal, int32_t window,
                                                int32_t block_n, int32_t nthreads) {
    int rc = check_dims(B, Hq, Hkv, Sq, Sk, D);
    if (rc) {
        return rc;
    }
    if (block_n <= 0 || v_token_vec == NULL) {
        return -3;
    }
    i8_ctx c = {q,  k,  v,  q_scale_vec, k_scale_vec, v_token_vec, q_scale, k_scale, v_scale, out,
                B,  Hq, Hkv, Sq,         Sk,          D,           scale,   causal != 0, window, block_n};
    run_tasks(i8_task, &c, B * Hq, nthreads);
    return 0;
}

/* ------------------------------------------------------------------------ */
/* INT8 attention, gate flavour (tests/hip_forward_int8qk_gate.hip:62-120):  */
/* dequantised fp32 Q/K/V in, fp64 scores, P quantised against the row's     */
/* GLOBAL max: pq = min(127, lround(p*127)); l from unquantised p.            */
/* ------------------------------------------------------------------------ */
typedef struct {
    const float *q, *k, *v;
    float* out;
    int64_t B, Hq, Hkv, Sq, Sk, D;
    double scale;
    int causal, window;
} i8g_ctx;

static void i8g_task(void* vctx, int64_t task) {
    i8g_ctx* c = (i8g_ctx*)vctx;
    int64_t b = task / c->Hq, h = task % c->Hq;
    int64_t ratio = c->Hq / c->Hkv, kvh = h / ratio;
    int64_t delta = c->Sk - c->Sq;
    const float* qb = c->q + (b * c->Hq + h) * c->Sq * c->D;
    const float* kb = c->k + (b * c->Hkv + kvh) * c->Sk * c->D;
    const float* vb = c->v + (b * c->Hkv + kvh) * c->Sk * c->D;
    float* ob = c->out + (b * c->Hq + h) * c->Sq * c->D;
    double* pr = (double*)malloc(sizeof(double) * (size_t)(c->Sk > 0 ? c->Sk : 1));
    for (int64_t i = 0; i < c->Sq; i++) {
        double mx = -INFINITY;
        int cnt = 0;
        for (int64_t j = 0; j < c->Sk; j++) {
            if (!visible(i, j, c->Sk, delta, c->causal, c->window)) {
                pr[j] = -INFINITY;
                continue;
            }
            double s = 0.0;
            for (int64_t d = 0; d < c->D; d++) {
                s += (double)qb[i * c->D + d] * (double)kb[j * c->D + d];
            }
            s *= c->scale;
            pr[j] = s;
            if (s > mx) {
                mx = s;
            }
            cnt++;
        }
        double sum = 0.0;
        for (int64_t j = 0; j < c->Sk; j++) {
            pr[j] = pr[j] == -INFINITY ? 0.0 : exp(pr[j] - mx);
            sum += pr[j];
        }
        for (int64_t d = 0; d < c->D; d++) {
            double acc = 0.0;
            for (int64_t j = 0; j < c->Sk; j++) {
                long q8 = lround(pr[j] * 127.0);
                if (q8 > 127) {
                    q8 = 127;
                }
                acc += ((double)q8 / 127.0) * (double)vb[j * c->D + d];
            }
            ob[i * c->D + d] = cnt ? (float)(acc / sum) : 0.0f;
        }
    }
    free(pr);
}

ORACLE_API int32_t oracle_attention_int8_gate(const float* q, const float* k, const float* v, float* out, int64_t B,
                                              int64_t Hq, int64_t Hkv, int64_t Sq, int64_t Sk, int64_t D, double scale,
                                              int32_t causal, int32_t window, int32_t nthreads) {
    int rc = check_dims(B, Hq, Hkv, Sq, Sk, D);
    if (rc) {
        return rc;
    }
    i8g_ctx c = {q, k, v, out, B, Hq, Hkv, Sq, Sk, D, scale, causal != 0, window};
    run_tasks(i8g_task, &c, B * Hq, nthreads);
    return 0;
}

/* ------------------------------------------------------------------------ */
/* Quantisers (rdnattention/__init__.py:313-343), in fp32 like torch:        */
/*   s = amax|x| / 127 (0 -> 1);  q = clamp(round_half_even(x / s), -127, 127) */
/* ------------------------------------------------------------------------ */
static int8_t quant1(float x, float s) {
    float r = nearbyintf(x / s); /* default rounding mode: ties to even, as torch.round */
    if (r > 127.0f) {
        r = 127.0f;
    }
    if (r < -127.0f) {
        r = -127.0f;
    }
    return (int8_t)r;
}

/* Per-token: x [rows, d] -> q [rows, d], s [rows] (quantize_int8_qk_pertoken) */
ORACLE_API void oracle_quant_pertoken(const float* x, int64_t rows, int64_t d, int8_t* q, float* s) {
    for (int64_t r = 0; r < rows; r++) {
        float m = 0.0f;
        for (int64_t i = 0; i < d; i++) {
            float a = fabsf(x[r * d + i]);
            m = a > m ? a : m;
        }
        float sc = m / 127.0f;
        if (sc == 0.0f) {
            sc = 1.0f;
        }
        s[r] = sc;
        for (int64_t i = 0; i < d; i++) {
            q[r * d + i] = quant1(x[r * d + i], sc);
        }
    }
}

/* Per-channel V: v [bh, seq, d] -> vi, v_channel [bh, d] (quantize_int8_perchannel_v) */
ORACLE_API void oracle_quant_perchannel(const float* v, int64_t bh, int64_t seq, int64_t d, int8_t* vi, float* vch) {
    for (int64_t h = 0; h < bh; h++) {
        for (int64_t i = 0; i < d; i++) {
            float m = 0.0f;
            for (int64_t s = 0; s < seq; s++) {
                float a = fabsf(v[(h * seq + s) * d + i]);
                m = a > m ? a : m;
            }
            float sc = m / 127.0f;
            if (sc == 0.0f) {
                sc = 1.0f;
            }
            vch[h * d + i] = sc;
            for (int64_t s = 0; s < seq; s++) {
                vi[(h * seq + s) * d + i] = quant1(v[(h * seq + s) * d + i], sc);
            }
        }
    }
}

/* Per-tensor: x [n] -> q [n], returns the scale (the per-tensor helper inside */
/* quantize_int8_perchannel_v, __init__.py:313-316).                           */
ORACLE_API float oracle_quant_pertensor(const float* x, int64_t n, int8_t* q) {
    float m = 0.0f;
    for (int64_t i = 0; i < n; i++) {
        float a = fabsf(x[i]);
        m = a > m ? a : m;
    }
    float sc = m / 127.0f;
    if (sc == 0.0f) {
        sc = 1.0f;
    }
    for (int64_t i = 0; i < n; i++) {
        q[i] = quant1(x[i], sc);
    }
    return sc;
}

/* ------------------------------------------------------------------------ */
/* Input generators of the reference's gates, so parity cases can run on    */
/* exactly the inputs the reference's own tests use.                          */
/*   mode 0: frand            (tests/hip_forward_gate.hip:31-37)              */
/*           s = s*1664525 + 1013904223; ((s>>16) & 4095)/4096 - 0.5          */
/*   mode 1: frandGaussianish (tests/hip_forward_int8qk_gate.hip:44-50)       */
/*           mean of three frand draws                                        */
/* The seed is advanced in place so consecutive fills continue one stream,   */
/* as the gates fill Q, then K, then V from one seed.                         */
/* ------------------------------------------------------------------------ */
static float lcg_frand(uint32_t* s) {
    *s = *s * 1664525u + 1013904223u;
    return (float)((*s >> 16) & 4095u) / 4096.0f - 0.5f;
}

ORACLE_API void oracle_lcg_fill(float* out, int64_t n, uint32_t* seed, int32_t mode) {
    for (int64_t i = 0; i < n; i++) {
        if (mode == 1) {
            float a = lcg_frand(seed);
            float b = lcg_frand(seed);
            float c = lcg_frand(seed);
            out[i] = (a + b + c) / 3.0f;
        } else {
            out[i] = lcg_frand(seed);
        }
    }
}
