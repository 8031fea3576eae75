/* cpu_baseline.c -- CPU baseline timed by bench.py (TEST INFRASTRUCTURE ONLY).
 *
 * Portable-C restatement of the reference's threaded CPU GEMV entries, run on the GPU box's
 * host cores beside the GPU result.  Threading follows q4pool (q4gemv.h:408-670): a persistent
 * pthread pool, the caller thread works too, rows split into contiguous blocks of
 * ceil(out/T) (q4gemv.h:456-460), each row summed by one thread in fixed order.  The row math
 * is the oracle's (bgl_oracle.c), rewritten as flat loops the compiler can vectorise; results
 * are bit-identical to the oracle row functions (integer group sums are exact and the fp32 fold
 * runs in the same order).
 */
#include "bgl_oracle.h"
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

#define MAXT 64

typedef struct or_pool or_pool_t;
typedef struct { or_pool_t *p; int wi; } warg_t;

typedef struct {
    int kind, bits, out, in;
    const void *packed, *scales; const uint8_t *sub;
    const int8_t *xq; const float *ascale; const float *x; const float *bias; float *y;
    const or_expert *ex;      /* kind JOB_MOE: one expert matrix (moe_matvec_af_row per row) */
} job_t;
#define JOB_MOE (-1)

struct or_pool {
    int nthreads, max_in;
    pthread_t th[MAXT];
    pthread_mutex_t mtx;
    pthread_cond_t cv_go, cv_done;
    int gen, done, stop;
    job_t job;
    int8_t *xq; float *ascale;
    warg_t wargs[MAXT];
};

#if defined(__x86_64__)
#define VEC_CLONES __attribute__((target_clones("avx2", "default")))
#else
#define VEC_CLONES
#endif

VEC_CLONES
static float row_g256sf(const uint8_t *pr, const float *ws, const uint8_t *sub, const int8_t *xq,
                        const float *as, int in) {
    int ng256 = in >> 8;
    float acc = 0.0f;
    for (int gs = 0; gs < ng256; gs++) {
        int32_t comb = 0;
        for (int s = 0; s < 4; s++) {
            const uint8_t *gp = pr + (size_t)(gs * 4 + s) * 32;
            const int8_t *xp = xq + (size_t)(gs * 4 + s) * 64;
            int32_t isum = 0;
            for (int b = 0; b < 32; b++)
                isum += ((int)(gp[b] & 15) - 8) * xp[2 * b] + ((int)(gp[b] >> 4) - 8) * xp[2 * b + 1];
            comb += isum * (int32_t)sub[gs * 4 + s];
        }
        acc += (float)comb * ws[gs] * (1.0f / 63.0f) * as[gs];
    }
    return acc;
}

VEC_CLONES
static float row_q4g64_sdot(const uint8_t *pr, const float *ws, const int8_t *xq, const float *as, int in) {
    int ng = in >> 6;
    float acc = 0.0f;
    for (int g = 0; g < ng; g++) {
        const uint8_t *gp = pr + (size_t)g * 32;
        const int8_t *xp = xq + (size_t)g * 64;
        int32_t isum = 0;
        for (int b = 0; b < 32; b++)
            isum += ((int)(gp[b] & 15) - 8) * xp[2 * b] + ((int)(gp[b] >> 4) - 8) * xp[2 * b + 1];
        acc += (float)isum * ws[g] * as[g];
    }
    return acc;
}

static void run_range(or_pool *p, int wi) {
    job_t *j = &p->job;
    int per = (j->out + p->nthreads - 1) / p->nthreads;
    int r0 = wi * per, r1 = r0 + per;
    if (r1 > j->out) r1 = j->out;
    if (r0 >= r1) return;
    int in = j->in;
    if (j->kind == JOB_MOE) {
        for (int r = r0; r < r1; r++) j->y[r] = (float)or_moe_row(j->ex, in, r, j->x);
        return;
    }
    for (int r = r0; r < r1; r++) {
        float b = j->bias ? j->bias[r] : 0.0f, dot;
        if (j->kind == 3)
            dot = row_g256sf((const uint8_t *)j->packed + (size_t)r * (in / 2), (const float *)j->scales + (size_t)r * (in >> 8),
                             j->sub + (size_t)r * (in >> 6), j->xq, j->ascale, in);
        else if (j->kind == 1 && j->xq)
            dot = row_q4g64_sdot((const uint8_t *)j->packed + (size_t)r * (in / 2), (const float *)j->scales + (size_t)r * (in >> 6),
                                 j->xq, j->ascale, in);
        else {
            float yr;
            if (j->kind == 4) {
                size_t rb = (size_t)(in / 64) * j->bits * 8;
                or_qng64_matvec_f32((const uint8_t *)j->packed + (size_t)r * rb, (const float *)j->scales + (size_t)r * (in / 64),
                                    j->bits, j->x, NULL, &yr, 1, in);
            } else {
                const void *pk; const void *sc;
                if (j->kind == 2) { pk = (const int8_t *)j->packed + (size_t)r * in; sc = (const float *)j->scales + (size_t)r * (in / 64); }
                else if (j->kind == 5) { pk = (const uint8_t *)j->packed + (size_t)r * (in / 2); sc = (const uint16_t *)j->scales + (size_t)r * (in / 32); }
                else { pk = (const uint8_t *)j->packed + (size_t)r * (in / 2); sc = (const float *)j->scales + (size_t)r * (in / 64); }
                or_gemm_f32(j->kind, j->bits, pk, sc, j->x, NULL, &yr, 1, in, 1);
            }
            dot = yr;
        }
        j->y[r] = b + dot;
    }
}

static void *worker_main(void *arg) {
    warg_t *wa = (warg_t *)arg;
    or_pool *p = wa->p;
    int last = 0;
    for (;;) {
        pthread_mutex_lock(&p->mtx);
        while (p->gen == last && !p->stop) pthread_cond_wait(&p->cv_go, &p->mtx);
        if (p->stop) { pthread_mutex_unlock(&p->mtx); return NULL; }
        last = p->gen;
        pthread_mutex_unlock(&p->mtx);
        run_range(p, wa->wi);
        pthread_mutex_lock(&p->mtx);
        if (++p->done == p->nthreads) pthread_cond_signal(&p->cv_done);
        pthread_mutex_unlock(&p->mtx);
    }
}

or_pool *or_pool_create(int nthreads, int max_in) {
    if (nthreads < 1) nthreads = 1;
    if (nthreads > MAXT) nthreads = MAXT;
    or_pool *p = (or_pool *)calloc(1, sizeof(or_pool));
    p->nthreads = nthreads; p->max_in = max_in;
    pthread_mutex_init(&p->mtx, NULL);
    pthread_cond_init(&p->cv_go, NULL); pthread_cond_init(&p->cv_done, NULL);
    p->xq = (int8_t *)malloc((size_t)max_in);
    p->ascale = (float *)malloc(sizeof(float) * (size_t)(max_in / 64 + 1));
    for (int i = 1; i < nthreads; i++) {
        p->wargs[i].p = p; p->wargs[i].wi = i;
        pthread_create(&p->th[i], NULL, worker_main, &p->wargs[i]);
    }
    return p;
}

void or_pool_destroy(or_pool *p) {
    pthread_mutex_lock(&p->mtx);
    p->stop = 1;
    pthread_cond_broadcast(&p->cv_go);
    pthread_mutex_unlock(&p->mtx);
    for (int i = 1; i < p->nthreads; i++) pthread_join(p->th[i], NULL);
    free(p->xq); free(p->ascale);
    pthread_mutex_destroy(&p->mtx);
    pthread_cond_destroy(&p->cv_go); pthread_cond_destroy(&p->cv_done);
    free(p);
}

int or_pool_threads(const or_pool *p) { return p->nthreads; }

static void go_and_wait(or_pool *p) {
    pthread_mutex_lock(&p->mtx);
    p->done = 1;
    p->gen++;
    pthread_cond_broadcast(&p->cv_go);
    pthread_mutex_unlock(&p->mtx);
    run_range(p, 0);
    pthread_mutex_lock(&p->mtx);
    while (p->done < p->nthreads) pthread_cond_wait(&p->cv_done, &p->mtx);
    pthread_mutex_unlock(&p->mtx);
}

/* gemv_q4g256sf_sdot_mt (q4gemv_g256.h:339-364): quantize once on the caller, pool the rows. */
void or_pool_gemv_g256sf_sdot(or_pool *p, const uint8_t *packed, const float *wsuper, const uint8_t *sub,
                              const float *x, const float *bias, float *y, int out, int in) {
    or_quant_act_i8(x, in, 256, p->xq, p->ascale);
    job_t j = {3, 0, out, in, packed, wsuper, sub, p->xq, p->ascale, x, bias, y, NULL};
    p->job = j;
    go_and_wait(p);
}

/* gemv_q4g64_sdot_mt (q4gemv.h:701-722). */
void or_pool_gemv_q4g64_sdot(or_pool *p, const uint8_t *packed, const float *scales,
                             const float *x, const float *bias, float *y, int out, int in) {
    or_quant_act_i8(x, in, 64, p->xq, p->ascale);
    job_t j = {1, 0, out, in, packed, scales, NULL, p->xq, p->ascale, x, bias, y, NULL};
    p->job = j;
    go_and_wait(p);
}

/* gemv_q4g64_mt / gemv_q8g64_mt / qng64_matvec_f32 fp32-activation rows through the pool. */
void or_pool_gemv_f32(or_pool *p, int kind, int bits, const void *packed, const void *scales,
                      const float *x, const float *bias, float *y, int out, int in) {
    job_t j = {kind, bits, out, in, packed, scales, NULL, NULL, NULL, x, bias, y, NULL};
    p->job = j;
    go_and_wait(p);
}

/* moe_matvec_af_mt (qwen_infer.c:3223-3457): one expert matvec, its rows in contiguous blocks over
 * the pool, each row the double-accumulated moe_matvec_af_row. */
static void pool_moe_matvec(or_pool *p, const or_expert *w, int out, int in, const float *x, float *y) {
    job_t j;
    memset(&j, 0, sizeof j);
    j.kind = JOB_MOE; j.out = out; j.in = in; j.x = x; j.y = y; j.ex = w;
    p->job = j;
    go_and_wait(p);
}

/* moe_ffn_batched (qwen_infer.c:5238-5350) with routing supplied, every expert matvec through the
 * pool: or_moe_ffn_bucketed's order (experts ascending, members in token order, then the shared
 * experts), so the outputs are bit-identical to it. */
void or_pool_moe_ffn_bucketed(or_pool *p, const or_expert *gate, const or_expert *up, const or_expert *down, int E,
                              const or_expert *sh_gate, const or_expert *sh_up, const or_expert *sh_down,
                              int H, int I, int Ish, int T, int K, const float *x,
                              const int *top_idx, const float *top_w, float *out) {
    int *cnt = (int *)calloc((size_t)E, sizeof(int));
    int *mtok = (int *)malloc(sizeof(int) * (size_t)E * T);
    float *mw = (float *)malloc(sizeof(float) * (size_t)E * T);
    for (int b = 0; b < T; b++)
        for (int k = 0; k < K; k++) {
            int e = top_idx[(size_t)b * K + k];
            mtok[(size_t)e * T + cnt[e]] = b; mw[(size_t)e * T + cnt[e]] = top_w[(size_t)b * K + k]; cnt[e]++;
        }
    for (size_t i = 0; i < (size_t)T * H; i++) out[i] = 0.0f;
    int Imax = I > Ish ? I : Ish;
    float *g = (float *)malloc(sizeof(float) * (size_t)Imax), *u = (float *)malloc(sizeof(float) * (size_t)Imax);
    float *d = (float *)malloc(sizeof(float) * (size_t)H);
    for (int e = 0; e < E; e++)
        for (int m = 0; m < cnt[e]; m++) {
            int b = mtok[(size_t)e * T + m];
            float wgt = mw[(size_t)e * T + m];
            pool_moe_matvec(p, &gate[e], I, H, x + (size_t)b * H, g);
            pool_moe_matvec(p, &up[e], I, H, x + (size_t)b * H, u);
            or_moe_swiglu_inplace(g, u, I);
            pool_moe_matvec(p, &down[e], H, I, g, d);
            for (int c = 0; c < H; c++) out[(size_t)b * H + c] += wgt * d[c];
        }
    if (sh_gate && sh_up && sh_down)
        for (int b = 0; b < T; b++) {
            pool_moe_matvec(p, sh_gate, Ish, H, x + (size_t)b * H, g);
            pool_moe_matvec(p, sh_up, Ish, H, x + (size_t)b * H, u);
            or_moe_swiglu_inplace(g, u, Ish);
            pool_moe_matvec(p, sh_down, H, Ish, g, d);
            for (int c = 0; c < H; c++) out[(size_t)b * H + c] += d[c];
        }
    free(cnt); free(mtok); free(mw); free(g); free(u); free(d);
}
