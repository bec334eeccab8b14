/*
 * stk_oracle.c -- CPU oracle for the streaming top-k SAE encoder.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (the HIP library, the
 * Python package) may call, link or load this file; only tests/, the smoke
 * check in __graft_entry__.py and the cpu_baseline leg of bench.py use it,
 * and only as the checker.
 *
 * Semantics restated here (reference paths are relative to the reference
 * checkout):
 *
 *   orc_scores_f64   score[i,f] = sum_d X[i,d]*W[f,d] + b[f], accumulated in
 *                    double.  This is the quantity streamtopk_sae/reference.py:17
 *                    computes ("X @ W_enc.T + b_enc"), evaluated on the upcast
 *                    fp32 inputs and without the bf16 rounding of the
 *                    reference's own matmul.
 *
 *   orc_exact        top-k of the fp32-rounded double scores per row, sorted by
 *                    value descending; equal values are ordered by lower latent
 *                    index first; NaN ranks above every number, as torch.topk
 *                    does (reference.py:18).  Indices are int32 (reference.py:19).
 *
 *   orc_approx       the approximate variant: top-c of each contiguous group of
 *                    128 latents (streamtopk_sae/csrc/cuda/streamtopk_approx.cu:31,
 *                    62-64, 118-166), padded with (-FLT_MAX, -1) when a group holds
 *                    fewer than c latents (streamtopk_approx.cu:17-18 of
 *                    topk_buffer.cuh init), then top-k over the flattened
 *                    candidates (streamtopk_sae/ops.py:80-81).
 *
 * The streaming restatement of the reference's CPU kernel lives in
 * stk_oracle_cpu.c (compiled with the reference's reassociating flags).
 */
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <math.h>
#include <float.h>

#define ORC_APPROX_GROUP 128

/* Monotone map float -> uint32 (NaN canonicalised to the top). */
static uint32_t orc_ordered(float v)
{
    uint32_t u;
    if (isnan(v)) return 0xFFFFFFFFu;
    memcpy(&u, &v, 4);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

/* 64-bit sort key: value order in the high word, lower index wins ties. */
static uint64_t orc_key(float v, int64_t idx)
{
    return ((uint64_t)orc_ordered(v) << 32) | (uint64_t)(0xFFFFFFFFu - (uint32_t)idx);
}

static int cmp_key_desc(const void* a, const void* b)
{
    uint64_t x = *(const uint64_t*)a, y = *(const uint64_t*)b;
    return (x < y) - (x > y);
}

int orc_abi_version(void) { return 1; }

int orc_scores_f64(const float* X, const float* W, const float* b,
                   int64_t B, int64_t d, int64_t F, double* S)
{
    for (int64_t i = 0; i < B; ++i)
        for (int64_t f = 0; f < F; ++f) {
            double acc = 0.0;
            const float* x = X + i * d;
            const float* w = W + f * d;
            for (int64_t t = 0; t < d; ++t) acc += (double)x[t] * (double)w[t];
            S[i * F + f] = acc + (double)b[f];
        }
    return 0;
}

/* Top-k of one row of fp32 scores under the key order; writes sorted output. */
static int topk_row(const float* s, int64_t F, int64_t k, float* V, int32_t* I,
                    uint64_t* tmp)
{
    for (int64_t f = 0; f < F; ++f) tmp[f] = orc_key(s[f], f);
    qsort(tmp, (size_t)F, sizeof(uint64_t), cmp_key_desc);
    for (int64_t j = 0; j < k; ++j) {
        int64_t f = (int64_t)(0xFFFFFFFFu - (uint32_t)(tmp[j] & 0xFFFFFFFFu));
        V[j] = s[f];
        I[j] = (int32_t)f;
    }
    return 0;
}

int orc_exact(const float* X, const float* W, const float* b,
              int64_t B, int64_t d, int64_t F, int64_t k,
              float* V, int32_t* I, int nthreads)
{
    if (k < 1 || k > F) return 1;
    (void)nthreads;
    int rc = 0;
#pragma omp parallel num_threads(nthreads > 0 ? nthreads : 1)
    {
        float* s = (float*)malloc((size_t)F * sizeof(float));
        uint64_t* tmp = (uint64_t*)malloc((size_t)F * sizeof(uint64_t));
        if (!s || !tmp) {
#pragma omp atomic write
            rc = 2;
        } else {
#pragma omp for schedule(dynamic, 1)
            for (int64_t i = 0; i < B; ++i) {
                const float* x = X + i * d;
                for (int64_t f = 0; f < F; ++f) {
                    const float* w = W + f * d;
                    double acc = 0.0;
                    for (int64_t t = 0; t < d; ++t) acc += (double)x[t] * (double)w[t];
                    s[f] = (float)(acc + (double)b[f]);
                }
                topk_row(s, F, k, V + i * k, I + i * k, tmp);
            }
        }
        free(s);
        free(tmp);
    }
    return rc;
}

/* Top-k of precomputed fp32 scores (B, F): used by tests that build scores
 * themselves (known-answer constructions). */
int orc_topk_scores(const float* S, int64_t B, int64_t F, int64_t k,
                    float* V, int32_t* I)
{
    if (k < 1 || k > F) return 1;
    uint64_t* tmp = (uint64_t*)malloc((size_t)F * sizeof(uint64_t));
    if (!tmp) return 2;
    for (int64_t i = 0; i < B; ++i) topk_row(S + i * F, F, k, V + i * k, I + i * k, tmp);
    free(tmp);
    return 0;
}

/* Approximate variant: per-128-group top-c, then top-k of the union.
 * cand_v / cand_i are (B, ceil(F/128), c), sorted descending per group and
 * padded with (-FLT_MAX, -1); either may be NULL. */
int orc_approx(const float* X, const float* W, const float* b,
               int64_t B, int64_t d, int64_t F, int64_t k, int64_t c,
               float* V, int32_t* I, float* cand_v, int32_t* cand_i)
{
    if (k < 1 || k > c || k > F) return 1;
    const int64_t G = ORC_APPROX_GROUP;
    const int64_t nt = (F + G - 1) / G;
    float* s = (float*)malloc((size_t)F * sizeof(float));
    uint64_t* gk = (uint64_t*)malloc((size_t)G * sizeof(uint64_t));
    uint64_t* flat = (uint64_t*)malloc((size_t)(nt * c) * sizeof(uint64_t));
    float* fv = (float*)malloc((size_t)(nt * c) * sizeof(float));
    int32_t* fi = (int32_t*)malloc((size_t)(nt * c) * sizeof(int32_t));
    if (!s || !gk || !flat || !fv || !fi) { free(s); free(gk); free(flat); free(fv); free(fi); return 2; }
    for (int64_t i = 0; i < B; ++i) {
        const float* x = X + i * d;
        for (int64_t f = 0; f < F; ++f) {
            const float* w = W + f * d;
            double acc = 0.0;
            for (int64_t t = 0; t < d; ++t) acc += (double)x[t] * (double)w[t];
            s[f] = (float)(acc + (double)b[f]);
        }
        for (int64_t t = 0; t < nt; ++t) {
            int64_t f0 = t * G, n = (F - f0 < G) ? F - f0 : G;
            for (int64_t j = 0; j < n; ++j) gk[j] = orc_key(s[f0 + j], f0 + j);
            qsort(gk, (size_t)n, sizeof(uint64_t), cmp_key_desc);
            for (int64_t j = 0; j < c; ++j) {
                int64_t p = t * c + j;
                if (j < n) {
                    int64_t f = (int64_t)(0xFFFFFFFFu - (uint32_t)(gk[j] & 0xFFFFFFFFu));
                    fv[p] = s[f];
                    fi[p] = (int32_t)f;
                } else {
                    fv[p] = -FLT_MAX;
                    fi[p] = -1;
                }
                if (cand_v) cand_v[(i * nt + t) * c + j] = fv[p];
                if (cand_i) cand_i[(i * nt + t) * c + j] = fi[p];
            }
        }
        /* Final top-k over the flattened candidates; padding sorts last. */
        for (int64_t p = 0; p < nt * c; ++p)
            flat[p] = (fi[p] < 0) ? 0 : orc_key(fv[p], fi[p]);
        qsort(flat, (size_t)(nt * c), sizeof(uint64_t), cmp_key_desc);
        for (int64_t j = 0; j < k; ++j) {
            int64_t f = (int64_t)(0xFFFFFFFFu - (uint32_t)(flat[j] & 0xFFFFFFFFu));
            V[i * k + j] = s[f];
            I[i * k + j] = (int32_t)f;
        }
    }
    free(s); free(gk); free(flat); free(fv); free(fi);
    return 0;
}
