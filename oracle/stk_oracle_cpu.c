/*
 * stk_oracle_cpu.c -- restatement of the reference's CPU streaming kernel.
 *
 * TEST INFRASTRUCTURE ONLY (see stk_oracle.c).  bench.py times this function
 * as its cpu_baseline ("port" of the reference CPU path).
 *
 * Follows streamtopk_sae/csrc/cpu/streamtopk_cpu.cpp:15-67 and
 * streamtopk_sae/csrc/cpu/topk_buffer.hpp:9-72:
 *   - rows are independent; the reference runs them serially
 *     (streamtopk_cpu.cpp:76-78); here an OpenMP loop over rows may run them
 *     in parallel, which leaves each row's result unchanged;
 *   - F is walked in tiles of 512 latents (streamtopk_cpu.cpp:12,33-35);
 *   - each score starts from the bias and accumulates x*w over d in fp32
 *     (streamtopk_cpu.cpp:41-44);
 *   - a score enters the buffer only if strictly greater than the current
 *     threshold (streamtopk_cpu.cpp:49-55, topk_buffer.hpp:30-42);
 *   - k <= 64: descending insertion buffer, equal values keep the earlier
 *     (lower-index) entry ahead (topk_buffer.hpp:37);
 *   - k > 64: min-heap with sift-down (topk_buffer.hpp:43-60), so the output
 *     is in heap order, not sorted (streamtopk_cpu.cpp:58);
 *   - buffer slots start at (-inf, -1) (topk_buffer.hpp:14-20).
 * The file is compiled with reassociating float flags, as the reference's
 * CPU extension is (setup.py:12), so the dot product vectorises.
 */
#include <stdint.h>
#include <stdlib.h>
#include <math.h>

#define ORC_T_CPU 512

typedef struct {
    int k;
    int heap;
    float* v;
    int* ix;
} orc_buf;

static float buf_threshold(const orc_buf* b) { return b->heap ? b->v[0] : b->v[b->k - 1]; }

static void buf_insert(orc_buf* b, float val, int idx)
{
    const int K = b->k;
    float* v = b->v;
    int* ix = b->ix;
    if (!b->heap) {
        if (val <= v[K - 1]) return;
        int pos = K - 1;
        while (pos > 0 && v[pos - 1] < val) {
            v[pos] = v[pos - 1];
            ix[pos] = ix[pos - 1];
            --pos;
        }
        v[pos] = val;
        ix[pos] = idx;
    } else {
        if (val <= v[0]) return;
        v[0] = val;
        ix[0] = idx;
        int i = 0;
        for (;;) {
            int l = 2 * i + 1, r = 2 * i + 2, m = i;
            if (l < K && v[l] < v[m]) m = l;
            if (r < K && v[r] < v[m]) m = r;
            if (m == i) break;
            float tv = v[i]; v[i] = v[m]; v[m] = tv;
            int ti = ix[i]; ix[i] = ix[m]; ix[m] = ti;
            i = m;
        }
    }
}

/* Exposed so the selection rule can be checked on its own against the
 * reference's TopKBuffer (oracle/_ref) on arbitrary score streams. */
int orc_buffer_stream(const float* scores, int64_t n, int64_t k, float* V, int32_t* I)
{
    if (k < 1) return 1;
    orc_buf b;
    b.k = (int)k;
    b.heap = k > 64;
    b.v = (float*)malloc((size_t)k * sizeof(float));
    b.ix = (int*)malloc((size_t)k * sizeof(int));
    if (!b.v || !b.ix) { free(b.v); free(b.ix); return 2; }
    for (int64_t j = 0; j < k; ++j) { b.v[j] = -INFINITY; b.ix[j] = -1; }
    float thr = buf_threshold(&b);
    for (int64_t j = 0; j < n; ++j) {
        if (scores[j] > thr) {
            buf_insert(&b, scores[j], (int)j);
            thr = buf_threshold(&b);
        }
    }
    for (int64_t j = 0; j < k; ++j) { V[j] = b.v[j]; I[j] = (int32_t)b.ix[j]; }
    free(b.v);
    free(b.ix);
    return 0;
}

static void process_row(int64_t i, const float* X, const float* W, const float* bias,
                        float* V, int32_t* I, int64_t k, int64_t F, int64_t d,
                        orc_buf* b, float* scores)
{
    for (int64_t j = 0; j < k; ++j) { b->v[j] = -INFINITY; b->ix[j] = -1; }
    const float* xi = X + i * d;
    for (int64_t f0 = 0; f0 < F; f0 += ORC_T_CPU) {
        int64_t f_end = (f0 + ORC_T_CPU < F) ? f0 + ORC_T_CPU : F;
        int64_t tile = f_end - f0;
        for (int64_t j = 0; j < tile; ++j) {
            const float* wj = W + (f0 + j) * d;
            float s = bias[f0 + j];
            for (int64_t t = 0; t < d; ++t) s += xi[t] * wj[t];
            scores[j] = s;
        }
        float thr = buf_threshold(b);
        for (int64_t j = 0; j < tile; ++j) {
            if (scores[j] > thr) {
                buf_insert(b, scores[j], (int)(f0 + j));
                thr = buf_threshold(b);
            }
        }
    }
    for (int64_t j = 0; j < k; ++j) {
        V[i * k + j] = b->v[j];
        I[i * k + j] = (int32_t)b->ix[j];
    }
}

int orc_cpu_stream(const float* X, const float* W, const float* bias,
                   int64_t B, int64_t d, int64_t F, int64_t k,
                   float* V, int32_t* I, int nthreads)
{
    if (k < 1 || k > F) return 1;
    int rc = 0;
#pragma omp parallel num_threads(nthreads > 0 ? nthreads : 1)
    {
        orc_buf b;
        b.k = (int)k;
        b.heap = k > 64;
        b.v = (float*)malloc((size_t)k * sizeof(float));
        b.ix = (int*)malloc((size_t)k * sizeof(int));
        float* scores = (float*)malloc(ORC_T_CPU * sizeof(float));
        if (!b.v || !b.ix || !scores) {
#pragma omp atomic write
            rc = 2;
        } else {
#pragma omp for schedule(dynamic, 1)
            for (int64_t i = 0; i < B; ++i) process_row(i, X, W, bias, V, I, k, F, d, &b, scores);
        }
        free(b.v);
        free(b.ix);
        free(scores);
    }
    return rc;
}
