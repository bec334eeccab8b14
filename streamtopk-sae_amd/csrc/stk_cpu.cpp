// stk_cpu.cpp -- host (CPU) streaming top-k encoder, fp32, OpenMP.
//
// Counterpart of the reference's CPU path (streamtopk_sae/csrc/cpu/
// streamtopk_cpu.cpp:15-125).  The reference walks rows serially and streams
// the whole of W once per row; here each OpenMP thread owns a contiguous
// range of latents, scores it for every row while that slice of W is hot in
// cache (W is read from memory once in total), keeps a per-row min-heap of
// the best k keys, and the per-thread heaps are merged per row at the end.
// Scores are accumulated in fp32 with eight partial sums per dot product and
// the bias added last; selection uses the same 64-bit key order as the device
// path (value descending, lower index first on ties, NaN first).
#include <omp.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <vector>

#include "../../include/streamtopk.h"
#include "stk_internal.h"

namespace {

inline uint64_t cpu_key(float v, int64_t idx)
{
    uint32_t u;
    std::memcpy(&u, &v, 4);
    uint32_t r = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    if (v != v) r = 0xFFFFFFFFu;
    return ((uint64_t)r << 32) | (uint64_t)(0xFFFFFFFFu - (uint32_t)idx);
}

inline float cpu_key_value(uint64_t key)
{
    uint32_t r = (uint32_t)(key >> 32);
    uint32_t u = (r & 0x80000000u) ? (r & 0x7FFFFFFFu) : ~r;
    float v;
    std::memcpy(&v, &u, 4);
    return v;
}

// Min-heap of at most k keys; heap[0] is the smallest kept key.
struct KeyHeap {
    uint64_t* h;
    int n, k;
    uint64_t threshold() const { return n < k ? 0ull : h[0]; }
    void push(uint64_t key)
    {
        if (n < k) {
            int i = n++;
            h[i] = key;
            while (i > 0) {
                int p = (i - 1) / 2;
                if (h[p] <= h[i]) break;
                std::swap(h[p], h[i]);
                i = p;
            }
        } else if (key > h[0]) {
            h[0] = key;
            int i = 0;
            for (;;) {
                int l = 2 * i + 1, r = l + 1, m = i;
                if (l < n && h[l] < h[m]) m = l;
                if (r < n && h[r] < h[m]) m = r;
                if (m == i) break;
                std::swap(h[m], h[i]);
                i = m;
            }
        }
    }
};

inline float dot8(const float* __restrict x, const float* __restrict w, int64_t d)
{
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    int64_t t = 0;
    for (; t + 8 <= d; t += 8)
        for (int e = 0; e < 8; ++e) acc[e] += x[t + e] * w[t + e];
    float s = ((acc[0] + acc[4]) + (acc[1] + acc[5])) + ((acc[2] + acc[6]) + (acc[3] + acc[7]));
    for (; t < d; ++t) s += x[t] * w[t];
    return s;
}

}  // namespace

extern "C" int stk_cpu_forward(const float* X, const float* W, const float* b, float* V, int32_t* I,
                               int64_t B, int64_t d, int64_t F, int64_t k, int num_threads)
{
    stk::clear_error();
    if (B < 0 || d < 1 || F < 1) return stk::set_error(STK_E_INVALID, "invalid shape");
    if (F > 0x7FFFFFFELL) return stk::set_error(STK_E_INVALID, "F exceeds the int32 index range");
    if (k < 1 || k > F) return stk::set_error(STK_E_INVALID, "k out of range");
    if (!stk::k_supported(k))
        return stk::set_error(STK_E_INVALID, "streamtopk_cpu: unsupported k=%lld. Supported: 1,2,4,8,16,32,64,128.",
                              (long long)k);
    if (B == 0) return 0;
    if (!X || !W || !b || !V || !I) return stk::set_error(STK_E_INVALID, "null tensor pointer");

    int nt = num_threads > 0 ? num_threads : omp_get_max_threads();
    if (nt < 1) nt = 1;
    // Each thread scores a contiguous latent range for all rows.
    const int64_t kBlock = 64;   // latents per cache block
    int64_t nblocks = (F + kBlock - 1) / kBlock;
    if (nt > nblocks) nt = (int)nblocks;
    std::vector<uint64_t> heaps((size_t)nt * B * k);
    std::vector<int> heap_n((size_t)nt * B, 0);

#pragma omp parallel num_threads(nt)
    {
        const int tid = omp_get_thread_num();
        const int T = omp_get_num_threads();
        const int64_t blo = nblocks * tid / T, bhi = nblocks * (tid + 1) / T;
        uint64_t* hp = heaps.data() + (size_t)tid * B * k;
        int* hn = heap_n.data() + (size_t)tid * B;
        float sc[kBlock];
        for (int64_t blk = blo; blk < bhi; ++blk) {
            const int64_t f0 = blk * kBlock;
            const int64_t nf = std::min<int64_t>(kBlock, F - f0);
            for (int64_t i = 0; i < B; ++i) {
                const float* xi = X + i * d;
                for (int64_t j = 0; j < nf; ++j) sc[j] = dot8(xi, W + (f0 + j) * d, d) + b[f0 + j];
                KeyHeap heap{hp + i * k, hn[i], (int)k};
                uint64_t thr = heap.threshold();
                for (int64_t j = 0; j < nf; ++j) {
                    const uint64_t key = cpu_key(sc[j], f0 + j);
                    if (key > thr) {
                        heap.push(key);
                        thr = heap.threshold();
                    }
                }
                hn[i] = heap.n;
            }
        }
    }

    // Merge the per-thread heaps row by row and emit sorted output.
#pragma omp parallel for num_threads(nt) schedule(static)
    for (int64_t i = 0; i < B; ++i) {
        std::vector<uint64_t> all;
        all.reserve((size_t)nt * k);
        for (int t = 0; t < nt; ++t) {
            const uint64_t* hp = heaps.data() + ((size_t)t * B + i) * k;
            all.insert(all.end(), hp, hp + heap_n[(size_t)t * B + i]);
        }
        std::partial_sort(all.begin(), all.begin() + k, all.end(), std::greater<uint64_t>());
        for (int64_t j = 0; j < k; ++j) {
            V[i * k + j] = cpu_key_value(all[j]);
            I[i * k + j] = (int32_t)(0xFFFFFFFFu - (uint32_t)all[j]);
        }
    }
    return 0;
}
