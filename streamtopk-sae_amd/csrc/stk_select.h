// stk_select.h -- workgroup-wide top-k selection over 64-bit sort keys held in
// LDS (radix select by 8-bit digits, most significant first), plus the rank
// sort used to emit the final k keys in descending order.
#pragma once
#include "stk_device.h"

namespace stk {

constexpr int kSelCap = 4096;   // keys held in LDS by one selection workgroup
constexpr int kMaxK = 128;

struct SelShared {
    uint64_t buf[kSelCap];
    uint32_t hist[kWaves][256];
    uint64_t sel[kMaxK];
    uint64_t tmax[kThreads];
    uint64_t prefix, mask, thr;
    uint32_t remaining;
    int cnt, sel_cnt, done;
};

constexpr int kRankMax = 512;   // candidates ranked directly (more -> radix select first)

// Every thread passes the largest key it holds (0 if none).  Returns a key T
// such that at least min(k, #keys) keys are >= T: the k-th largest of the
// per-thread maxima (those k maxima are themselves >= T), or 1 (accept every
// real key) when fewer than k threads hold a key.
__device__ inline uint64_t kth_of_maxima(SelShared& S, uint64_t m, int k, int tid)
{
    S.tmax[tid] = m;
    if (tid == 0) S.thr = 1;
    const int nz = __syncthreads_count(m != 0);
    if (nz < k) return 1;
    if (m != 0) {
        int r = 0;
        for (int i = 0; i < kThreads; i += 16) {
            u64x2 v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) v[u] = *(const u64x2*)(S.tmax + i + 2 * u);
#pragma unroll
            for (int u = 0; u < 8; ++u) r += (int)(v[u][0] > m) + (int)(v[u][1] > m);
        }
        if (r == k - 1) S.thr = m;
    }
    __syncthreads();
    return S.thr;
}

// Finds the digit prefix of the k-th largest key among buf[0..n): afterwards
// exactly k keys satisfy (key & S.mask) >= S.prefix.  Requires n >= k >= 1.
__device__ inline void radix_kth(SelShared& S, int n, int k, int tid)
{
    const int lane = tid & 63, wave = tid >> 6;
    if (tid == 0) { S.prefix = 0; S.mask = 0; S.remaining = (uint32_t)k; S.done = 0; }
    __syncthreads();
    for (int shift = 56; shift >= 0; shift -= 8) {
        for (int i = tid; i < kWaves * 256; i += kThreads) (&S.hist[0][0])[i] = 0;
        __syncthreads();
        const uint64_t prefix = S.prefix, mask = S.mask;
        for (int i = tid; i < n; i += kThreads) {
            const uint64_t key = S.buf[i];
            if ((key & mask) == prefix) atomicAdd(&S.hist[wave][(key >> shift) & 255u], 1u);
        }
        __syncthreads();
        if (wave == 0) {
            uint32_t c[4];
#pragma unroll
            for (int e = 0; e < 4; ++e)
                c[e] = S.hist[0][4 * lane + e] + S.hist[1][4 * lane + e] + S.hist[2][4 * lane + e] +
                       S.hist[3][4 * lane + e];
            const uint32_t lsum = c[0] + c[1] + c[2] + c[3];
            uint32_t suf = lsum;   // inclusive suffix sum over lanes
#pragma unroll
            for (int off = 1; off < 64; off <<= 1) {
                const uint32_t t = __shfl_down(suf, off, 64);
                if (lane + off < 64) suf += t;
            }
            const uint32_t rem = S.remaining;
            const uint64_t ball = __ballot(suf >= rem);
            const int L = ball ? 63 - __builtin_clzll(ball) : 0;
            if (lane == L) {
                uint32_t above = suf - lsum;
                int D = 4 * L;
                uint32_t cd = c[0];
#pragma unroll
                for (int e = 3; e >= 0; --e) {
                    if (above + c[e] >= rem) { D = 4 * L + e; cd = c[e]; break; }
                    above += c[e];
                }
                const uint32_t r2 = rem - above;
                S.prefix = prefix | ((uint64_t)D << shift);
                S.mask = mask | (0xFFull << shift);
                S.remaining = r2;
                S.done = (cd == r2);
            }
        }
        __syncthreads();
        if (S.done) break;
    }
}

// Keeps the k largest of buf[0..n) in buf[0..k) (unsorted); S.thr becomes the
// smallest kept key.  Requires n > k.
__device__ inline void select_compact(SelShared& S, int n, int k, int tid)
{
    radix_kth(S, n, k, tid);
    const uint64_t prefix = S.prefix, mask = S.mask;
    if (tid == 0) S.sel_cnt = 0;
    __syncthreads();
    for (int i = tid; i < n; i += kThreads) {
        const uint64_t key = S.buf[i];
        if ((key & mask) >= prefix) {
            const int p = atomicAdd(&S.sel_cnt, 1);
            if (p < kMaxK) S.sel[p] = key;
        }
    }
    __syncthreads();
    if (tid < k) S.buf[tid] = S.sel[tid];
    if (tid < 64) {
        const int lane = tid;
        uint64_t m = ~0ull;
        for (int i = lane; i < k; i += 64) m = (S.sel[i] < m) ? S.sel[i] : m;
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) {
            const uint32_t lo = __shfl_xor((uint32_t)m, off, 64);
            const uint32_t hi = __shfl_xor((uint32_t)(m >> 32), off, 64);
            const uint64_t o = ((uint64_t)hi << 32) | lo;
            m = (o < m) ? o : m;
        }
        if (lane == 0) { S.thr = m; S.cnt = k; }
    }
    __syncthreads();
}

// Rank of `key` among buf[0..n) in descending key order (keys are unique).
__device__ inline int rank_desc(const SelShared& S, int n, uint64_t key)
{
    int r = 0;
    int i = 0;
    for (; i + 16 <= n; i += 16) {
        u64x2 v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) v[u] = *(const u64x2*)(S.buf + i + 2 * u);
#pragma unroll
        for (int u = 0; u < 8; ++u) r += (int)(v[u][0] > key) + (int)(v[u][1] > key);
    }
    for (; i < n; ++i) r += (int)(S.buf[i] > key);
    return r;
}

// Reduces buf[0..cnt) to its top k and calls emit(rank, key) for rank < k,
// rank 0 being the largest.  Returns the number of keys emitted.
template <class Emit>
__device__ inline int emit_topk(SelShared& S, int k, int tid, Emit emit)
{
    __syncthreads();
    int n = S.cnt < kSelCap ? S.cnt : kSelCap;
    if (n > kRankMax) {
        select_compact(S, n, k, tid);
        n = k;
    }
    __syncthreads();
    for (int i = tid; i < n; i += kThreads) {
        const uint64_t key = S.buf[i];
        const int r = rank_desc(S, n, key);
        if (r < k) emit(r, key);
    }
    return n < k ? n : k;
}

}  // namespace stk
