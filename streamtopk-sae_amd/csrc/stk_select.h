// stk_select.h -- workgroup-wide top-k selection over 64-bit sort keys held in
// LDS (radix select by 8-bit digits, most significant first), ranking by
// counting that emits the final k keys in descending order, and slot
// reservation with one LDS atomic per wave.
#pragma once
#include "stk_device.h"

namespace stk {

constexpr int kSelCap = 4096;   // keys held in LDS by one selection workgroup
constexpr int kMaxK = 128;

// The LDS state of one selection workgroup of NT threads (NT / 64 waves).
template <int NT>
struct SelSharedT {
    static constexpr int NW = NT / 64;
    uint64_t buf[kSelCap];
    uint32_t hist[NW][256];
    union {                  // never live together: each use ends at a barrier
        uint64_t sel[kMaxK];   // select_compact's kept keys
        uint64_t tmax[NT];     // kth_of_maxima's per-thread maxima
    };
    uint64_t wthr[NW];
    uint64_t prefix, mask, thr;
    alignas(16) uint32_t vote[2 * NW];   // block_any slots
    uint32_t remaining;
    int cnt, sel_cnt, done;
};
using SelShared = SelSharedT<kThreads>;

// Slots for c >= 0 items of each lane from the LDS counter *ctr, with one
// atomic per wave (same-address LDS atomics serialise lane by lane): returns
// the lane's first slot; the wave's slots are in lane order.  Every lane of
// the wave must take part.
__device__ inline int wave_reserve(int* ctr, int c)
{
    const int lane = (int)__lane_id();
    int x = c;   // inclusive scan over the lanes
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const int t = __shfl_up(x, off, 64);
        if (lane >= off) x += t;
    }
    const int total = __shfl(x, 63, 64);
    int base = 0;
    if (lane == 0 && total > 0) base = atomicAdd(ctr, total);
    return __shfl(base, 0, 64) + x - c;
}

// wave_reserve for one item per flagged lane.
__device__ inline int wave_reserve1(int* ctr, bool f)
{
    const uint64_t b = __ballot(f);
    const int pre = (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(b >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)b, 0u));
    int base = 0;
    if (__lane_id() == 0 && b != 0) base = atomicAdd(ctr, __popcll(b));
    return __shfl(base, 0, 64) + pre;
}

// Every thread passes the largest key it holds (0 if none).  Returns a key T
// such that at least k keys are >= T, or 1 (accept every real key) when a
// wave holds too few keys.  k is split over the NW waves (k_w = k / NW, the
// first k % NW waves one more); wave w's bound is the k_w-th largest of
// its 64 maxima, which are themselves keys, and T is the smallest bound over
// the waves with k_w > 0: at least sum k_w = k keys reach T.  Ranking within
// a wave costs 1 / NW of ranking all the workgroup's maxima.
template <int NT>
__device__ inline uint64_t kth_of_maxima(SelSharedT<NT>& S, uint64_t m, int k, int tid)
{
    constexpr int NW = NT / 64;
    const int lane = tid & 63, wave = tid >> 6;
    const int kw = k / NW + (wave < k % NW ? 1 : 0);
    S.tmax[tid] = m;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const int nz = __popcll(__ballot(m != 0));
    uint64_t tw = ~0ull;   // no bound from this wave
    if (kw > 0 && nz < kw) {
        tw = 1;
    } else if (kw > 0) {
        int r = 0;
        const uint64_t* wm = S.tmax + wave * 64;
#pragma unroll
        for (int i = 0; i < 64; i += 8) {
            u64x2 v[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) v[u] = *(const u64x2*)(wm + i + 2 * u);
#pragma unroll
            for (int u = 0; u < 4; ++u) r += (int)(v[u][0] > m) + (int)(v[u][1] > m);
        }
        // keys are distinct, so exactly one non-zero maximum has rank kw - 1
        const uint64_t hit = __ballot(m != 0 && r == kw - 1);
        const int src = __builtin_ctzll(hit);
        const uint32_t lo = __builtin_amdgcn_readlane((uint32_t)m, src);
        const uint32_t hi = __builtin_amdgcn_readlane((uint32_t)(m >> 32), src);
        tw = ((uint64_t)hi << 32) | lo;
    }
    if (lane == 0) S.wthr[wave] = tw;
    __syncthreads();
    uint64_t T = S.wthr[0];
#pragma unroll
    for (int w = 1; w < NW; ++w) T = S.wthr[w] < T ? S.wthr[w] : T;
    return T;
}

// Finds the digit prefix of the k-th largest key among buf[0..n): afterwards
// exactly k keys satisfy (key & S.mask) >= S.prefix.  Requires n >= k >= 1.
template <int NT>
__device__ inline void radix_kth(SelSharedT<NT>& S, int n, int k, int tid)
{
    constexpr int NW = NT / 64;
    const int lane = tid & 63, wave = tid >> 6;
    if (tid == 0) { S.prefix = 0; S.mask = 0; S.remaining = (uint32_t)k; S.done = 0; }
    __syncthreads();
    for (int shift = 56; shift >= 0; shift -= 8) {
        for (int i = tid; i < NW * 256; i += NT) (&S.hist[0][0])[i] = 0;
        __syncthreads();
        const uint64_t prefix = S.prefix, mask = S.mask;
        for (int i = tid; i < n; i += NT) {
            const uint64_t key = S.buf[i];
            if ((key & mask) == prefix) atomicAdd(&S.hist[wave][(key >> shift) & 255u], 1u);
        }
        __syncthreads();
        if (wave == 0) {
            uint32_t c[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                c[e] = S.hist[0][4 * lane + e];
#pragma unroll
                for (int w = 1; w < NW; ++w) c[e] += S.hist[w][4 * lane + e];
            }
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
template <int NT>
__device__ inline void select_compact(SelSharedT<NT>& S, int n, int k, int tid)
{
    radix_kth(S, n, k, tid);
    const uint64_t prefix = S.prefix, mask = S.mask;
    if (tid == 0) S.sel_cnt = 0;
    __syncthreads();
    for (int i0 = 0; i0 < n; i0 += NT) {
        const int i = i0 + tid;
        const uint64_t key = i < n ? S.buf[i] : 0ull;
        const bool f = i < n && (key & mask) >= prefix;
        const int p = wave_reserve1(&S.sel_cnt, f);
        if (f && p < kMaxK) S.sel[p] = key;
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

// Rank of buf[pos] = `key` among buf[0..n) in descending key order: the
// number of larger keys.  Keys hold their latent index, so the keys of one
// encode are distinct; kTies also counts the equal keys at lower positions,
// which keeps the ranks a permutation when a caller's keys repeat (shard
// results merged by stk_topk_merge).  Every thread reads the same LDS words
// (broadcast), 16 keys per round.
template <bool kTies, int NT>
__device__ inline int rank_desc(const SelSharedT<NT>& S, int n, uint64_t key, int pos)
{
    int r = 0;
    int i = 0;
    for (; i + 16 <= n; i += 16) {
        u64x2 v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) v[u] = *(const u64x2*)(S.buf + i + 2 * u);
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            if (kTies) {
                r += (int)(v[u][0] > key || (v[u][0] == key && i + 2 * u < pos)) +
                     (int)(v[u][1] > key || (v[u][1] == key && i + 2 * u + 1 < pos));
            } else {
                r += (int)(v[u][0] > key) + (int)(v[u][1] > key);
            }
        }
    }
    for (; i < n; ++i) r += (int)(S.buf[i] > key || (kTies && S.buf[i] == key && i < pos));
    return r;
}

// Reduces buf[0..cnt) to its top k and calls emit(rank, key) for rank < k,
// rank 0 being the largest.  Up to NT keys are ranked directly by counting
// (thread t ranks key t), more are first reduced to the k largest by radix
// selection.  Returns the number of keys emitted.
template <bool kTies = false, int NT, class Emit>
__device__ inline int emit_topk(SelSharedT<NT>& S, int k, int tid, Emit emit)
{
    __syncthreads();
    int n = S.cnt < kSelCap ? S.cnt : kSelCap;
    if (n > NT) {
        select_compact(S, n, k, tid);   // k <= kMaxK <= NT keys remain
        n = k;
    }
    if (tid < n) {
        const uint64_t key = S.buf[tid];
        const int r = rank_desc<kTies>(S, n, key, tid);
        if (r < k) emit(r, key);
    }
    return n < k ? n : k;
}

}  // namespace stk
