// stk_kernels.hip -- gfx950 kernels of the streaming fused top-k SAE encoder.
//
//   sample_kernel  : fp32 scores of a strided sample of latents (split over d),
//                    the seed of the per-row thresholds.
//   seed_kernel    : per row, the exact top-k of the sample -> seed keys and
//                    the row threshold (the seed's k-th key).
//   main_kernel    : streams W once; MFMA scores for 256 latents x up to 128
//                    rows per tile; scores above the row threshold go to a
//                    per-row LDS queue that is rank-compacted to its top-k
//                    whenever it fills.  Emits each workgroup's queue.
//   merge_kernel   : per row, top-k of the seed plus every workgroup queue.
//
// The reference's pass 1 / pass 2 split (streamtopk_exact.cu:58-187 tile
// kernel, :429-499 merge kernel) maps to main_kernel / merge_kernel; its
// per-thread insertion buffers (topk_buffer.cuh) are replaced by threshold
// filtering against a row threshold that only ever rises, so almost no
// selection work is done in the streaming kernel.
#include "stk_kernels.h"

namespace stk {

// ---------------------------------------------------------------------------
// main_kernel
// ---------------------------------------------------------------------------
template <int DT, int NB>
__global__ __launch_bounds__(kMainThreads, 2) void main_kernel(MainArgs a)
{
    constexpr int BT = 32 * NB;
    constexpr int FRAGS = 1;
    constexpr int WAVES = kMainWaves;
    constexpr int DS = Dt<DT>::DS;
    extern __shared__ __align__(16) unsigned char smem[];
    unsigned char* xs0 = smem;
    unsigned char* xs1 = smem + BT * kXRowStride;
    uint64_t* q = (uint64_t*)(smem + 2 * BT * kXRowStride);
    const int cap = a.cap;
    uint64_t* thr = q + (size_t)BT * cap;
    int* cnt = (int*)(thr + BT);

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int h = lane >> 5, jl = lane & 31;
    const int64_t b0 = (int64_t)blockIdx.y * BT;
    const int64_t B = a.B, F = a.F;
    const int k = a.k;

    for (int i = tid; i < BT; i += kMainThreads) {
        cnt[i] = 0;
        thr[i] = (a.thr0 != nullptr && b0 + i < B) ? a.thr0[b0 + i] : 0ull;
    }

    TileStream<DT, NB, FRAGS, WAVES> ts;
    ts.W = (const unsigned char*)a.W;
    ts.w_row_bytes = a.d * Dt<DT>::esize;
    ts.bias = a.bias;
    ts.F = F;
    ts.tile_begin = (int64_t)blockIdx.x * a.tiles_per_wg;
    {
        const int64_t t1 = ts.tile_begin + a.tiles_per_wg;
        ts.ntiles = (int)((t1 < a.num_tiles ? t1 : a.num_tiles) - ts.tile_begin);
    }
    ts.nds = (int)(a.d / DS);
    ts.nds4 = (ts.nds + 3) & ~3;
    ts.tid = tid;
    ts.lane = lane;
    ts.wave = wave;
    ts.h = h;
    ts.jl = jl;
    ts.init_x((const unsigned char*)a.X, B, b0, a.d);
    const int64_t smask = a.samp_count ? ((int64_t)1 << a.samp_log2) - 1 : 0;

    constexpr int kRowsPerWave = BT / WAVES;   // queue rows this wave compacts (<= 64)
    f32x16 acc[FRAGS][NB];
    ts.run(acc, xs0, xs1, [&](int t, f32x16 (&ac)[FRAGS][NB], const float (&bias_r)[FRAGS][16]) {
        // latent of accumulator register r of this lane: fl + 8*(r/4) + r%4
        const int64_t fl = (ts.tile_begin + t) * (int64_t)kTileLatents + wave * 32 + h * 4;
        uint32_t vmask = 0;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int64_t f = fl + (r >> 2) * 8 + (r & 3);
            bool ok = f < F;
            if (a.samp_count && (f & smask) == 0 && (f >> a.samp_log2) < a.samp_count) ok = false;
            vmask |= ok ? (1u << r) : 0u;
        }
        // ---- filter against the row thresholds (float pre-check, exact key check) ----
        uint32_t pend[NB];
#pragma unroll
        for (int n = 0; n < NB; ++n) {
            const int j = 32 * n + jl;
            const uint64_t tk = thr[j];
            const float tv = tk ? key_value(tk) : -__builtin_inff();
            uint32_t m = 0;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const float sc = ac[0][n][r] + bias_r[0][r];
                m |= (!(sc < tv)) ? (1u << r) : 0u;
            }
            m &= (b0 + j < B) ? vmask : 0u;
            if (m && tk) {
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    if ((m >> r & 1u) && !(make_key(ac[0][n][r] + bias_r[0][r], fl + (r >> 2) * 8 + (r & 3)) > tk))
                        m &= ~(1u << r);
            }
            pend[n] = m;
        }

        // ---- append / compact until every passing score is placed or dropped ----
        for (int it = 0; it < 4096; ++it) {
            uint32_t any = 0;
#pragma unroll
            for (int n = 0; n < NB; ++n) any |= pend[n];
            if (!__syncthreads_or(any != 0)) break;
            // one slot reservation per (lane, row), then predicated stores
#pragma unroll
            for (int n = 0; n < NB; ++n) {
                if (pend[n] == 0) continue;
                const int j = 32 * n + jl;
                const int pos = atomicAdd(&cnt[j], __builtin_popcount(pend[n]));
                uint64_t* qj = q + (size_t)j * cap;
                int slot = pos;
                uint32_t keep = 0;
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    if (pend[n] >> r & 1u) {
                        if (slot < cap)
                            qj[slot] = make_key(ac[0][n][r] + bias_r[0][r], fl + (r >> 2) * 8 + (r & 3));
                        else
                            keep |= 1u << r;
                        ++slot;
                    }
                }
                pend[n] = keep;
            }
            __syncthreads();
            // wave w compacts its rows w*kRowsPerWave + i whose queue is full
            {
                const int myrow = wave * kRowsPerWave + (lane < kRowsPerWave ? lane : 0);
                uint64_t full = __ballot(lane < kRowsPerWave && cnt[myrow] >= cap);
                while (full) {
                    const int i = __builtin_ctzll(full);
                    full &= full - 1;
                    const int row = wave * kRowsPerWave + i;
                    uint64_t* qr = q + (size_t)row * cap;
                    uint64_t e[3];
                    int rk[3] = {0, 0, 0};
#pragma unroll
                    for (int m = 0; m < 3; ++m) e[m] = (lane + 64 * m < cap) ? qr[lane + 64 * m] : 0ull;
                    for (int ii = 0; ii < cap; ii += 2) {
                        const u64x2 v = *(const u64x2*)(qr + ii);
#pragma unroll
                        for (int m = 0; m < 3; ++m) rk[m] += (int)(v[0] > e[m]) + (int)(v[1] > e[m]);
                    }
#pragma unroll
                    for (int m = 0; m < 3; ++m) {
                        if (lane + 64 * m < cap && rk[m] < k) {
                            qr[rk[m]] = e[m];
                            if (rk[m] == k - 1) thr[row] = e[m];
                        }
                    }
                    if (lane == 0) cnt[row] = k;
                }
            }
            __syncthreads();
            // drop pending scores that fell below a raised threshold
#pragma unroll
            for (int n = 0; n < NB; ++n) {
                if (pend[n] == 0) continue;
                const uint64_t tk = thr[32 * n + jl];
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    if ((pend[n] >> r & 1u) && !(make_key(ac[0][n][r] + bias_r[0][r], fl + (r >> 2) * 8 + (r & 3)) > tk))
                        pend[n] &= ~(1u << r);
            }
        }
    });

    // ---- emit this workgroup's queues ----
    __syncthreads();
    for (int idx = tid; idx < BT * cap; idx += kMainThreads) {
        const int row = idx / cap, e = idx - row * cap;
        if (b0 + row < B) {
            const int c = cnt[row] < cap ? cnt[row] : cap;
            const size_t seg = (size_t)(b0 + row) * a.nwg + blockIdx.x;
            if (e < c) a.out_keys[seg * cap + e] = q[(size_t)row * cap + e];
            if (e == 0) a.out_cnt[seg] = c;
        }
    }
}

// ---------------------------------------------------------------------------
// sample_kernel: P[row][i] = X[row] . W[i << samp_log2] + b[i << samp_log2]
// for the sampled latents i < count.  A workgroup owns 32 sampled latents x 32
// rows; its four waves take interleaved quarters of the d-steps and their fp32
// partial sums are added in a fixed order (deterministic).  Operands are read
// straight from global memory (W rows once, X rows from L2).
// ---------------------------------------------------------------------------
template <int DT>
__global__ __launch_bounds__(kThreads) void sample_kernel(SampleArgs a)
{
    constexpr int ES = Dt<DT>::esize;
    constexpr int DS = Dt<DT>::DS;
    __shared__ float red[kWaves - 1][16][64 + 1];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int h = lane >> 5, jl = lane & 31;
    const int64_t ib = (int64_t)blockIdx.x * 32;
    const int64_t jb = (int64_t)blockIdx.y * 32;
    const int64_t d = a.d;
    const int64_t nds = (d + DS - 1) / DS;

    int64_t i = ib + jl;
    i = (i < a.count) ? i : a.count - 1;
    const unsigned char* wp = (const unsigned char*)a.W + (i << a.samp_log2) * d * ES + h * 64;
    const int64_t j = jb + jl;
    const bool jok = j < a.B;
    const unsigned char* xp = (const unsigned char*)a.X + (jok ? j : 0) * d * ES + h * 64;

    f32x16 acc;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] = 0.f;
    for (int64_t s0 = wave; s0 < nds; s0 += 4 * kWaves) {
        u32x4 wq[4][4], xq[4][4];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const int64_t s = s0 + t * kWaves;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int64_t e0 = s * DS + h * (DS / 2) + q * (DS / 8);
                const bool ok = s < nds && e0 < d;
                wq[t][q] = ok ? *(const u32x4*)(wp + s * kStepBytes + q * 16) : u32x4{0u, 0u, 0u, 0u};
                xq[t][q] = (ok && jok) ? *(const u32x4*)(xp + s * kStepBytes + q * 16) : u32x4{0u, 0u, 0u, 0u};
            }
        }
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int q = 0; q < 4; ++q) mfma_quad<DT>(acc, wq[t][q], xq[t][q]);
    }
    if (wave > 0) {
#pragma unroll
        for (int r = 0; r < 16; ++r) red[wave - 1][r][lane] = acc[r];
    }
    __syncthreads();
    if (wave == 0 && jok) {
        float* prow = a.P + j * a.count;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int64_t ii = ib + (r >> 2) * 8 + h * 4 + (r & 3);
            if (ii < a.count) {
                const float s = ((acc[r] + red[0][r][lane]) + red[1][r][lane]) + red[2][r][lane];
                prow[ii] = s + a.bias[ii << a.samp_log2];
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Selection kernels (one workgroup per row).
// ---------------------------------------------------------------------------
__device__ inline void append_key(SelShared& S, uint64_t key, bool& stalled)
{
    const int pos = atomicAdd(&S.cnt, 1);
    if (pos < kSelCap)
        S.buf[pos] = key;
    else
        stalled = true;
}

// Per row: exact top-k of the sampled scores -> seed keys and row threshold.
__global__ __launch_bounds__(kThreads) void seed_kernel(SeedArgs a)
{
    constexpr int kItems = kSampleTarget / kThreads;
    __shared__ SelShared S;
    const int tid = threadIdx.x;
    const int64_t row = blockIdx.x;
    const int k = a.k;
    const float* prow = a.P + row * a.count;
    uint64_t key[kItems];
    uint64_t m = 0;
#pragma unroll
    for (int t = 0; t < kItems; ++t) {
        const int64_t i = tid + (int64_t)t * kThreads;
        key[t] = (i < a.count) ? make_key(prow[i], i << a.samp_log2) : 0ull;
        m = key[t] > m ? key[t] : m;
    }
    if (tid == 0) S.cnt = 0;
    const uint64_t T = kth_of_maxima(S, m, k, tid);
    bool stalled = false;
#pragma unroll
    for (int t = 0; t < kItems; ++t)
        if (key[t] != 0 && key[t] >= T) append_key(S, key[t], stalled);
    emit_topk(S, k, tid, [&](int r, uint64_t kk) {
        a.seed_keys[row * k + r] = kk;
        if (r == k - 1) a.thr[row] = kk;
    });
}

// Per row: top-k of the seed keys plus every main_kernel workgroup queue.
__global__ __launch_bounds__(kThreads) void merge_kernel(MergeArgs a)
{
    __shared__ SelShared S;
    const int tid = threadIdx.x;
    const int64_t row = blockIdx.x;
    const int k = a.k;
    // pass 1: each thread's largest key (seed entry tid, segments tid + 256 j)
    uint64_t m = 0;
    if (a.seed_keys != nullptr && tid < k) m = a.seed_keys[row * k + tid];
    for (int64_t seg = tid; seg < a.nseg; seg += kThreads) {
        const int64_t sid = row * a.nseg + seg;
        const int c = a.seg_cnt[sid];
        const uint64_t* keys = a.seg_keys + sid * a.cap;
#pragma unroll 8
        for (int e = 0; e < c; ++e) {
            const uint64_t kk = keys[e];
            m = kk > m ? kk : m;
        }
    }
    if (tid == 0) S.cnt = 0;
    const uint64_t T = kth_of_maxima(S, m, k, tid);
    // pass 2: append every key >= the running threshold; compact when full
    bool seed_done = !(a.seed_keys != nullptr && tid < k);
    int64_t seg = tid;
    int e = 0;
    for (;;) {
        const uint64_t thr = S.thr > T ? S.thr : T;
        bool stalled = false;
        if (!seed_done) {
            const uint64_t kk = a.seed_keys[row * k + tid];
            if (kk >= thr) append_key(S, kk, stalled);
            seed_done = !stalled;
        }
        while (!stalled && seg < a.nseg) {
            const int64_t sid = row * a.nseg + seg;
            const int c = a.seg_cnt[sid];
            const uint64_t* keys = a.seg_keys + sid * a.cap;
            while (e < c) {
                const uint64_t kk = keys[e];
                if (kk >= thr) {
                    append_key(S, kk, stalled);
                    if (stalled) break;
                }
                ++e;
            }
            if (stalled) break;
            seg += kThreads;
            e = 0;
        }
        __syncthreads();
        if (S.cnt >= kSelCap) select_compact(S, kSelCap, k, tid);
        if (!__syncthreads_or(stalled)) break;
    }
    emit_topk(S, k, tid, [&](int r, uint64_t kk) {
        a.V[row * k + r] = key_value(kk);
        a.I[row * k + r] = key_index(kk);
    });
}

// ---------------------------------------------------------------------------
// Host-side launch helpers
// ---------------------------------------------------------------------------
size_t main_lds_bytes(int NB, int cap)
{
    const size_t BT = 32 * (size_t)NB;
    return 2 * BT * kXRowStride + BT * (size_t)cap * 8 + BT * 8 + BT * 4;
}

template <int DT, int NB>
static hipError_t launch_main_t(const MainArgs& a, dim3 grid, hipStream_t st)
{
    const size_t lds = main_lds_bytes(NB, a.cap);
    auto kern = main_kernel<DT, NB>;
    hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(kern, grid, dim3(kMainThreads), lds, st, a);
    return hipGetLastError();
}

hipError_t launch_main(int dt, int NB, const MainArgs& a, dim3 grid, hipStream_t st)
{
#define STK_CASE(DTV, NBV) \
    if (dt == DTV && NB == NBV) return launch_main_t<DTV, NBV>(a, grid, st);
    STK_CASE(DT_BF16, 1) STK_CASE(DT_BF16, 2) STK_CASE(DT_BF16, 4)
    STK_CASE(DT_F16, 1) STK_CASE(DT_F16, 2) STK_CASE(DT_F16, 4)
    STK_CASE(DT_F32, 1) STK_CASE(DT_F32, 2) STK_CASE(DT_F32, 4)
#undef STK_CASE
    return hipErrorInvalidValue;
}

hipError_t launch_sample(int dt, const SampleArgs& a, dim3 grid, hipStream_t st)
{
    if (dt == DT_BF16) hipLaunchKernelGGL(sample_kernel<DT_BF16>, grid, dim3(kThreads), 0, st, a);
    else if (dt == DT_F16) hipLaunchKernelGGL(sample_kernel<DT_F16>, grid, dim3(kThreads), 0, st, a);
    else if (dt == DT_F32) hipLaunchKernelGGL(sample_kernel<DT_F32>, grid, dim3(kThreads), 0, st, a);
    else return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t launch_seed(const SeedArgs& a, int64_t rows, hipStream_t st)
{
    hipLaunchKernelGGL(seed_kernel, dim3((unsigned)rows), dim3(kThreads), 0, st, a);
    return hipGetLastError();
}

hipError_t launch_merge(const MergeArgs& a, int64_t rows, hipStream_t st)
{
    hipLaunchKernelGGL(merge_kernel, dim3((unsigned)rows), dim3(kThreads), 0, st, a);
    return hipGetLastError();
}

}  // namespace stk
