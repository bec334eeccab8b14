// stk_approx.hip -- kernels of the approximate (top-c per 128-latent group)
// variant that materialise the per-group candidates, for callers that ask for
// the candidate buffer (streamtopk_approx.cu:264-274 side effect).
//
//   group_kernel : MFMA scores for 256 latents (two groups) x up to 128 rows per
//                  tile, then per (row, group) a bitonic sort of the group's 128
//                  keys in LDS; writes each group's top-c, descending, padded
//                  with (-FLT_MAX, -1) past the end of F
//                  (streamtopk_approx.cu:42-167).
//   cand_kernel  : per row, top-k over all group candidates -- the final
//                  torch.topk + gather of the reference (ops.py:80-81), on the
//                  device.
#include "stk_kernels.h"

namespace stk {

size_t group_lds_bytes(int NB)
{
    const size_t BT = 32 * (size_t)NB;
    return 2 * BT * kXRowStride + 2 * 32 * kApproxGroup * sizeof(uint64_t);
}

template <int DT, int NB>
__global__ __launch_bounds__(kThreads, 1) void group_kernel(GroupArgs a)
{
    constexpr int BT = 32 * NB;
    constexpr int FRAGS = 2;
    constexpr int ES = Dt<DT>::esize;
    constexpr int DS = Dt<DT>::DS;
    constexpr int G = kApproxGroup;
    extern __shared__ __align__(16) unsigned char smem[];
    unsigned char* xs0 = smem;
    unsigned char* xs1 = smem + BT * kXRowStride;
    uint64_t* keys = (uint64_t*)(smem + 2 * BT * kXRowStride);   // [2 groups][32 cols][G]

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int h = lane >> 5, jl = lane & 31;
    const int64_t b0 = (int64_t)blockIdx.y * BT;
    const int64_t B = a.B, d = a.d, F = a.F;
    const int c = a.c;

    MainLoop<DT, NB, FRAGS> ml;
    ml.X = (const unsigned char*)a.X;
    ml.B = B;
    ml.d = d;
    ml.b0 = b0;
    ml.lane = lane;
    ml.h = h;
    const int64_t nds = (d + DS - 1) / DS;
    const unsigned char* W = (const unsigned char*)a.W;
    const int64_t num_tiles = (a.num_groups + 1) / 2;
    const int64_t t0 = (int64_t)blockIdx.x * a.tiles_per_wg;
    const int64_t t1 = (t0 + a.tiles_per_wg < num_tiles) ? t0 + a.tiles_per_wg : num_tiles;

    for (int64_t tile = t0; tile < t1; ++tile) {
        const int64_t fw0 = tile * kGroupTile + wave * 64;
#pragma unroll
        for (int fa = 0; fa < FRAGS; ++fa) {
            int64_t f = fw0 + fa * 32 + jl;
            f = (f < F) ? f : F - 1;
            ml.wrow[fa] = W + f * d * ES + h * 64;
        }
        f32x16 acc[FRAGS][NB];
#pragma unroll
        for (int fa = 0; fa < FRAGS; ++fa)
#pragma unroll
            for (int n = 0; n < NB; ++n)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[fa][n][r] = 0.f;
        ml.run(acc, 0, nds, xs0, xs1, tid);

        float bias_r[FRAGS][16];
#pragma unroll
        for (int fa = 0; fa < FRAGS; ++fa)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int64_t f = fw0 + fa * 32 + (r >> 2) * 8 + h * 4 + (r & 3);
                bias_r[fa][r] = a.bias[f < F ? f : 0];
            }

#pragma unroll
        for (int n = 0; n < NB; ++n) {
            // keys of this 32-column block: group g = wave / 2, slot within group
#pragma unroll
            for (int fa = 0; fa < FRAGS; ++fa)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int lt = wave * 64 + fa * 32 + (r >> 2) * 8 + h * 4 + (r & 3);
                    const int64_t f = tile * kGroupTile + lt;
                    const int g = lt / G, p = lt % G;
                    keys[((size_t)g * 32 + jl) * G + p] =
                        (f < F) ? make_key(acc[fa][n][r] + bias_r[fa][r], f) : 0ull;
                }
            __syncthreads();
            // bitonic sort (descending) of the 64 segments of G keys
            for (int size = 2; size <= G; size <<= 1) {
                for (int stride = size >> 1; stride > 0; stride >>= 1) {
                    for (int t = tid; t < 64 * (G / 2); t += kThreads) {
                        const int seg = t / (G / 2), u = t % (G / 2);
                        const int i = 2 * u - (u & (stride - 1));
                        const int jx = i + stride;
                        uint64_t* sk = keys + (size_t)seg * G;
                        const uint64_t x = sk[i], y = sk[jx];
                        const bool desc = ((i & size) == 0);
                        if (desc ? (x < y) : (x > y)) { sk[i] = y; sk[jx] = x; }
                    }
                    __syncthreads();
                }
            }
            // emit the top-c of each group of this column block
            for (int t = tid; t < 64 * c; t += kThreads) {
                const int seg = t / c, e = t % c;
                const int g = seg / 32, col = seg % 32;
                const int64_t row = b0 + 32 * n + col;
                const int64_t grp = tile * 2 + g;
                if (row < B && grp < a.num_groups) {
                    const uint64_t key = keys[(size_t)seg * G + e];
                    const size_t o = ((size_t)row * a.num_groups + grp) * c + e;
                    a.cand_vals[o] = key ? key_value(key) : -3.402823466e+38f;
                    a.cand_idxs[o] = key ? key_index(key) : -1;
                }
            }
            __syncthreads();
        }
    }
}

// Per row: top-k over the (value, index) candidates of every group.
__global__ __launch_bounds__(kThreads) void cand_kernel(CandArgs a)
{
    __shared__ SelShared S;
    const int tid = threadIdx.x;
    const int64_t row = blockIdx.x;
    const int k = a.k;
    if (tid == 0) { S.cnt = 0; S.thr = 0; }
    __syncthreads();
    int64_t cur = tid;
    const float* cv = a.cand_vals + row * a.per_row;
    const int32_t* ci = a.cand_idxs + row * a.per_row;
    for (;;) {
        const uint64_t thr = S.thr;
        bool stalled = false;
        while (cur < a.per_row) {
            const int32_t idx = ci[cur];
            if (idx >= 0) {
                const uint64_t key = make_key(cv[cur], idx);
                if (key > thr) {
                    const int pos = atomicAdd(&S.cnt, 1);
                    if (pos < kSelCap) {
                        S.buf[pos] = key;
                    } else {
                        stalled = true;
                        break;
                    }
                }
            }
            cur += kThreads;
        }
        __syncthreads();
        if (S.cnt >= kSelCap) select_compact(S, kSelCap, k, tid);
        if (!__syncthreads_or(stalled)) break;
    }
    const int n = S.cnt < kSelCap ? S.cnt : kSelCap;
    if (n > k) select_compact(S, n, k, tid);
    __syncthreads();
    const int m = n < k ? n : k;
    if (tid < m) {
        const uint64_t key = S.buf[tid];
        const int r = rank_desc(S, m, key);
        a.V[row * k + r] = key_value(key);
        a.I[row * k + r] = key_index(key);
    }
}

template <int DT, int NB>
static hipError_t launch_group_t(const GroupArgs& a, dim3 grid, hipStream_t st)
{
    const size_t lds = group_lds_bytes(NB);
    auto kern = group_kernel<DT, NB>;
    hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
    launch(kern, grid, dim3(kThreads), lds, st, a);
    return hipGetLastError();
}

hipError_t launch_group(int dt, int NB, const GroupArgs& a, dim3 grid, hipStream_t st)
{
#define STK_CASE(DTV, NBV) \
    if (dt == DTV && NB == NBV) return launch_group_t<DTV, NBV>(a, grid, st);
    STK_CASE(DT_BF16, 1) STK_CASE(DT_BF16, 2) STK_CASE(DT_BF16, 4)
    STK_CASE(DT_F16, 1) STK_CASE(DT_F16, 2) STK_CASE(DT_F16, 4)
    STK_CASE(DT_F32, 1) STK_CASE(DT_F32, 2) STK_CASE(DT_F32, 4)
#undef STK_CASE
    return hipErrorInvalidValue;
}

hipError_t launch_cand(const CandArgs& a, int64_t rows, hipStream_t st)
{
    launch(cand_kernel, dim3((unsigned)rows), dim3(kThreads), 0, st, a);
    return hipGetLastError();
}

}  // namespace stk
