// stk_approx.hip -- kernels of the approximate (top-c per 128-latent group)
// variant that materialise the per-group candidates, for callers that ask for
// the candidate buffer (streamtopk_approx.cu:264-274 side effect).
//
//   group_kernel : TileStream (W streamed once, MFMA scores for 256 latents =
//                  two groups x up to 128 rows per tile); per 32-row block the
//                  scores go to LDS as order-preserving words, then each
//                  16-lane row of a wave sorts one (row, group)'s 128 keys in
//                  registers (bitonic network, one-direction form: 8 keys per
//                  lane, lane exchanges by DPP; 32-bit keys, with a 64-bit pass where truncated
//                  scores tie) and writes the group's top-c, descending, padded
//                  with (-FLT_MAX, -1) past the end of F
//                  (streamtopk_approx.cu:42-167).
//   cand_kernel  : per row, top-k over all group candidates -- the final
//                  torch.topk + gather of the reference (ops.py:80-81), on the
//                  device.  Only the groups whose head reaches a lower bound of
//                  the row's k-th largest candidate are read past their head.
#include "stk_kernels.h"
#include "stk_select.h"

namespace stk {

constexpr int kOrdStride = kGroupTile + 4;   // LDS words per staged row (pad: no bank conflicts)
// Group heads are collected in LDS over kHeadTiles tiles, so that each row's
// heads reach global memory as whole 128-byte lines (16 groups of 8 bytes):
// written tile by tile, 16 bytes of a line at a time, they cost c3's
// group_kernel ~3-4 %.
constexpr int kHeadTiles = 8;
constexpr int kHeadSlots = 2 * kHeadTiles;   // groups per row and window

size_t group_lds_bytes(int NB)
{
    const size_t rings = 2 * (size_t)kGroupTile * kXRowStride + 2 * 32 * (size_t)NB * kXRowStride;
    return rings + 2 * kGroupTile * sizeof(float) + 32 * (size_t)kOrdStride * sizeof(uint32_t) +
           32 * (size_t)NB * kHeadSlots * sizeof(uint64_t);
}

// Key of lane l ^ X within the lane's 16-lane row, X = 1 .. 15.  XOR 1, 3
// and 2 are quad permutations, 7 and 15 mirror the half row and the row, 8
// rotates the row by 8; 4 goes through the LDS crossbar.
template <int X>
__device__ __forceinline__ uint32_t row_xor(uint32_t v)
{
    static_assert(X == 1 || X == 2 || X == 3 || X == 4 || X == 7 || X == 8 || X == 15, "lane exchange");
    if constexpr (X == 4) {
        return __shfl_xor(v, 4, 64);
    } else {
        // quad_perm [1,0,3,2], [2,3,0,1], [3,2,1,0]; row_half_mirror; row_ror:8; row_mirror
        constexpr int ctl = X == 1 ? 0xB1 : X == 2 ? 0x4E : X == 3 ? 0x1B : X == 7 ? 0x141 : X == 8 ? 0x128 : 0x140;
        return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, ctl, 0xF, 0xF, true);
    }
}

template <int X>
__device__ __forceinline__ uint64_t row_xor(uint64_t v)
{
    const uint32_t lo = row_xor<X>((uint32_t)v), hi = row_xor<X>((uint32_t)(v >> 32));
    return ((uint64_t)hi << 32) | lo;
}

// The bitonic network in its one-direction form, over the 128 keys of a
// 16-lane row; lane l holds entries 8l .. 8l+7 in v[0..7].  Merging sorted
// blocks of SIZE/2 into blocks of SIZE starts with a flip (entry e against
// the mirrored entry e ^ (SIZE-1)) and continues with half-cleaners (e against
// e ^ STRIDE); every comparator puts the larger key at the lower entry, so
// the result is descending.  Keys are distinct apart from the padding key 0.
template <class T>
__device__ __forceinline__ T kmax(T a, T b) { return a > b ? a : b; }
template <class T>
__device__ __forceinline__ T kmin(T a, T b) { return a > b ? b : a; }

template <int SIZE, class T>
__device__ __forceinline__ void bitonic_flip(T (&v)[8], int l)
{
    if constexpr (SIZE <= 8) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int p = j ^ (SIZE - 1);
            if (p < j) continue;
            const T x = v[j], y = v[p];
            v[j] = kmax(x, y);
            v[p] = kmin(x, y);
        }
    } else {
        // partner: lane l ^ (SIZE/8 - 1), register 7 - j
        const bool lower = (l & (SIZE / 16)) == 0;
        T o[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) o[j] = row_xor<SIZE / 8 - 1>(v[7 - j]);
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = lower ? kmax(v[j], o[j]) : kmin(v[j], o[j]);
    }
}

template <int STRIDE, class T>
__device__ __forceinline__ void bitonic_half(T (&v)[8], int l)
{
    if constexpr (STRIDE >= 8) {
        const bool lower = (l & (STRIDE / 8)) == 0;
        T o[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) o[j] = row_xor<STRIDE / 8>(v[j]);
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = lower ? kmax(v[j], o[j]) : kmin(v[j], o[j]);
    } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            if (j & STRIDE) continue;
            const T x = v[j], y = v[j + STRIDE];
            v[j] = kmax(x, y);
            v[j + STRIDE] = kmin(x, y);
        }
    }
    if constexpr (STRIDE > 1) bitonic_half<STRIDE / 2>(v, l);
}

// Sorts the row's 128 keys into descending order: entry e = 8l + j.  With
// SIZE < 128, sorts every aligned block of SIZE entries instead.
template <int SIZE = 128, class T>
__device__ __forceinline__ void bitonic_sort128(T (&v)[8], int l)
{
    if constexpr (SIZE > 2) bitonic_sort128<SIZE / 2, T>(v, l);
    bitonic_flip<SIZE>(v, l);
    if constexpr (SIZE >= 4) bitonic_half<SIZE / 4>(v, l);
}

// The row's top C (C = 16, 32, 64) in entries 0 .. C-1, descending, without
// sorting all 128: every aligned block of C entries is sorted, then blocks
// are merged pairwise keeping the larger half -- entry e of a block against
// the mirrored entry e ^ (SIZE - 1) of its partner block, the larger kept,
// which leaves each block a bitonic sequence holding the pair's top C, sorted
// again by the half-cleaners of size C.  Both blocks of a pair end up with the
// same sorted top C, so at the next level every block's mirror partner is a
// copy of the other half's top C.  Entries C .. 127 hold copies.
template <int C, int SIZE = 2 * C, class T>
__device__ __forceinline__ void bitonic_topc_merge(T (&v)[8], int l)
{
    if constexpr (SIZE <= 128) {
        static_assert(SIZE >= 16, "cross-lane partner blocks");
        T o[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) o[j] = row_xor<SIZE / 8 - 1>(v[7 - j]);
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = kmax(v[j], o[j]);
        bitonic_half<C / 2>(v, l);
        bitonic_topc_merge<C, SIZE * 2>(v, l);
    }
}

template <int C, class T>
__device__ __forceinline__ void bitonic_topc(T (&v)[8], int l)
{
    bitonic_sort128<C, T>(v, l);
    if constexpr (C < 128) bitonic_topc_merge<C>(v, l);
}

// Sorts one (row, group) segment of a staged 32-row block: the wave's 16-lane
// row l = lane % 16 takes the 128 staged words of block row rl, group g
// (latents 128 g .. of tile `tile`), sorts them in registers (8 per lane)
// and writes the group's top-c, descending, padded with (-FLT_MAX, -1) past
// the end of F, for output row rowblk + rl (streamtopk_approx.cu:118-166).
// The group's head key goes to slot 2 (tile % kHeadTiles) + g of the row's
// LDS head line hrow[rl].  Every lane of the wave takes part.
template <int C>
__device__ __forceinline__ void sort_segment(const GroupArgs& a, const uint32_t* ordv, uint64_t* hrow, int rl, int g,
                                             int l, int64_t rowblk, int64_t tile)
{
    constexpr int c = C;
    const int64_t B = a.B, G = a.num_groups;
    const int64_t f0 = tile * kGroupTile;
    const uint32_t* src = ordv + rl * kOrdStride + g * kApproxGroup;
    const u32x4 w0 = *(const u32x4*)(src + 8 * l), w1 = *(const u32x4*)(src + 8 * l + 4);
    // Short keys: the ordered word with its low 7 bits replaced by
    // 127 - position, so equal truncated words go to the lower
    // position; padding (word 0) sorts last.  Entries with equal
    // truncated words end up adjacent, so unless two such real
    // entries meet within the first c + 1, the short order is the
    // exact one.
    uint32_t v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j)
        v[j] = ((j < 4 ? w0[j] : w1[j - 4]) & ~0x7Fu) | (uint32_t)(127 - (8 * l + j));
    // c < 128: only the top c are selected and ordered (entries c ..
    // 127 end up holding copies); c = 128: the full sort
    bitonic_topc<C>(v, l);
    // Every LDS read of the checks below is issued before any is waited for:
    // the staged words of this lane's entries (a position always lies inside
    // the row), the entry after this lane's last, and for c < 128 the row's
    // words again (rather than held through the network).
    uint32_t word[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) word[j] = src[127u - (v[j] & 0x7Fu)];
    const uint32_t nx = __shfl_down(v[0], 1, 16);   // entry 8l + 8
    u32x4 r0 = {0u, 0u, 0u, 0u}, r1 = {0u, 0u, 0u, 0u};
    if constexpr (C < 128) {
        r0 = *(const u32x4*)(src + 8 * l);
        r1 = *(const u32x4*)(src + 8 * l + 4);
    }
    bool tie = false;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const uint32_t y = j < 7 ? v[j + 1] : nx;
        tie |= 8 * l + j < c - 1 && (y >> 7) != 0 && (v[j] >> 7) == (y >> 7);
    }
    if constexpr (C < 128) {
        // the (c+1)-th is not at hand: a real entry outside the top c
        // whose truncated word equals the c-th's shows as more than c
        // real entries at or above that word.  Entry c - 1 is register 7
        // of lane c/8 - 1 of this 16-lane row (read lane by lane: every
        // lane of the wave is active), the count is summed over the row
        // by rotations
        const int rq = (int)(__lane_id() >> 4);
        const uint32_t e0 = __builtin_amdgcn_readlane(v[7], c / 8 - 1);
        const uint32_t e1 = __builtin_amdgcn_readlane(v[7], 16 + c / 8 - 1);
        const uint32_t e2 = __builtin_amdgcn_readlane(v[7], 32 + c / 8 - 1);
        const uint32_t e3 = __builtin_amdgcn_readlane(v[7], 48 + c / 8 - 1);
        const uint32_t tc = (rq == 0 ? e0 : rq == 1 ? e1 : rq == 2 ? e2 : e3) >> 7;
        int above = 0;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const uint32_t ov = j < 4 ? r0[j] : r1[j - 4];
            above += (ov != 0u && (ov >> 7) >= tc) ? 1 : 0;
        }
        // row_ror:8, 4, 2, 1: every lane ends with the row's sum
        above += __builtin_amdgcn_mov_dpp(above, 0x128, 0xF, 0xF, false);
        above += __builtin_amdgcn_mov_dpp(above, 0x124, 0xF, 0xF, false);
        above += __builtin_amdgcn_mov_dpp(above, 0x122, 0xF, 0xF, false);
        above += __builtin_amdgcn_mov_dpp(above, 0x121, 0xF, 0xF, false);
        tie |= tc != 0u && above != c;
    }
    float val[8];
    uint32_t idx[8];
    const uint32_t fg = (uint32_t)(f0 + g * kApproxGroup);
    if (__ballot(tie) == 0) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const uint32_t pos = 127u - (v[j] & 0x7Fu);
            const bool real = (v[j] >> 7) != 0;
            val[j] = real ? key_value((uint64_t)word[j] << 32) : -3.402823466e+38f;
            idx[j] = real ? fg + pos : 0xFFFFFFFFu;
        }
    } else {
        // full keys for this wave's four segments
        uint64_t u[8];
        const u32x4 q0 = *(const u32x4*)(src + 8 * l), q1 = *(const u32x4*)(src + 8 * l + 4);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const uint32_t ov = j < 4 ? q0[j] : q1[j - 4];
            u[j] = ov ? (((uint64_t)ov << 32) | (0xFFFFFFFFu - (fg + 8 * l + j))) : 0ull;
        }
        bitonic_sort128(u, l);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            val[j] = u[j] ? key_value(u[j]) : -3.402823466e+38f;
            idx[j] = u[j] ? (uint32_t)key_index(u[j]) : 0xFFFFFFFFu;
        }
    }
    const int64_t row = rowblk + rl;
    const int64_t grp = 2 * tile + g;
    if (row < B && grp < G && 8 * l < c) {
        // the block's uniform part, then this lane's, recomputed at
        // every store (the empty asm hides rl's invariance: hoisted,
        // the 64-bit lane offsets of every block would be held in
        // registers through the tile loop, and spilled)
        const int64_t ob = (rowblk * G + 2 * tile) * c;
        int rlv = rl;
        asm volatile("" : "+v"(rlv));
        const int64_t o = ob + ((int64_t)rlv * G + g) * c + 8 * l;
        *(f32x4*)(a.cand_vals + o) = f32x4{val[0], val[1], val[2], val[3]};
        *(f32x4*)(a.cand_vals + o + 4) = f32x4{val[4], val[5], val[6], val[7]};
        *(u32x4*)(a.cand_idxs + o) = u32x4{idx[0], idx[1], idx[2], idx[3]};
        *(u32x4*)(a.cand_idxs + o + 4) = u32x4{idx[4], idx[5], idx[6], idx[7]};
        // the group's head (entry 0, this lane's first) as cand_kernel keys it
        if (l == 0)
            hrow[rl * kHeadSlots + 2 * (int)(tile % kHeadTiles) + g] =
                idx[0] != 0xFFFFFFFFu ? make_key(val[0], (int32_t)idx[0]) : 0ull;
    }
}

template <int DT, int NB, int C>
__global__ __launch_bounds__(kMainThreads, 1) void group_kernel(GroupArgs a)
{
    using TS = TileStream<DT, NB, kMainWaves>;
    static_assert(TS::kTileF == kGroupTile && kGroupTile == 2 * kApproxGroup, "one tile is two groups");
    extern __shared__ __align__(16) unsigned char smem[];
    float* bias_lds = (float*)(smem + TS::kRingBytes);             // [2][kGroupTile]
    uint32_t* ordv = (uint32_t*)(bias_lds + 2 * kGroupTile);       // [32 rows][kOrdStride]
    uint64_t* hbuf = (uint64_t*)(ordv + 32 * kOrdStride);          // [32*NB rows][kHeadSlots] head keys

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int h = lane >> 5, jl = lane & 31;
    const int l = lane & 15, sq = lane >> 4;
    const int64_t b0 = (int64_t)blockIdx.y * (32 * NB);
    const int64_t B = a.B, F = a.F, G = a.num_groups;
    const int64_t num_tiles = (G + 1) / 2;

    TS ts;
    ts.W = (const unsigned char*)a.W;
    ts.w_row_bytes = a.d * Dt<DT>::esize;
    ts.bias = a.bias;
    ts.F = F;
    ts.tile_begin = (int64_t)blockIdx.x * a.tiles_per_wg;
    {
        const int64_t t1 = ts.tile_begin + a.tiles_per_wg;
        ts.ntiles = (int)((t1 < num_tiles ? t1 : num_tiles) - ts.tile_begin);
    }
    ts.nds = (int)((a.d + Dt<DT>::DS - 1) / Dt<DT>::DS);
    ts.tail = (int)(a.d % Dt<DT>::DS);
    ts.nds2 = (ts.nds + 1) / 2 * 2;
    ts.tid = tid;
    ts.lane = lane;
    ts.wave = wave;
    ts.h = h;
    ts.jl = jl;
    ts.init_x((const unsigned char*)a.X, B, b0, a.d);

    f32x16 acc[NB];
    // the accumulators start at the bias (as in main_kernel, so the two
    // kernels' scores are bit-identical): ac holds the scores at the epilogue
    ts.template run<true>(acc, smem, bias_lds, [&](int t, f32x16 (&ac)[NB], const float (&)[16]) {
        const int64_t tile = ts.tile_begin + t;
        const int64_t f0 = tile * kGroupTile;
        // accumulator register r of this lane: row 32n + jl, latent lt0 + 8*(r/4) + r%4
        const int lt0 = wave * 32 + h * 4;
#pragma unroll
        for (int n = 0; n < NB; ++n) {
            if (n > 0) __syncthreads();   // the previous block's keys are read
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                u32x4 o;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int r = 4 * q + i;
                    o[i] = (f0 + lt0 + 8 * q + i < F) ? ordered_u32(ac[n][r]) : 0u;
                }
                *(u32x4*)(ordv + jl * kOrdStride + lt0 + 8 * q) = o;
            }
            __syncthreads();
            // 64 (row, group) segments per block, 4 per wave and round
#pragma unroll
            for (int rd = 0; rd < 2; ++rd) {
                const int seg = wave * 8 + rd * 4 + sq;
                const int rl = seg >> 1, g = seg & 1;
                sort_segment<C>(a, ordv, hbuf + 32 * n * kHeadSlots, rl, g, l, b0 + 32 * n, tile);
            }
        }
        // At the end of a head window (kHeadTiles aligned tiles) and after the
        // workgroup's last tile: the window's heads, whole lines per row where
        // the window is this workgroup's alone.  The next writes to hbuf come
        // after the next tile's first d-step barrier.
        if (tile % kHeadTiles == kHeadTiles - 1 || t == ts.ntiles - 1) {
            __syncthreads();   // every segment's head is in hbuf
            const int64_t wt = tile - tile % kHeadTiles;                    // the window's first tile
            const int64_t g0 = 2 * (wt > ts.tile_begin ? wt : ts.tile_begin);
            const int64_t g1 = 2 * tile + 2 < G ? 2 * tile + 2 : G;          // groups [g0, g1) are this workgroup's
            for (int i = tid; i < 32 * NB * kHeadSlots; i += kMainThreads) {
                const int r = i / kHeadSlots, sl = i % kHeadSlots;
                const int64_t row = b0 + r, grp = 2 * wt + sl;
                if (row < B && grp >= g0 && grp < g1) a.heads[row * G + grp] = hbuf[i];
            }
        }
    });
}

// Key of group g's head (its largest candidate), 0 for a padded group.
// Group g's head key from the compact heads (0 past the last group): one
// 8-byte word per group instead of a value and an index c entries apart.
__device__ __forceinline__ uint64_t head_key(const uint64_t* hd, int64_t g, int64_t G)
{
    const uint64_t h = hd[g < G ? g : G - 1];
    return g < G ? h : 0ull;
}

// Per row: top-k over the (value, index) candidates of every group.  Each
// group's candidates are in descending order, so the row's top k lie among
// the first k of every group, and a group whose head is below a key that k
// candidates reach holds none of them.  The heads' k-th largest maximum over
// the threads is such a key.
__global__ __launch_bounds__(kThreads) void cand_kernel(CandArgs a)
{
    __shared__ SelShared S;
    constexpr int U = 8;   // groups per thread whose heads are loaded together
    const int tid = threadIdx.x;
    const int64_t row = blockIdx.x;
    const int k = a.k, c = a.c;
    const int64_t G = a.num_groups;
    const float* cv = a.cand_vals + row * G * c;
    const int32_t* ci = a.cand_idxs + row * G * c;
    const uint64_t* hd = a.heads + row * G;

    uint64_t m = 0;
    for (int64_t g0 = tid; g0 < G; g0 += U * kThreads) {
        uint64_t hk[U];
#pragma unroll
        for (int u = 0; u < U; ++u) hk[u] = head_key(hd, g0 + u * kThreads, G);
#pragma unroll
        for (int u = 0; u < U; ++u) m = hk[u] > m ? hk[u] : m;
    }
    const uint64_t T = kth_of_maxima(S, m, k, tid);   // >= 1; k candidates are >= T
    if (tid == 0) { S.cnt = 0; S.thr = T - 1; }
    __syncthreads();

    const int kk = k < c ? k : c;
    int64_t g0 = tid;
    int u0 = 0, e0 = 0;   // resume point after a full buffer
    uint32_t vpar = 0;    // block_any's call parity
    for (;;) {
        const uint64_t thr = S.thr;
        bool stalled = false;
        for (; g0 < G; g0 += U * kThreads, u0 = 0, e0 = 0) {
            uint64_t hk[U];
#pragma unroll
            for (int u = 0; u < U; ++u) hk[u] = head_key(hd, g0 + u * kThreads, G);
#pragma unroll
            for (int u = 0; u < U; ++u) {
                if (stalled || u < u0 || hk[u] <= thr) continue;
                const int64_t base = (g0 + u * kThreads) * c;
                for (int e = (u == u0 ? e0 : 0); e < kk; ++e) {
                    const int32_t idx = ci[base + e];
                    if (idx < 0) break;
                    const uint64_t key = make_key(cv[base + e], idx);
                    if (key <= thr) break;
                    const int pos = atomicAdd(&S.cnt, 1);
                    if (pos >= kSelCap) {
                        stalled = true;
                        u0 = u;
                        e0 = e;
                        break;
                    }
                    S.buf[pos] = key;
                }
            }
            if (stalled) break;
        }
        __syncthreads();
        if (S.cnt >= kSelCap) select_compact(S, kSelCap, k, tid);
        if (!block_any<kThreads / 64>(stalled, S.vote, vpar, tid >> 6, tid & 63)) break;
    }
    const int n = S.cnt < kSelCap ? S.cnt : kSelCap;
    if (n > k) select_compact(S, n, k, tid);
    __syncthreads();
    const int mk = n < k ? n : k;
    if (tid < mk) {
        const uint64_t key = S.buf[tid];
        const int r = rank_desc<false>(S, mk, key, tid);
        a.V[row * k + r] = key_value(key);
        a.I[row * k + r] = key_index(key);
    }
}

template <int DT, int NB, int C>
static hipError_t launch_group_c(const GroupArgs& a, dim3 grid, hipStream_t st)
{
    const size_t lds = group_lds_bytes(NB);
    auto kern = group_kernel<DT, NB, C>;
    hipError_t e = ensure_lds((const void*)kern, lds);
    if (e != hipSuccess) return e;
    launch(kern, grid, dim3(kMainThreads), lds, st, a);
    return hipGetLastError();
}

template <int DT, int NB>
static hipError_t launch_group_t(const GroupArgs& a, dim3 grid, hipStream_t st)
{
    switch (a.c) {
    case 16: return launch_group_c<DT, NB, 16>(a, grid, st);
    case 32: return launch_group_c<DT, NB, 32>(a, grid, st);
    case 64: return launch_group_c<DT, NB, 64>(a, grid, st);
    case 128: return launch_group_c<DT, NB, 128>(a, grid, st);
    default: return hipErrorInvalidValue;
    }
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
