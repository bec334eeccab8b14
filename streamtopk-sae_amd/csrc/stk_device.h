// stk_device.h -- device-side building blocks for the streaming top-k encoder
// on gfx950 (CDNA4): sort keys, the MFMA quad step, the score main loop
// (TileStream: W and X staged in LDS, 8 waves, used by main_kernel and
// group_kernel) and queue compaction helpers.
//
// Score layout.  Each wavefront owns blocks of 32 latents (W rows, the MFMA
// "A" operand) and NB blocks of 32 batch rows (X rows, the MFMA "B" operand),
// and accumulates the fp32 scores W_blk . X_blk^T with
// v_mfma_f32_32x32x{16 bf16|16 f16|2 f32}.
//
// Permuted reduction axis.  One "d-step" covers 128 bytes of every W row
// (64 bf16/fp16 or 32 fp32 elements).  Lane l holds row (l % 32) of its block
// and the contiguous half h = l / 32 of the d-step: 64 bytes, fetched as four
// 16-byte loads ("quads").  The MFMA's reduction index k is paired with the
// physical d index through the same (lane-half, quad, element) map for both
// operands, so every product W[f,d]*X[j,d] is formed exactly once; only the
// order of the fp32 sum differs from a plain left-to-right dot product.
//
// Accumulator layout of v_mfma_f32_32x32x*: register r of lane l holds row
// 8*(r/4) + 4*(l/32) + (r%4), column l % 32 (every GPU parity test depends on
// it: a wrong map scores the wrong latent).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace stk {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint64_t u64x2 __attribute__((ext_vector_type(2)));

enum { DT_F32 = 0, DT_F16 = 1, DT_BF16 = 2 };

constexpr int kWaves = 4;            // wavefronts per workgroup
constexpr int kThreads = 64 * kWaves;
constexpr int kStepBytes = 128;      // bytes of one W/X row per d-step
constexpr int kXRowStride = 144;     // LDS bytes per staged X row (128 + 16 pad)

template <int DT> struct Dt;
template <> struct Dt<DT_BF16> { static constexpr int esize = 2; static constexpr int DS = 64; };
template <> struct Dt<DT_F16>  { static constexpr int esize = 2; static constexpr int DS = 64; };
template <> struct Dt<DT_F32>  { static constexpr int esize = 4; static constexpr int DS = 32; };

// ---------------------------------------------------------------------------
// 64-bit sort keys.  High word: order-preserving image of the fp32 score
// (NaN canonicalised above +inf, as torch.topk ranks NaN first).  Low word:
// 0xFFFFFFFF - latent index, so among equal scores the lower index ranks
// higher.  Key 0 never occurs for a real entry.
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint32_t ordered_u32(float v)
{
    uint32_t u = __float_as_uint(v);
    uint32_t r = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return (v != v) ? 0xFFFFFFFFu : r;
}

__device__ __forceinline__ float key_value(uint64_t key)
{
    uint32_t r = (uint32_t)(key >> 32);
    uint32_t u = (r & 0x80000000u) ? (r & 0x7FFFFFFFu) : ~r;
    return __uint_as_float(u);
}

__device__ __forceinline__ int32_t key_index(uint64_t key)
{
    return (int32_t)(0xFFFFFFFFu - (uint32_t)key);
}

__device__ __forceinline__ uint64_t make_key(float v, int64_t idx)
{
    return ((uint64_t)ordered_u32(v) << 32) | (uint64_t)(0xFFFFFFFFu - (uint32_t)idx);
}

// ---------------------------------------------------------------------------
// Threshold exchange helpers (main_kernel, mainl_kernel).  Every word the
// workgroups of one call share carries the call's tag (the workspace's epoch
// + 1, never 0) in its high half and its data in the low half, and is
// written and read whole with agent-scope atomic stores and loads (coherent
// across the XCDs' L2s word by word).  A reader polls the words it needs
// until enough carry the call's tag: no flag has to be ordered after the
// data, so no writer waits for its stores, and the last poll returns the
// data.  Words of earlier calls carry other tags; a workspace starts
// zero-filled, and tag 0 is never used.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void xch_put(uint64_t* p, uint32_t tag, uint32_t data)
{
    __hip_atomic_store(p, ((uint64_t)tag << 32) | data, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Wave-level: polls n <= 64 * U words p[0..n) (U per lane) until at least
// `need` of them carry `tag`, for at most `wait` ticks of the 100 MHz
// real-time counter; v[u] receives the low half of word lane + 64 u if it
// carries the tag, else 0.  Returns how many of the n words carry the tag in
// the last poll (>= need unless the wait ran out; the same in every lane).
// wait == 0: one poll; wait < 0: none (every v[u] 0, returns 0).
template <int U>
__device__ __forceinline__ int xch_poll(const uint64_t* p, int n, int need, uint32_t tag, int64_t wait, int lane,
                                        uint32_t (&v)[U])
{
    if (wait < 0) {
#pragma unroll
        for (int u = 0; u < U; ++u) v[u] = 0u;
        return 0;
    }
    const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
    for (;;) {
        int got = 0;
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int i = lane + 64 * u;
            bool tagged = false;
            v[u] = 0u;
            if (i < n) {
                const uint64_t w = __hip_atomic_load(p + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                tagged = (uint32_t)(w >> 32) == tag;
                v[u] = tagged ? (uint32_t)w : 0u;
            }
            got += __popcll(__ballot(tagged));
        }
        if (got >= need || (int64_t)(__builtin_amdgcn_s_memrealtime() - t0) >= wait) return got;
        __builtin_amdgcn_s_sleep(1);
    }
}

// Wave-level: a lower bound T of the k-th largest of the wave's non-zero
// values v (at least k of them), T <= T*, the exact k-th largest.  T* lies in
// [lo, hi], the smallest and largest non-zero values, so it shares their
// common leading bits; below those T is built bit by bit (the largest T with
// at least k values >= T) over 12 bits, the rest left 0: at most 2^-11 of a
// score image below T*.  The same in every lane.
template <int U>
__device__ __forceinline__ uint32_t xch_kth(const uint32_t (&v)[U], int k)
{
    uint32_t lo = ~0u, hi = 0u;
#pragma unroll
    for (int u = 0; u < U; ++u) {
        lo = (v[u] != 0u && v[u] < lo) ? v[u] : lo;
        hi = v[u] > hi ? v[u] : hi;
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const uint32_t l2 = __shfl_xor(lo, off), h2 = __shfl_xor(hi, off);
        lo = l2 < lo ? l2 : lo;
        hi = h2 > hi ? h2 : hi;
    }
    const uint32_t diff = lo ^ hi;
    if (diff == 0u) return hi;
    const int top = 31 - __builtin_clz(diff);
    uint32_t T = hi & ~((2u << top) - 1u);   // the common leading bits (2u << 31 wraps to 0: none)
    const int stop = top >= 11 ? top - 11 : 0;
    for (int bit = top; bit >= stop; --bit) {
        const uint32_t c = T | (1u << bit);
        int cnt = 0;
#pragma unroll
        for (int u = 0; u < U; ++u) cnt += __popcll(__ballot(v[u] >= c));
        T = cnt >= k ? c : T;
    }
    return T;
}

// Partial sums stored in a workspace keep no denormal (a positive one's bits
// could pass for an exchange tag in a word's high half): they are stored as
// zero, a change below any fp32 score's rounding once the bias is added.
__device__ __forceinline__ f32x4 flush_denorm4(f32x4 v)
{
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = __builtin_fabsf(v[e]) < 1.17549435e-38f ? 0.f : v[e];
    return v;
}

// The threshold key of score image T: the largest key below every key of
// that score (0, accept everything, for T = 0).
__device__ __forceinline__ uint64_t xch_key(uint32_t T)
{
    return T ? ((uint64_t)T << 32) - 1 : 0ull;
}

// Buffer resource (raw, gfx9 family): loads at byte offsets >= num_records
// return zeros, which bounds rows past B and latents past F, and a zero-length
// resource makes whole steps read as zeros.
// The streaming kernels build every resource uniform over the wave; its fields
// go through readfirstlane so that the compiler keeps it in scalar registers
// whatever its uniformity analysis concludes (a resource it takes for
// divergent costs a waterfall loop around every load).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, int64_t num_records)
{
    const uint64_t b = (uint64_t)base;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)b);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(b >> 32));
    const int n = __builtin_amdgcn_readfirstlane((int)num_records);
    return __builtin_amdgcn_make_buffer_rsrc((void*)(((uint64_t)hi << 32) | lo), (short)0, n, 0x00020000);
}

// LDS loads (global -> LDS, no registers): lane i of one instruction writes
// the 16 bytes at ldsbase + 16*i.
__device__ __forceinline__ void lds_load16(__amdgpu_buffer_rsrc_t r, unsigned char* ldsbase, int voff, int soff)
{
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)ldsbase, 16, voff, soff, 0, 0);
}

// ---------------------------------------------------------------------------
// Workgroup-wide OR of p.  Every thread of the workgroup calls it, the same
// number of times.  HIP's __syncthreads_or reads the workgroup size from the
// kernel's implicit arguments, and where registers are short the compiler
// reloads it at every call (a scalar memory load and its wait).  Here lane 0
// of each wave stores whether any lane of the wave has p into the wave's
// slot, one barrier, and every lane reads all slots.  The slots alternate
// between two sets from call to call (parity, a per-thread call counter), so a
// wave's store for the next call cannot meet a slower wave's read of this one:
// the next call's barrier lies between them.  vote: 2 * WAVES words of LDS,
// 16-byte aligned.
// ---------------------------------------------------------------------------
template <int WAVES>
__device__ __forceinline__ bool block_any(bool p, uint32_t* vote, uint32_t& parity, int wave, int lane)
{
    uint32_t* v = vote + (parity & 1u) * WAVES;
    ++parity;
    const bool wp = __ballot(p) != 0;
    if (lane == 0) v[wave] = wp ? 1u : 0u;
    __syncthreads();
    if constexpr (WAVES % 4 == 0) {
        u32x4 acc = *(const u32x4*)v;
#pragma unroll
        for (int w = 4; w < WAVES; w += 4) acc |= *(const u32x4*)(v + w);
        return (acc[0] | acc[1] | acc[2] | acc[3]) != 0u;
    } else {
        uint32_t acc = 0;
#pragma unroll
        for (int w = 0; w < WAVES; ++w) acc |= v[w];
        return acc != 0u;
    }
}

// Ring layout: row r's 16-byte chunk c sits in slot c ^ ((r >> 1) & 7) of the
// row's 128 bytes, so that the MFMA-layout reads (32 rows x one chunk per
// half-wave) hit 16 distinct 16-byte bank groups.
__device__ __forceinline__ int xswz(int r) { return (r >> 1) & 7; }

// ---------------------------------------------------------------------------
// One quad (16 bytes of W for this lane x 16 bytes of X) through the MFMA.
// ---------------------------------------------------------------------------
template <int DT>
__device__ __forceinline__ void mfma_quad(f32x16& acc, u32x4 a, u32x4 b);

template <>
__device__ __forceinline__ void mfma_quad<DT_BF16>(f32x16& acc, u32x4 a, u32x4 b)
{
    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                  __builtin_bit_cast(bf16x8, b), acc, 0, 0, 0);
}

template <>
__device__ __forceinline__ void mfma_quad<DT_F16>(f32x16& acc, u32x4 a, u32x4 b)
{
    acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                 __builtin_bit_cast(f16x8, b), acc, 0, 0, 0);
}

template <>
__device__ __forceinline__ void mfma_quad<DT_F32>(f32x16& acc, u32x4 a, u32x4 b)
{
#pragma unroll
    for (int e = 0; e < 4; ++e)
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(a[e]), __uint_as_float(b[e]), acc, 0, 0, 0);
}

// ---------------------------------------------------------------------------
// Compacts the queue segments (in global memory) of this wave's rows that are
// full to their top-k: rows wave*R .. wave*R + R - 1 (R <= 64), segment of
// row r at qrow(r), cap keys; cnt and thr in LDS.  Segment keys are read
// through L2 (agent-scope atomic loads): other waves' plain stores are
// complete (fence + barrier before the call) but the reading CU's L1 may hold
// lines of an earlier compaction.  scr: cap keys of LDS for this wave.
// ---------------------------------------------------------------------------
template <int R, class RowSeg>
__device__ __forceinline__ void compact_full_rows(int* cnt, uint64_t* thr, uint64_t* scr, RowSeg qrow,
                                                  int cap, int k, int wave, int lane)
{
    const int myrow = wave * R + (lane < R ? lane : 0);
    uint64_t full = __ballot(lane < R && cnt[myrow] >= cap);
    while (full) {
        const int i = __builtin_ctzll(full);
        full &= full - 1;
        const int row = wave * R + i;
        auto* q = qrow(row);
        uint64_t e[3];
#pragma unroll
        for (int m = 0; m < 3; ++m) {
            const int idx = lane + 64 * m;
            e[m] = (idx < cap) ? __hip_atomic_load(q + idx, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0ull;
            if (idx < cap) scr[idx] = e[m];
        }
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        int rk[3] = {0, 0, 0};
        for (int ii = 0; ii < cap; ii += 2) {
            const u64x2 v = *(const u64x2*)(scr + ii);
#pragma unroll
            for (int m = 0; m < 3; ++m) rk[m] += (int)(v[0] > e[m]) + (int)(v[1] > e[m]);
        }
#pragma unroll
        for (int m = 0; m < 3; ++m) {
            if (lane + 64 * m < cap && rk[m] < k) {
                q[rk[m]] = e[m];
                if (rk[m] == k - 1) thr[row] = e[m];
            }
        }
        if (lane == 0) cnt[row] = k;
        __builtin_amdgcn_wave_barrier();
    }
}

// Rank-compacts the n keys q[0..n) (k < n <= cap <= 192, distinct, written
// by this wave or read back through L2) to their k largest, in q[0..k), and
// returns the k-th largest.  One wave; scr is cap keys of LDS scratch.
__device__ __forceinline__ uint64_t compact_row(uint64_t* q, int n, uint64_t* scr, int cap, int k, int lane)
{
    uint64_t e[3];
#pragma unroll
    for (int m = 0; m < 3; ++m) {
        const int idx = lane + 64 * m;
        e[m] = (idx < n) ? __hip_atomic_load(q + idx, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0ull;
        if (idx < cap) scr[idx] = e[m];
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    // ranks among the n keys (the zero padding up to n rounded to even ranks below every key)
    int rk[3] = {0, 0, 0};
    for (int ii = 0; ii < n; ii += 2) {
        const u64x2 v = *(const u64x2*)(scr + ii);
#pragma unroll
        for (int m = 0; m < 3; ++m) rk[m] += (int)(v[0] > e[m]) + (int)(v[1] > e[m]);
    }
    uint64_t kth = 0;
#pragma unroll
    for (int m = 0; m < 3; ++m) {
        if (lane + 64 * m < n && rk[m] < k) {
            q[rk[m]] = e[m];
            if (rk[m] == k - 1) kth = e[m];
        }
    }
    // exactly one lane holds the k-th key
    const uint64_t hit = __ballot(kth != 0);
    const int src = __builtin_ctzll(hit);
    const uint32_t lo = __builtin_amdgcn_readlane((uint32_t)kth, src);
    const uint32_t hi = __builtin_amdgcn_readlane((uint32_t)(kth >> 32), src);
    __builtin_amdgcn_wave_barrier();
    return ((uint64_t)hi << 32) | lo;
}

// ---------------------------------------------------------------------------
// TileStream: the score main loop with both operands staged in LDS.  A tile
// is 32*WAVES latents x 32*NB rows and takes nds2 d-steps: the nds real ones
// rounded up to even (a padding step loads a valid step again and skips its
// MFMAs).
//   W: each d-step's kTileF rows x 128 bytes are read with whole-line
//      nontemporal loads (W is read once: no cache allocation), eight lanes
//      per row step, two steps ahead in registers, and stored to a two-buffer
//      LDS ring; each wave then reads its 32 rows in the MFMA layout.  Loads
//      straight into the MFMA layout touch 32 rows per instruction, 32 bytes
//      of each line, and stream W at ~6 TB/s; whole-line nontemporal loads
//      reach ~7 TB/s.
//   X: the row block's 32*NB rows of the step, the same way with ordinary
//      loads (every workgroup of the row block re-reads X from L2).
// One barrier per d-step.  The loads of the next tile's first steps are in
// flight across the epilogue.  Every load is unconditional (rows past F or B
// and steps past the end are clamped to valid addresses; the scores they
// produce are never selected).
//
// run() calls epi(t, acc, bias) after the last d-step of tile t and then
// resets acc and waits for every outstanding memory operation: the epilogue
// may issue a data-dependent number of global stores, which the compiler
// cannot count, and the wait restores its exact counts for the d-step loop
// (the prefetched loads it includes have had the whole epilogue to land).
// The epilogue may use LDS other than ring buffer 0 (which holds the next
// tile's first step) and the bias buffers.  Ring buffer 1 (W and X) is idle
// during it: its last readers passed the tile's last barrier and its next
// writer runs after the epilogue, so an epilogue that uses it must end with a
// workgroup barrier.  The bias of tile t comes from LDS: wave 0 loads the next
// tile's bias inside the d-step loop and stores it within the same iteration.
// With kBiasInit the accumulators of each tile start at the bias of their
// latents (so acc holds the scores, bias included, when epi runs: the MFMAs
// add the products onto it); otherwise they start at zero and epi receives
// the bias to add.
// ---------------------------------------------------------------------------
template <int DT, int NB, int WAVES>
struct TileStream {
    static constexpr int DS = Dt<DT>::DS;
    static constexpr int ES = Dt<DT>::esize;
    static constexpr int kThr = 64 * WAVES;
    static constexpr int kTileF = 32 * WAVES;                      // latents per tile
    static constexpr int kWChunks = kTileF * 8 / kThr;             // 16-byte W chunks per thread per step
    static constexpr int kXTotal = 32 * NB * 8;                    // 16-byte X chunks per step
    static constexpr int kXChunks = (kXTotal + kThr - 1) / kThr;   // per thread
    static constexpr int kWBuf = kTileF * kXRowStride;             // bytes of one W ring buffer
    static constexpr int kXBuf = 32 * NB * kXRowStride;            // bytes of one X ring buffer
    static constexpr int kRingBytes = 2 * kWBuf + 2 * kXBuf;
    static_assert(kXTotal % kThr == 0 || kXChunks == 1, "X chunk split");
    static_assert(kTileF * 8 % kThr == 0, "W chunk split");

    static constexpr int kQE = 16 / ES;                            // elements per 16-byte chunk

    const float* bias;
    int64_t F;
    int64_t tile_begin;
    int ntiles, nds, nds2;
    int tail;                    // elements of d in the last d-step when it is partial, else 0
    int tid, lane, wave, h, jl;
    const unsigned char* W;
    int64_t w_row_bytes;

    // load cursor (uniform) and this thread's chunk pointers in the cursor's tile
    int lt, ls;
    const unsigned char* lw[kWChunks];
    const unsigned char* lx[kXChunks];
    bool xok[kXChunks];

    __device__ __forceinline__ void init_x(const unsigned char* X, int64_t B, int64_t b0, int64_t d)
    {
#pragma unroll
        for (int p = 0; p < kXChunks; ++p) {
            const int c = tid + kThr * p;
            const int row = (c >> 3) % (32 * NB), c16 = c & 7;
            int64_t r = b0 + row;
            r = (r < B) ? r : B - 1;
            lx[p] = X + (r * d) * ES + c16 * 16;
            xok[p] = c < kXTotal;
        }
    }

    __device__ __forceinline__ void set_rows(int t)
    {
        const int64_t tile = tile_begin + (t < ntiles ? t : ntiles - 1);
#pragma unroll
        for (int p = 0; p < kWChunks; ++p) {
            const int c = tid + kThr * p;
            int64_t f = tile * kTileF + (c >> 3);
            f = (f < F) ? f : F - 1;
            lw[p] = W + f * w_row_bytes + (c & 7) * 16;
        }
    }

    __device__ __forceinline__ void issue(u32x4 (&xr)[kXChunks], u32x4 (&wr)[kWChunks])
    {
        const int s = (lt >= ntiles || ls >= nds) ? nds - 1 : ls;
        const int64_t so = (int64_t)s * kStepBytes;
        if (tail != 0 && s == nds - 1) {
            // partial last step: a chunk past d reads the step's first chunk
            // (in bounds: the step starts below d) and is zeroed
#pragma unroll
            for (int p = 0; p < kXChunks; ++p) {
                const int c8 = (tid + kThr * p) & 7;
                const bool ok = c8 * kQE < tail;
                const u32x4 v = *(const u32x4*)(lx[p] + so - (ok ? 0 : c8 * 16));
                xr[p] = ok ? v : u32x4{0u, 0u, 0u, 0u};
            }
#pragma unroll
            for (int p = 0; p < kWChunks; ++p) {
                const int c8 = (tid + kThr * p) & 7;
                const bool ok = c8 * kQE < tail;
                const u32x4 v = __builtin_nontemporal_load((const u32x4*)(lw[p] + so - (ok ? 0 : c8 * 16)));
                wr[p] = ok ? v : u32x4{0u, 0u, 0u, 0u};
            }
        } else {
#pragma unroll
            for (int p = 0; p < kXChunks; ++p) xr[p] = *(const u32x4*)(lx[p] + so);
#pragma unroll
            for (int p = 0; p < kWChunks; ++p) wr[p] = __builtin_nontemporal_load((const u32x4*)(lw[p] + so));
        }
        if (lt < ntiles && ++ls == nds2) {
            ls = 0;
            ++lt;
            if (lt < ntiles) set_rows(lt);
        }
    }

    __device__ __forceinline__ void store(const u32x4 (&xr)[kXChunks], const u32x4 (&wr)[kWChunks],
                                          unsigned char* xs, unsigned char* wsb) const
    {
#pragma unroll
        for (int p = 0; p < kWChunks; ++p) {
            const int c = tid + kThr * p;
            *(u32x4*)(wsb + (c >> 3) * kXRowStride + (c & 7) * 16) = wr[p];
        }
#pragma unroll
        for (int p = 0; p < kXChunks; ++p) {
            const int c = tid + kThr * p;
            if (kXTotal % kThr == 0 || xok[p]) *(u32x4*)(xs + (c >> 3) * kXRowStride + (c & 7) * 16) = xr[p];
        }
    }

    __device__ __forceinline__ void compute(f32x16 (&acc)[NB], const unsigned char* xs, const unsigned char* wsb) const
    {
        u32x4 w[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) w[q] = *(const u32x4*)(wsb + (wave * 32 + jl) * kXRowStride + h * 64 + q * 16);
        // two 32-row blocks at a time: two independent accumulation chains
        constexpr int NP = NB < 2 ? NB : 2;
#pragma unroll
        for (int n0 = 0; n0 < NB; n0 += NP) {
            u32x4 bx[NP][4];
#pragma unroll
            for (int n = 0; n < NP; ++n)
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    bx[n][q] = *(const u32x4*)(xs + (32 * (n0 + n) + jl) * kXRowStride + h * 64 + q * 16);
#pragma unroll
            for (int q = 0; q < 4; ++q)
#pragma unroll
                for (int n = 0; n < NP; ++n) mfma_quad<DT>(acc[n0 + n], w[q], bx[n][q]);
        }
    }

    __device__ __forceinline__ void bias_load(float (&bn)[kTileF / 64], int t) const
    {
        const int64_t f0 = (tile_begin + t) * kTileF + lane * (kTileF / 64);
#pragma unroll
        for (int e = 0; e < kTileF / 64; ++e) {
            const int64_t f = f0 + e;
            bn[e] = bias[(f < F) ? f : F - 1];
        }
    }

    __device__ __forceinline__ void bias_store(const float (&bn)[kTileF / 64], float* buf) const
    {
#pragma unroll
        for (int e = 0; e < kTileF / 64; ++e) buf[lane * (kTileF / 64) + e] = bn[e];
    }

    // Bias of this lane's latents: entry r is latent (within the tile)
    // wave*32 + 8*(r/4) + 4*h + r%4.
    __device__ __forceinline__ void bias_read(float (&bv)[16], const float* buf) const
    {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const f32x4 v = *(const f32x4*)(buf + wave * 32 + g * 8 + h * 4);
#pragma unroll
            for (int e = 0; e < 4; ++e) bv[4 * g + e] = v[e];
        }
    }

    __device__ __forceinline__ void acc_reset(f32x16 (&acc)[NB], const float* bias_buf, bool from_bias) const
    {
        if (from_bias) {
            float bv[16];
            bias_read(bv, bias_buf);
#pragma unroll
            for (int n = 0; n < NB; ++n)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[n][r] = bv[r];
        } else {
#pragma unroll
            for (int n = 0; n < NB; ++n)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[n][r] = 0.f;
        }
    }

    template <bool kBiasInit, class Epi>
    __device__ __forceinline__ void run(f32x16 (&acc)[NB], unsigned char* ring, float* bias_lds, Epi epi)
    {
        if (ntiles <= 0) return;
        unsigned char* ws0 = ring;
        unsigned char* ws1 = ring + kWBuf;
        unsigned char* xs0 = ring + 2 * kWBuf;
        unsigned char* xs1 = ring + 2 * kWBuf + kXBuf;
        lt = 0;
        ls = 0;
        set_rows(0);
        u32x4 w0[kWChunks], w1[kWChunks];
        u32x4 x0[kXChunks], x1[kXChunks];
        // the first two steps' loads go out first; wave 0's bias loads after
        // them, so that neither waits for the other's round trip
        issue(x0, w0);
        issue(x1, w1);
        float bn0[kTileF / 64];
        if (wave == 0) bias_load(bn0, 0);
        store(x0, w0, xs0, ws0);
        if (wave == 0) bias_store(bn0, bias_lds);
        issue(x0, w0);
        __syncthreads();
        acc_reset(acc, bias_lds, kBiasInit);
        for (int t = 0; t < ntiles; ++t) {
            float* bnext = bias_lds + ((t + 1) & 1) * kTileF;
            for (int s = 0; s < nds2; s += 2) {
                float bn[kTileF / 64];
                if (wave == 0) bias_load(bn, t + 1);   // past the last tile: clamped, unused
                if (s < nds) compute(acc, xs0, ws0);
                store(x1, w1, xs1, ws1);
                issue(x1, w1);
                __syncthreads();
                if (s + 1 < nds) compute(acc, xs1, ws1);
                store(x0, w0, xs0, ws0);
                issue(x0, w0);
                if (wave == 0) bias_store(bn, bnext);
                __syncthreads();
            }
            float bv[16];
            if (!kBiasInit) bias_read(bv, bias_lds + (t & 1) * kTileF);
            epi(t, acc, bv);
            acc_reset(acc, bias_lds + ((t + 1) & 1) * kTileF, kBiasInit);   // past the last tile: unused
            __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0)
        }
    }
};

}  // namespace stk
