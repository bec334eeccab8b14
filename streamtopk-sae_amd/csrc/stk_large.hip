// stk_large.hip -- the streaming kernel for large batches (compute-bound).
//
// mainl_kernel: one workgroup of 4 waves (one per SIMD, up to 512 registers
// each) owns 256 rows and a contiguous range of 256-latent tiles.  Each wave
// scores 64 latents x 256 rows per tile: 2 x 8 blocks of
// v_mfma_f32_32x32x16 with the 256 accumulators per lane in AGPRs, so every W
// byte fetched feeds 256 rows and every staged X byte feeds 256 latents.
//   - W: straight from global memory into registers, 2 d-steps ahead; each
//     16-byte quad is reloaded as soon as its last MFMA of the step issued.
//     The pipeline restarts at every tile, so the epilogue holds no prefetch.
//   - X: 256 rows x 128 bytes per d-step, 2 d-steps ahead in registers, then
//     through a 2-buffer LDS ring (one barrier per d-step).
//   - bias: the tile's 256 values are loaded at the tile start and staged in
//     LDS for the epilogue.
//   - epilogue: scores not below the row threshold are appended to the row's
//     queue segment in global memory (counters in LDS).  A full segment is
//     rank-compacted to its top-k, which raises the row threshold.
//   - grid: workgroups are placed so that the row blocks sharing a W range
//     run on one XCD (workgroup i runs on XCD i % 8), and W is fetched into
//     that XCD's L2 once for all of them.
// mainl_kernel<DT, true> (sample mode) computes the raw scores of the
// sampled latents with the same machinery: one 256-latent tile of them per
// workgroup and a d range per workgroup, partial sums summed in a fixed order
// by thr_kernel.
// The reference has no counterpart: its B >= #SMs path streams all of W per
// row (streamtopk_exact.cu:506-638).
#include "stk_kernels.h"

namespace stk {

namespace {

constexpr int kLWaves = 4;
constexpr int kLNB = 8;                      // 32-row blocks per workgroup
constexpr int kLFrags = 2;                   // 32-latent fragments per wave
constexpr int kLTile = 32 * kLFrags * kLWaves;   // 256 latents per tile
constexpr int kLXChunks = kLargeRows * 8 / kLargeThreads;   // 16-byte X chunks per thread per d-step

// Buffer resource (raw, gfx9 family): loads at byte offsets >= num_records
// return zeros, which bounds rows past B and latents past F, and a zero-length
// resource makes whole steps read as zeros.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, int64_t num_records)
{
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)num_records, 0x00020000);
}

template <int DT, bool SAMPLE>
struct BigStream {
    const unsigned char* W;
    int64_t row_bytes;           // bytes of a W row and of an X row (d elements)
    const unsigned char* X;
    int64_t B, b0, F;
    int64_t tile_begin;
    int ntiles, nds, nds2;
    int s_lo, s_hi;              // d-steps [s_lo, s_hi) of every tile
    int samp_log2;               // SAMPLE: tile t covers sampled latents t*256 ..
    int tid, lane, wave, h, jl;

    // W and X cursors (tile, step), uniform; a tile's pipeline ends at the tile
    int wt, ws, xt, xsn;
    __amdgpu_buffer_rsrc_t wres, xres, zres;
    int wvoff[kLFrags];          // row of this lane's latent within the tile, + lane half
    int xvoff[kLXChunks];        // row of this thread's X chunk within the row block

    __device__ __forceinline__ void init()
    {
        // encode: offsets within the tile; sample: within this wave's 64-latent
        // run of a sampled block (its own resource base)
        const int wbase = SAMPLE ? 0 : wave * (32 * kLFrags);
#pragma unroll
        for (int a = 0; a < kLFrags; ++a)
            wvoff[a] = (wbase + a * 32 + jl) * (int)row_bytes + h * 64;
#pragma unroll
        for (int p = 0; p < kLXChunks; ++p) xvoff[p] = ((tid >> 3) + 32 * p) * (int)row_bytes + (tid & 7) * 16;
        const int64_t nrows = (B - b0 < kLargeRows) ? B - b0 : kLargeRows;
        xres = make_rsrc(X + b0 * row_bytes, nrows * row_bytes);
        zres = make_rsrc(X, 0);
    }

    __device__ __forceinline__ void begin_tile(int t)
    {
        wt = xt = t;
        ws = xsn = s_lo;
        set_w_tile(t);
    }

    __device__ __forceinline__ void set_w_tile(int t)
    {
        const int64_t tile0 = (tile_begin + t) * kLTile;
        if (SAMPLE) {
            // the wave's 64 sampled latents are consecutive latents of one block
            const int64_t f0 = sample_latent(tile0 + wave * (32 * kLFrags), samp_log2);
            wres = make_rsrc(W + f0 * row_bytes, (int64_t)(32 * kLFrags) * row_bytes);
        } else {
            int64_t n = F - tile0;
            n = n < kLTile ? (n > 0 ? n : 0) : kLTile;
            wres = make_rsrc(W + tile0 * row_bytes, n * row_bytes);
        }
    }

    // Resource and step offset of the W cursor's step; advances the cursor.
    __device__ __forceinline__ void next_w(__amdgpu_buffer_rsrc_t& r, int& so)
    {
        const bool live = wt < ntiles && ws < s_hi;
        r = live ? wres : zres;
        so = live ? ws * kStepBytes : 0;
        ++ws;
    }

    __device__ __forceinline__ void load_wq(u32x4 (&w)[kLFrags][4], int q, __amdgpu_buffer_rsrc_t r, int so) const
    {
#pragma unroll
        for (int a = 0; a < kLFrags; ++a) w[a][q] = __builtin_amdgcn_raw_buffer_load_b128(r, wvoff[a] + q * 16, so, 0);
    }

    __device__ __forceinline__ void issue_w(u32x4 (&w)[kLFrags][4])
    {
        __amdgpu_buffer_rsrc_t r;
        int so;
        next_w(r, so);
#pragma unroll
        for (int q = 0; q < 4; ++q) load_wq(w, q, r, so);
    }

    __device__ __forceinline__ void issue_x(u32x4 (&x)[kLXChunks])
    {
        const bool live = xt < ntiles && xsn < s_hi;
        const __amdgpu_buffer_rsrc_t r = live ? xres : zres;
        const int so = live ? xsn * kStepBytes : 0;
#pragma unroll
        for (int p = 0; p < kLXChunks; ++p) x[p] = __builtin_amdgcn_raw_buffer_load_b128(r, xvoff[p], so, 0);
        ++xsn;
    }

    __device__ __forceinline__ void store_x(const u32x4 (&x)[kLXChunks], unsigned char* xs) const
    {
#pragma unroll
        for (int p = 0; p < kLXChunks; ++p)
            *(u32x4*)(xs + ((tid >> 3) + 32 * p) * kXRowStride + (tid & 7) * 16) = x[p];
    }

    // One d-step.  The X operands of all 8 row blocks for quad q + 1 are read
    // from LDS while the 16 MFMAs of quad q run; after them, quad q of this
    // wave's W is reloaded with the step two ahead (its last use has issued).
    // One d-step on LDS buffer `xs`.  Each quad interleaves its 16 MFMAs with
    // the 8 LDS reads of the next quad and the reloads of its own W registers,
    // so those issue while an MFMA executes: the MFMAs of fragment 0 come
    // first (reads interleaved), then fragment 1, with fragment 0's W reload
    // issued among them.
    __device__ __forceinline__ void step(f32x16 (&acc)[kLFrags][kLNB], u32x4 (&w)[kLFrags][4],
                                         const unsigned char* xs)
    {
        __amdgpu_buffer_rsrc_t r;
        int so;
        next_w(r, so);
        const unsigned char* xl = xs + jl * kXRowStride + h * 64;
        u32x4 bA[kLNB], bB[kLNB];
#pragma unroll
        for (int n = 0; n < kLNB; ++n) bA[n] = *(const u32x4*)(xl + (32 * n) * kXRowStride);
        __builtin_amdgcn_sched_barrier(0);   // quad 0's operands are all in flight before any MFMA
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            u32x4 (&cur)[kLNB] = (q & 1) ? bB : bA;
            u32x4 (&nxt)[kLNB] = (q & 1) ? bA : bB;
            if (q < 3) {
#pragma unroll
                for (int n = 0; n < kLNB; ++n) nxt[n] = *(const u32x4*)(xl + (32 * n) * kXRowStride + (q + 1) * 16);
            }
#pragma unroll
            for (int n = 0; n < kLNB; ++n) mfma_quad<DT>(acc[0][n], w[0][q], cur[n]);
            w[0][q] = __builtin_amdgcn_raw_buffer_load_b128(r, wvoff[0] + q * 16, so, 0);
#pragma unroll
            for (int n = 0; n < kLNB; ++n) mfma_quad<DT>(acc[1][n], w[1][q], cur[n]);
            w[1][q] = __builtin_amdgcn_raw_buffer_load_b128(r, wvoff[1] + q * 16, so, 0);
            // pattern: (MFMA, DS read) x 8, (MFMA, VMEM read), MFMA x 7, then the last VMEM
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // MFMA
                if (q < 3) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);   // DS read
            }
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);   // VMEM read
            __builtin_amdgcn_sched_group_barrier(0x008, 7, 0);
            __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
};

// An accumulator element read into a VGPR at the point of use.  Volatile, so
// the compiler cannot keep VGPR copies of all 256 accumulators alive across
// the epilogue's passes (which spills).
__device__ __forceinline__ float agpr_read(float x)
{
    float r;
    asm volatile("v_accvgpr_read_b32 %0, %1" : "=v"(r) : "a"(x));
    return r;
}

}  // namespace

size_t mainl_lds_bytes(int cap)
{
    return 2 * (size_t)kLargeRows * kXRowStride + kLTile * sizeof(float) + kLargeRows * 8 + kLargeRows * 4 +
           (size_t)kLWaves * cap * 8 + (size_t)kLargeRows * sizeof(uint64_t*);
}

template <int DT, bool SAMPLE>
__global__ __launch_bounds__(kLargeThreads, 1) void mainl_kernel(MainLArgs a)
{
    extern __shared__ __align__(16) unsigned char smem[];
    unsigned char* xs0 = smem;
    unsigned char* xs1 = smem + kLargeRows * kXRowStride;
    float* bias_s = (float*)(smem + 2 * kLargeRows * kXRowStride);   // [kLTile]
    uint64_t* thr = (uint64_t*)(bias_s + kLTile);                    // [rows]
    int* cnt = (int*)(thr + kLargeRows);                              // [rows]
    uint64_t** qrow = (uint64_t**)(cnt + kLargeRows);                 // [rows] segment of each row
    uint64_t* cscr = (uint64_t*)(qrow + kLargeRows);                  // [waves][cap]
    const int cap = a.cap, k = a.k;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int h = lane >> 5, jl = lane & 31;

    // workgroup -> (row block, W range): the row blocks of a W range share an XCD.
    // Sample mode: workgroup -> (row block, sample tile, d range).
    int rb, rg, ks = 0;
    {
        const int id = blockIdx.x;
        if (SAMPLE) {
            rb = id % a.nbc;
            const int stiles = a.nsamp / kLTile;
            rg = (id / a.nbc) % stiles;
            ks = id / (a.nbc * stiles);
        } else if ((a.nr & 7) == 0) {
            const int slot = id >> 3;
            rb = slot % a.nbc;
            rg = (slot / a.nbc) * 8 + (id & 7);
        } else {
            rb = id % a.nbc;
            rg = id / a.nbc;
        }
    }
    const int64_t b0 = (int64_t)rb * kLargeRows;
    const int64_t B = a.B, F = a.F;

    if (!SAMPLE) {
        for (int i = tid; i < kLargeRows; i += kLargeThreads) {
            const int64_t row = b0 + i;
            cnt[i] = 0;
            thr[i] = (row < B) ? a.thr0[row] : 0ull;
            qrow[i] = a.list_keys + ((row < B) ? row : 0) * a.list_cap + a.head_span + (int64_t)rg * cap;
        }
    }

    BigStream<DT, SAMPLE> bs;
    bs.W = (const unsigned char*)a.W;
    bs.row_bytes = a.d * Dt<DT>::esize;
    bs.X = (const unsigned char*)a.X;
    bs.B = B;
    bs.b0 = b0;
    bs.F = F;
    bs.nds = (int)(a.d / Dt<DT>::DS);
    bs.samp_log2 = a.samp_log2;
    if (SAMPLE) {
        bs.tile_begin = rg;
        bs.ntiles = 1;
        bs.s_lo = (int)((int64_t)ks * bs.nds / a.ksplit);
        bs.s_hi = (int)((int64_t)(ks + 1) * bs.nds / a.ksplit);
    } else {
        bs.tile_begin = (int64_t)rg * a.tiles_per_wg;
        const int64_t t1 = bs.tile_begin + a.tiles_per_wg;
        const int64_t nt = (t1 < a.num_tiles ? t1 : a.num_tiles) - bs.tile_begin;
        bs.ntiles = nt > 0 ? (int)nt : 0;
        bs.s_lo = 0;
        bs.s_hi = bs.nds;
    }
    bs.nds2 = (bs.s_hi - bs.s_lo + 1) / 2 * 2;
    bs.tid = tid;
    bs.lane = lane;
    bs.wave = wave;
    bs.h = h;
    bs.jl = jl;

    if (bs.ntiles > 0) {
        bs.init();
        u32x4 wA[kLFrags][4], wB[kLFrags][4];
        u32x4 xA[kLXChunks], xB[kLXChunks];

        f32x16 acc[kLFrags][kLNB];
#pragma unroll
        for (int fa = 0; fa < kLFrags; ++fa)
#pragma unroll
            for (int n = 0; n < kLNB; ++n)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[fa][n][r] = 0.f;

        for (int t = 0; t < bs.ntiles; ++t) {
            const int64_t tile0 = (bs.tile_begin + t) * kLTile;
            // The pipeline is restarted per tile so that no prefetch registers are
            // live in the epilogue (one exposed load latency per tile of nds steps).
            float bnext = 0.f;
            if (!SAMPLE) {
                const int64_t f = tile0 + tid;
                bnext = a.bias[f < F ? f : F - 1];
            }
            bs.begin_tile(t);
            bs.issue_w(wA);
            bs.issue_w(wB);
            bs.issue_x(xA);
            bs.issue_x(xB);
            bs.store_x(xA, xs0);
            bs.issue_x(xA);
            __syncthreads();
            // a padded last step (s >= nds) reads zeros: every step computes unconditionally
            for (int s = 0; s < bs.nds2; s += 2) {
                bs.step(acc, wA, xs0);
                bs.store_x(xB, xs1);
                bs.issue_x(xB);
                __syncthreads();
                bs.step(acc, wB, xs1);
                bs.store_x(xA, xs0);
                bs.issue_x(xA);
                __syncthreads();
            }
            if (SAMPLE) {
                // raw partial scores of this d range: P[ks][row][sample index]
                float* P = a.P + (int64_t)ks * B * a.nsamp;
#pragma unroll
                for (int n = 0; n < kLNB; ++n) {
                    const int64_t row = b0 + 32 * n + jl;
                    if (row < B) {
#pragma unroll
                        for (int fa = 0; fa < kLFrags; ++fa)
#pragma unroll
                            for (int r4 = 0; r4 < 4; ++r4) {
                                const int64_t i = tile0 + wave * 64 + fa * 32 + r4 * 8 + h * 4;
                                f32x4 v;
#pragma unroll
                                for (int e = 0; e < 4; ++e) v[e] = acc[fa][n][r4 * 4 + e];
                                *(f32x4*)(P + row * a.nsamp + i) = v;
                            }
                    }
                }
                continue;
            }
            bias_s[tid] = bnext;
            __syncthreads();

            // ---- epilogue: bias, threshold filter, append to the row segments ----
            uint32_t vmask[kLFrags];
            {
                const bool edge = tile0 + kLTile > F ||
                                  (a.sampled && (is_sampled(tile0, a.samp_log2, a.samp_blocks) ||
                                                 is_sampled(tile0 + kLTile - 1, a.samp_log2, a.samp_blocks)));
#pragma unroll
                for (int fa = 0; fa < kLFrags; ++fa) {
                    uint32_t m = 0xFFFFu;
                    if (edge) {
                        m = 0;
                        const int64_t fl = tile0 + wave * 64 + fa * 32 + h * 4;
#pragma unroll
                        for (int r = 0; r < 16; ++r) {
                            const int64_t f = fl + (r >> 2) * 8 + (r & 3);
                            const bool ok = f < F && !(a.sampled && is_sampled(f, a.samp_log2, a.samp_blocks));
                            m |= ok ? (1u << r) : 0u;
                        }
                    }
                    vmask[fa] = m;
                }
            }
            // Scores are read from the accumulators (AGPRs) at each use and the
            // bias of this lane's 32 latents is held in VGPRs; the prefetch
            // registers are dead here.
            // Latent of bit 16*fa + r of a row mask: lat0 + fa*32 + 8*(r/4) + r%4.
            const int lat0 = (int)tile0 + wave * 64 + h * 4;
            float bl[kLFrags * 16];
#pragma unroll
            for (int fa = 0; fa < kLFrags; ++fa)
#pragma unroll
                for (int r = 0; r < 16; ++r) bl[fa * 16 + r] = bias_s[wave * 64 + h * 4 + fa * 32 + (r >> 2) * 8 + (r & 3)];
            uint32_t pend[kLNB];
#pragma unroll
            for (int n = 0; n < kLNB; ++n) {
                const int j = 32 * n + jl;
                const uint64_t tk = thr[j];
                const float tv = tk ? key_value(tk) : -__builtin_inff();
                uint32_t m = 0;
#pragma unroll
                for (int fa = 0; fa < kLFrags; ++fa)
#pragma unroll
                    for (int r = 0; r < 16; ++r)
                        m |= (!(agpr_read(acc[fa][n][r]) + bl[fa * 16 + r] < tv)) ? (1u << (16 * fa + r)) : 0u;
                m &= vmask[0] | (vmask[1] << 16);
                pend[n] = (b0 + j < B) ? m : 0u;
            }
            for (int it = 0; it < 1 << 20; ++it) {
                bool overflow = false;
                // reserve the slots of every row block first, then wait once
                int base[kLNB];
#pragma unroll
                for (int n = 0; n < kLNB; ++n)
                    base[n] = pend[n] ? atomicAdd(&cnt[32 * n + jl], __builtin_popcount(pend[n])) : 0;
                __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0)
                // Per row block: the 32 biased scores of every lane go to this
                // wave's LDS staging area (the X buffers are idle here), then each
                // lane walks only its own set bits and reads each score back by
                // address: max-popcount iterations instead of 32 divergent blocks.
                float* stage = (float*)xs0 + wave * (kLFrags * 16 * 64);
#pragma unroll
                for (int n = 0; n < kLNB; ++n) {
                    const uint32_t m = pend[n];
                    if (__ballot(m != 0) == 0) continue;
#pragma unroll
                    for (int fa = 0; fa < kLFrags; ++fa)
#pragma unroll
                        for (int r = 0; r < 16; ++r)
                            stage[(fa * 16 + r) * 64 + lane] = agpr_read(acc[fa][n][r]) + bl[fa * 16 + r];
                    uint64_t* q = qrow[32 * n + jl];
                    uint32_t keep = 0, mm = m;
                    int slot = base[n];
                    while (mm) {
                        const int bit = __builtin_ctz(mm);
                        mm &= mm - 1u;
                        if (slot < cap) {
                            const int off = (bit >> 4) * 32 + ((bit & 15) >> 2) * 8 + (bit & 3);
                            q[slot] = make_key(stage[bit * 64 + lane], lat0 + off);
                        } else {
                            keep |= 1u << bit;
                        }
                        ++slot;
                    }
                    pend[n] = keep;
                    overflow |= keep != 0;
                }
                if (!__syncthreads_or(overflow)) break;
                __threadfence_block();   // this thread's segment stores are complete
                __syncthreads();
                compact_full_rows<kLargeRows / kLWaves>(cnt, thr, cscr + wave * cap,
                                                       [&](int r) { return qrow[r]; }, cap, k, wave, lane);
                __threadfence_block();
                __syncthreads();
#pragma unroll
                for (int n = 0; n < kLNB; ++n) {
                    if (pend[n] == 0) continue;
                    const uint64_t tk = thr[32 * n + jl];
#pragma unroll
                    for (int fa = 0; fa < kLFrags; ++fa)
#pragma unroll
                        for (int r = 0; r < 16; ++r) {
                            const int bit = 16 * fa + r;
                            const int off = fa * 32 + (r >> 2) * 8 + (r & 3);
                            if ((pend[n] >> bit & 1u) &&
                                !(make_key(agpr_read(acc[fa][n][r]) + bl[fa * 16 + r], lat0 + off) > tk))
                                pend[n] &= ~(1u << bit);
                        }
                }
            }
#pragma unroll
            for (int fa = 0; fa < kLFrags; ++fa)
#pragma unroll
                for (int n = 0; n < kLNB; ++n)
#pragma unroll
                    for (int r = 0; r < 16; ++r) acc[fa][n][r] = 0.f;
            // The epilogue issued a data-dependent number of queue stores, which
            // the compiler cannot count; waiting for them here lets it keep
            // exact vmcnt waits in the next tile's d-step loop.
            __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0)
        }
    }

    if (SAMPLE) return;
    __syncthreads();
    for (int i = tid; i < kLargeRows; i += kLargeThreads) {
        const int64_t row = b0 + i;
        if (row < B) a.seg_cnt[row * a.nr + rg] = cnt[i] < cap ? cnt[i] : cap;
    }
}

template <int DT, bool SAMPLE>
static hipError_t launch_mainl_t(const MainLArgs& a, int grid, hipStream_t st)
{
    const size_t lds = mainl_lds_bytes(a.cap);
    auto kern = mainl_kernel<DT, SAMPLE>;
    hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
    launch(kern, dim3((unsigned)grid), dim3(kLargeThreads), lds, st, a);
    return hipGetLastError();
}

hipError_t launch_mainl(int dt, const MainLArgs& a, int grid, hipStream_t st)
{
    if (dt == DT_BF16) return launch_mainl_t<DT_BF16, false>(a, grid, st);
    if (dt == DT_F16) return launch_mainl_t<DT_F16, false>(a, grid, st);
    if (dt == DT_F32) return launch_mainl_t<DT_F32, false>(a, grid, st);
    return hipErrorInvalidValue;
}

hipError_t launch_mainl_sample(int dt, const MainLArgs& a, int grid, hipStream_t st)
{
    if (dt == DT_BF16) return launch_mainl_t<DT_BF16, true>(a, grid, st);
    if (dt == DT_F16) return launch_mainl_t<DT_F16, true>(a, grid, st);
    if (dt == DT_F32) return launch_mainl_t<DT_F32, true>(a, grid, st);
    return hipErrorInvalidValue;
}

}  // namespace stk
