// stk_large.hip -- the streaming kernel for large batches (compute-bound).
//
// mainl_kernel: one workgroup of 4 waves (one per SIMD, up to 512 registers
// each) owns 256 rows and a contiguous range of 256-latent tiles.  The waves
// form a 2 x 2 grid: each scores 128 latents x 128 rows per tile as 4 x 4
// blocks of v_mfma_f32_32x32x16, with the 256 accumulators per lane in AGPRs.
// Both operands come from LDS; each 16-byte operand read feeds 4 MFMAs.
//   - W and X: whole 128-byte lines loaded straight from global memory into
//     2-stage LDS rings (buffer loads with the lds flag: no staging
//     registers, no LDS-store instructions), one d-step ahead; 128-byte rows
//     with the 16-byte chunks swizzled, so the MFMA-layout reads hit no bank
//     conflicts.  One barrier per d-step.  The W lines are shared through L2
//     by the row blocks of the W range.
//   - The next step's LDS loads are spread through the first two quads'
//     MFMAs (one per MFMA), not issued as a burst: with one wave per SIMD, a
//     vector-memory instruction that cannot issue stalls the MFMAs behind it.
//   - The pipeline restarts at every tile, so the epilogue holds no prefetch.
//   - bias: the tile's 256 values are loaded at the tile start and staged in
//     LDS for the epilogue.
//   - epilogue, one row block at a time and no barrier between blocks: the
//     accumulators are read once, biased, compared with the row threshold
//     and staged in LDS; each lane reserves its survivors' slots in the row's
//     queue segment in global memory (counters in LDS), and the wave's
//     survivors are spread over its lanes for the stores.  Survivors that
//     find a segment full wait for one barrier per tile; then the full
//     segments are rank-compacted to their top-k, which raises the row
//     thresholds, and the rest is re-filtered and appended.
//   - grid: workgroups are placed so that the row blocks sharing a W range
//     run on one XCD (workgroup i runs on XCD i % 8), and W is fetched into
//     that XCD's L2 once for all of them.
//   - row thresholds: after the first tile every workgroup publishes the
//     largest score of each 64-latent quarter of it per row, and each row's
//     owner takes the k-th largest of those maxima (the threshold exchange,
//     as main_kernel's; MainLArgs::xch).
// mainl_kernel<DT, true> (sample mode) computes the raw scores of the
// sampled latents with the same machinery, for grids too small for the
// exchange: one 256-latent tile of them per workgroup and a d range per
// workgroup, partial sums summed in a fixed order by thr_kernel.
// The reference has no counterpart: its B >= #SMs path streams all of W per
// row (streamtopk_exact.cu:506-638).
#include "stk_kernels.h"

namespace stk {

namespace {

constexpr int kLWaves = 4;
// The waves form a 2 x 2 grid over the 256 x 256 tile: wave w scores latents
// (w & 1) * 128 .. +127 for rows (w >> 1) * 128 .. +127, as 4 x 4 blocks of
// 32 x 32.  Each operand block read from LDS feeds 4 MFMAs.
constexpr int kLNB = 4;                      // 32-row blocks per wave
constexpr int kLFrags = 4;                   // 32-latent fragments per wave
constexpr int kLTile = 256;                  // latents per tile
static_assert(2 * 32 * kLFrags == kLTile && 2 * 32 * kLNB == kLargeRows, "2 x 2 wave grid");
constexpr int kLWChunks = kLTile * 8 / kLargeThreads;       // 16-byte W chunks per thread per d-step
constexpr int kLWStage = kLTile * kStepBytes;               // W ring stage: 256 rows x 128 B (swizzled)
constexpr int kLXStage = kLargeRows * kStepBytes;           // X ring stage: 256 rows x 128 B (swizzled)
constexpr int kLXChunks = kLargeRows * 8 / kLargeThreads;  // 16-byte X chunks per thread per d-step

typedef __attribute__((address_space(1))) uint64_t gu64;   // a key in global memory

// Calls f(std::integral_constant<int, i>) for i = 0 .. N-1 (compile-time i, so
// that accumulator indices stay static).
template <int N, int I = 0, class Fn>
__device__ __forceinline__ void static_for(Fn&& f)
{
    if constexpr (I < N) {
        f(std::integral_constant<int, I>{});
        static_for<N, I + 1>(f);
    }
}

template <int DT, bool SAMPLE>
struct BigStream {
    const unsigned char* W;
    int64_t row_bytes;           // bytes of a W row and of an X row (d elements)
    const unsigned char* X;
    int64_t B, b0, F;
    int64_t tile_begin;
    int ntiles, nds, nds2;
    int tail;                    // elements of d in the last d-step when it is partial, else 0
    int s_lo, s_hi;              // d-steps [s_lo, s_hi) of every tile
    int samp_log2;               // SAMPLE: tile t covers sampled latents t*256 ..
    int tid, lane, wave, h, jl;

    // load cursors (absolute d-steps), uniform
    int ws, xs;
    __amdgpu_buffer_rsrc_t wres, xres, zres;      // wres: this wave's 64-row run of the tile
    int wvoff[kLWChunks];        // W LDS load i of this wave: this lane's source offset in the wave's run
    int xvoff[kLXChunks];        // X LDS load i of this wave: this lane's source offset in the row block
    int xrd[4];                  // X operand read offset of quad q (row jl of block 0)

    __device__ __forceinline__ void init()
    {
        // LDS load i of wave w fills rows 64 w + 8 i .. +7 of a stage (W: the
        // wave's 64-row run of the tile; X: of the row block): lane -> row +
        // lane / 8, slot lane % 8, which holds chunk slot ^ xswz(row)
#pragma unroll
        for (int i = 0; i < kLWChunks; ++i) {
            const int r = 8 * i + (lane >> 3);   // row within the wave's 64
            wvoff[i] = r * (int)row_bytes + (((lane & 7) ^ xswz(r)) * 16);
            xvoff[i] = (wave * 64 + r) * (int)row_bytes + (((lane & 7) ^ xswz(r)) * 16);
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) xrd[q] = jl * kStepBytes + (((h * 4 + q) ^ xswz(jl)) * 16);
        const int64_t nrows = (B - b0 < kLargeRows) ? B - b0 : kLargeRows;
        xres = make_rsrc(X + b0 * row_bytes, nrows * row_bytes);
        zres = make_rsrc(X, 0);
    }

    __device__ __forceinline__ void begin_tile(int t)
    {
        ws = xs = s_lo;
        const int64_t tile0 = (tile_begin + t) * kLTile;
        if (SAMPLE) {
            // each 64-row run is 64 consecutive latents of one sampled block
            const int64_t f0 = sample_latent(tile0 + 64 * wave, samp_log2);
            wres = make_rsrc(W + f0 * row_bytes, (int64_t)64 * row_bytes);
        } else {
            const int64_t f0 = tile0 + 64 * wave;
            int64_t n = F - f0;
            n = n < 64 ? (n > 0 ? n : 0) : 64;
            wres = make_rsrc(W + (n > 0 ? f0 : 0) * row_bytes, n * row_bytes);
        }
    }

    // The partial last d-step (tail != 0): a lane whose source chunk of load i
    // lies past d takes an offset beyond every resource's size, so the load
    // returns zeros.
    __device__ __forceinline__ int tail_off(int off, int i) const
    {
        const int r = 8 * i + (lane >> 3);
        const int chunk = (lane & 7) ^ xswz(r);
        return chunk * (16 / Dt<DT>::esize) < tail ? off : 0x40000000;
    }

    // W of step ws (zeros past s_hi) straight into the W stage, whole 128-byte
    // lines: this wave's 64-row run.
    __device__ __forceinline__ void issue_w(unsigned char* wst)
    {
        const int w = __builtin_amdgcn_readfirstlane(ws);
        const bool live = w < s_hi;
        const __amdgpu_buffer_rsrc_t r = live ? wres : zres;
        const int so = live ? w * kStepBytes : 0;
        if (tail != 0 && w == nds - 1) {
#pragma unroll
            for (int i = 0; i < kLWChunks; ++i)
                lds_load16(r, wst + (wave * 64 + 8 * i) * kStepBytes, tail_off(wvoff[i], i), so);
        } else {
#pragma unroll
            for (int i = 0; i < kLWChunks; ++i) lds_load16(r, wst + (wave * 64 + 8 * i) * kStepBytes, wvoff[i], so);
        }
        ++ws;
    }

    // X of step xs (zeros past s_hi and for rows past B) straight into the X stage.
    __device__ __forceinline__ void issue_x(unsigned char* xst)
    {
        const int x = __builtin_amdgcn_readfirstlane(xs);
        const bool live = x < s_hi;
        const __amdgpu_buffer_rsrc_t r = live ? xres : zres;
        const int so = live ? x * kStepBytes : 0;
        if (tail != 0 && x == nds - 1) {
#pragma unroll
            for (int i = 0; i < kLXChunks; ++i)
                lds_load16(r, xst + (wave * 64 + 8 * i) * kStepBytes, tail_off(xvoff[i], i), so);
        } else {
#pragma unroll
            for (int i = 0; i < kLXChunks; ++i) lds_load16(r, xst + (wave * 64 + 8 * i) * kStepBytes, xvoff[i], so);
        }
        ++xs;
    }

    // One d-step from LDS stages wst / xst, with the next step's LDS loads
    // folded into the MFMA stream: W(s+1) into wnx during quad 0 and X(s+1)
    // into xnx during quad 1, one load instruction between MFMAs, so that the
    // texture path works in the background instead of stalling the wave's
    // in-order issue.  Each quad also reads the 8 operand blocks (4 W
    // fragments, 4 X blocks) of the next.
    __device__ __forceinline__ void step(f32x16 (&acc)[kLFrags][kLNB], const unsigned char* wst,
                                         const unsigned char* xst, unsigned char* wnx, unsigned char* xnx)
    {
        const unsigned char* wl = wst + (wave & 1) * (32 * kLFrags) * kStepBytes;
        const unsigned char* xl = xst + (wave >> 1) * (32 * kLNB) * kStepBytes;
        u32x4 bA[kLNB], bB[kLNB], aA[kLFrags], aB[kLFrags];
#pragma unroll
        for (int n = 0; n < kLNB; ++n) bA[n] = *(const u32x4*)(xl + xrd[0] + (32 * n) * kStepBytes);
#pragma unroll
        for (int fa = 0; fa < kLFrags; ++fa) aA[fa] = *(const u32x4*)(wl + xrd[0] + (32 * fa) * kStepBytes);
        __builtin_amdgcn_sched_barrier(0);   // quad 0's operands are all in flight before any MFMA
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            u32x4 (&cur)[kLNB] = (q & 1) ? bB : bA;
            u32x4 (&nxt)[kLNB] = (q & 1) ? bA : bB;
            u32x4 (&wc)[kLFrags] = (q & 1) ? aB : aA;
            u32x4 (&wn)[kLFrags] = (q & 1) ? aA : aB;
            if (q < 3) {
#pragma unroll
                for (int fa = 0; fa < kLFrags; ++fa)
                    wn[fa] = *(const u32x4*)(wl + xrd[q + 1] + (32 * fa) * kStepBytes);
#pragma unroll
                for (int n = 0; n < kLNB; ++n) nxt[n] = *(const u32x4*)(xl + xrd[q + 1] + (32 * n) * kStepBytes);
            }
#pragma unroll
            for (int fa = 0; fa < kLFrags; ++fa)
#pragma unroll
                for (int n = 0; n < kLNB; ++n) mfma_quad<DT>(acc[fa][n], wc[fa], cur[n]);
            if (q == 0) issue_w(wnx);
            if (q == 1) issue_x(xnx);
            // (MFMA, DS read) x 8, then quads 0 and 1: (MFMA, LDS load) x 8; others: MFMA x 8
            if (q < 3) {
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // MFMA
                    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);   // DS read
                }
            }
            if (q < 2) {
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);   // VMEM read (to LDS)
                }
            } else if (q < 3) {
                __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);
            } else {
                __builtin_amdgcn_sched_group_barrier(0x008, 16, 0);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    }
};

// m * 2 + !(v < tv): one bit of a score mask, shifted in from the top
// (v_cmp into VCC, then the add takes VCC as its carry-in).
__device__ __forceinline__ uint32_t mask_step(uint32_t m, float v, float tv)
{
    uint32_t r;
    asm("v_cmp_nlt_f32 vcc, %1, %2\n\tv_addc_co_u32 %0, vcc, %3, %3, vcc" : "=v"(r) : "v"(v), "v"(tv), "v"(m) : "vcc");
    return r;
}

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
    return 2 * (size_t)kLWStage + 2 * (size_t)kLXStage + kLTile * sizeof(float) + kLargeRows * 8 + kLargeRows * 4 +
           (size_t)kLWaves * cap * 8 + (size_t)kLargeRows * sizeof(uint64_t*);
}

template <int DT, bool SAMPLE>
__global__ __launch_bounds__(kLargeThreads, 1) void mainl_kernel(MainLArgs a)
{
    extern __shared__ __align__(16) unsigned char smem[];
    unsigned char* wst0 = smem;                                       // W ring
    unsigned char* wst1 = smem + kLWStage;
    unsigned char* xs0 = smem + 2 * kLWStage;                         // X ring (swizzled)
    unsigned char* xs1 = xs0 + kLXStage;
    float* bias_s = (float*)(xs1 + kLXStage);                         // [kLTile]
    uint64_t* thr = (uint64_t*)(bias_s + kLTile);                    // [rows]
    int* cnt = (int*)(thr + kLargeRows);                              // [rows]
    // [rows] segment of each row.  Typed as global pointers: read back from LDS,
    // a plain pointer would make every segment access a flat instruction, which
    // the LDS waits (lgkmcnt) of the survivor walk would then wait for.
    gu64** qrow = (gu64**)(cnt + kLargeRows);
    uint64_t* cscr = (uint64_t*)(qrow + kLargeRows);                  // [waves][cap]
    const int cap = a.cap, k = a.k;

    // wave is read into a scalar register so that the compiler knows it is
    // uniform: the per-wave buffer resources then stay in scalar registers
    // (a resource the compiler takes for divergent costs a waterfall loop
    // around every load).
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int h = lane >> 5, jl = lane & 31;
    const int lw0 = (wave & 1) * (32 * kLFrags);   // this wave's first latent of the tile
    const int rw0 = (wave >> 1) * (32 * kLNB);     // this wave's first row of the row block

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

    // this call's tag (MainArgs::epoch), recorded for this call's merge
    uint32_t tag = 0;
    if (!SAMPLE) {
        tag = call_tag(a.epoch);
        if (blockIdx.x == 0 && tid == 0) {
            *a.cur = tag;
            clear_stale_err(a.err, tag);
        }
        for (int i = tid; i < kLargeRows; i += kLargeThreads) {
            const int64_t row = b0 + i;
            cnt[i] = 0;
            thr[i] = (row < B && a.thr0 != nullptr) ? a.thr0[row] : 0ull;
            qrow[i] = (gu64*)(a.list_keys + ((row < B) ? row : 0) * a.list_cap + a.head_span + (int64_t)rg * cap);
        }
    }

    BigStream<DT, SAMPLE> bs;
    bs.W = (const unsigned char*)a.W;
    bs.row_bytes = a.d * Dt<DT>::esize;
    bs.X = (const unsigned char*)a.X;
    bs.B = B;
    bs.b0 = b0;
    bs.F = F;
    bs.nds = (int)((a.d + Dt<DT>::DS - 1) / Dt<DT>::DS);
    bs.tail = (int)(a.d % Dt<DT>::DS);
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
            // Per d-step: W and X one step ahead, loaded straight into 2-stage
            // LDS rings (128-byte rows, 16-byte chunks swizzled) during the
            // first two quads of the step before; one barrier per d-step, after
            // the wave's own loads of the next step have landed.  Loads past the
            // last step read zeros.
            bs.begin_tile(t);
            bs.issue_w(wst0);   // W(0)
            bs.issue_x(xs0);    // X(0)
            // a padded last step (s >= nds) reads zeros: every step computes unconditionally
            for (int s = 0; s < bs.nds2; s += 2) {
                __builtin_amdgcn_s_waitcnt(0x0070);   // vmcnt(0) lgkmcnt(0): W/X(s) in stage 0
                __builtin_amdgcn_s_barrier();         // ... for every wave; stage 1 free
                bs.step(acc, wst0, xs0, wst1, xs1);   // loads W/X(s+1) into stage 1
                __builtin_amdgcn_s_waitcnt(0x0070);
                __builtin_amdgcn_s_barrier();
                bs.step(acc, wst1, xs1, wst0, xs0);   // loads W/X(s+2) into stage 0
            }
            // the loads past the last step (zeros) land before the rings are reused
            __builtin_amdgcn_s_waitcnt(0x0070);   // vmcnt(0) lgkmcnt(0)
            __syncthreads();
            if (SAMPLE) {
                // raw partial scores of this d range (split ks)
                float* P = a.P + (int64_t)ks * a.p_split;
#pragma unroll
                for (int n = 0; n < kLNB; ++n) {
                    const int64_t row = b0 + rw0 + 32 * n + jl;
                    if (row < B) {
#pragma unroll
                        for (int fa = 0; fa < kLFrags; ++fa)
#pragma unroll
                            for (int r4 = 0; r4 < 4; ++r4) {
                                const int64_t i = tile0 + lw0 + fa * 32 + r4 * 8 + h * 4;
                                f32x4 v;
#pragma unroll
                                for (int e = 0; e < 4; ++e) v[e] = acc[fa][n][r4 * 4 + e];
                                *(f32x4*)(P + row * a.p_row + i) = flush_denorm4(v);
                            }
                    }
                }
                continue;
            }
            bias_s[tid] = bnext;
            __syncthreads();

            // ---- epilogue: bias, threshold filter, append to the row segments ----
            // One row block at a time, with no barrier between blocks.  Its 64
            // scores per lane are read from the accumulators once, in
            // straight-line code, biased and compared with the row threshold;
            // they go to this wave's LDS staging area ([bit][lane], in the idle W
            // ring), where the survivor walk reads them back.  Bit 16*fa + r of a
            // row mask is latent lat0 + fa*32 + 8*(r/4) + r%4; this lane's row is
            // rw0 + 32*n + jl.  Survivors that find their row segment full are
            // kept in ovf[n] and handled after one barrier for the whole tile.
            const bool edge = tile0 + kLTile > F ||
                              (a.sampled && (is_sampled(tile0, a.samp_log2, a.samp_blocks) ||
                                             is_sampled(tile0 + kLTile - 1, a.samp_log2, a.samp_blocks)));
            const int lat0 = (int)tile0 + lw0 + h * 4;
            const float* bias_l = bias_s + lw0 + h * 4;   // + fa*32 + 8*(r/4) + r%4
            // latents past F or in the sample are never candidates here
            uint64_t vmask = ~0ull;
            if (edge) {
                vmask = 0;
#pragma unroll
                for (int bit = 0; bit < 16 * kLFrags; ++bit) {
                    const int64_t f = lat0 + (bit >> 4) * 32 + ((bit & 15) >> 2) * 8 + (bit & 3);
                    const bool ok = f < F && !(a.sampled && is_sampled(f, a.samp_log2, a.samp_blocks));
                    vmask |= ok ? (1ull << bit) : 0ull;
                }
            }
            // This wave's staging area: [lane][64 scores]; 16-byte chunk c of a
            // lane's 256 bytes sits in slot c ^ (lane & 15), so that the b128
            // writes of 16 consecutive lanes hit distinct banks.
            float* stage = (float*)wst0 + wave * (16 * kLFrags * 64);
            // This wave's survivor descriptors (the X ring is idle): up to 64 per lane.
            uint32_t* dlist = (uint32_t*)xs0 + wave * (64 * 64);
            auto stage_at = [&](int ln, int bit) -> float {
                return stage[ln * 64 + ((((bit >> 2) ^ (ln & 15))) << 2) + (bit & 3)];
            };
            // Stages row block n's biased scores; returns the mask of those not
            // below threshold tv.
            // this lane's 64 bias values, in registers for all row blocks
            f32x4 bias_r[kLFrags * 4];
#pragma unroll
            for (int i = 0; i < kLFrags * 4; ++i) bias_r[i] = *(const f32x4*)(bias_l + (i >> 2) * 32 + 8 * (i & 3));
            auto stage_block = [&](auto nc, float tv) -> uint64_t {
                constexpr int n = decltype(nc)::value;
                uint64_t msk = 0;
#pragma unroll
                for (int fa = 0; fa < kLFrags; ++fa) {
                    uint32_t m = 0;
#pragma unroll
                    for (int r4 = 3; r4 >= 0; --r4) {
                        const f32x4 bv = bias_r[fa * 4 + r4];
                        f32x4 v;
#pragma unroll
                        for (int e = 0; e < 4; ++e) v[e] = agpr_read(acc[fa][n][4 * r4 + e]) + bv[e];
                        *(f32x4*)(stage + lane * 64 + (((4 * fa + r4) ^ (lane & 15)) << 2)) = v;
#pragma unroll
                        for (int e = 3; e >= 0; --e) m = mask_step(m, v[e], tv);   // bits 15 .. 0
                    }
                    msk |= (uint64_t)m << (16 * fa);
                }
                return msk;
            };
            // Appends the staged scores of the bits of pend (row block n) to the
            // rows' segments; returns the bits that found their segment full.
            // The lanes' survivors are spread over the whole wave: each lane
            // lists its own as descriptors (slot, bit, lane) at its offset in the
            // wave's list, then every lane stores one listed survivor per round.
            auto append = [&](auto nc, uint64_t pend) -> uint64_t {
                constexpr int n = decltype(nc)::value;
                const int row = rw0 + 32 * n + jl;
                const int c = __popcll(pend);
                const int base = c ? atomicAdd(&cnt[row], c) : 0;
                __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0)
                int nfit = cap - base;
                nfit = nfit < 0 ? 0 : (nfit > c ? c : nfit);
                // exclusive prefix sum of nfit (<= 64) over the wave, from its bit planes
                int off = 0, total = 0;
#pragma unroll
                for (int bp = 0; bp < 7; ++bp) {
                    const uint64_t bal = __ballot((nfit >> bp) & 1);
                    off += (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(bal >> 32),
                                                          __builtin_amdgcn_mbcnt_lo((uint32_t)bal, 0u)) << bp;
                    total += __popcll(bal) << bp;
                }
                uint64_t mm = pend;
                for (int i = 0; i < nfit; ++i) {
                    const int bit = __builtin_ctzll(mm);
                    mm &= mm - 1u;
                    dlist[off + i] = ((uint32_t)(base + i) << 12) | ((uint32_t)bit << 6) | (uint32_t)lane;
                }
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                for (int j = lane; j < total; j += 64) {
                    const uint32_t dsc = dlist[j];
                    const int ln = dsc & 63, bit = (dsc >> 6) & 63, slot = (int)(dsc >> 12);
                    const int lat = (int)tile0 + lw0 + (ln >> 5) * 4 + (bit >> 4) * 32 + ((bit & 15) >> 2) * 8 + (bit & 3);
                    qrow[rw0 + 32 * n + (ln & 31)][slot] = make_key(stage_at(ln, bit), lat);
                }
                __builtin_amdgcn_wave_barrier();
                return mm;
            };
            if (a.xch && t == 0) {
                // ---- threshold exchange after the first tile (MainArgs::xch's,
                // with kLXchPerWg maxima per row and workgroup) ----
                const int nw = a.xnr * kLXchPerWg;  // maxima per row, <= 512 (host)
                const int nrows = (int)(B - b0 < kLargeRows ? B - b0 : kLargeRows);
                // the row block passes through an empty asm so that no address
                // derived from it is hoisted out of the tile loop
                int64_t rbl = rb;
                asm volatile("" : "+s"(rbl));
                uint64_t* xmax = a.xmax + rbl * kLargeRows * nw;   // [kLargeRows][nw]
                uint64_t* xthr = a.xthr + rbl * kLargeRows;        // [kLargeRows]
                // 1. per row of this wave, the largest score (NaN left out) of
                //    each 64-latent half of its 128 latents
                static_for<kLNB>([&](auto nc) {
                    constexpr int n = decltype(nc)::value;
                    const int row = rw0 + 32 * n + jl;
#pragma unroll
                    for (int q = 0; q < 2; ++q) {
                        float m = -__builtin_inff();
#pragma unroll
                        for (int f2 = 0; f2 < 2; ++f2) {
                            const int fa = 2 * q + f2;
#pragma unroll
                            for (int r = 0; r < 16; ++r) {
                                const float v = agpr_read(acc[fa][n][r]) + bias_r[fa * 4 + (r >> 2)][r & 3];
                                m = __builtin_fmaxf(m, ((vmask >> (16 * fa + r)) & 1ull) ? v : -__builtin_inff());
                            }
                        }
                        uint32_t o = ordered_u32(m);
                        const uint32_t o2 = __shfl_xor(o, 32);
                        o = o2 > o ? o2 : o;
                        if (h == 0 && row < nrows)
                            xch_put(xmax + (int64_t)row * nw + rg * kLXchPerWg + (wave & 1) * 2 + q, tag, o);
                    }
                });
                // 2. owned rows rg, rg + xnr, ...: the k-th largest of the
                //    row's maxima once max(k, 3/4 nw) have arrived (this
                //    workgroup has tiles, so rg < xnr)
                const int quorum = (3 * nw + 3) / 4;
                const int need = a.k > quorum ? a.k : quorum;
                for (int j = wave;; j += kLWaves) {
                    const int row = rg + j * a.xnr;
                    if (row >= nrows) break;
                    uint32_t v[8];
                    uint32_t T = 0;
                    const int got = xch_poll<8>(xmax + (int64_t)row * nw, nw, need, tag, a.xwait, lane, v);
                    // any k arrived maxima bound the k-th score, a quorum or not
                    if (got >= a.k) T = xch_kth<8>(v, a.k);
                    if (got < need && lane == 0 && a.xwait > 0) atomicAdd(a.xto, 1u);
                    if (lane == 0) xch_put(xthr + row, tag, T);
                }
                // 3. wave w reads rows 64 w .. 64 w + 63; a row whose threshold
                //    has not arrived when the wait runs out reads 0 (every
                //    score passes), the others keep theirs
                {
                    uint32_t v[1];
                    const int base = 64 * wave;
                    const int n = nrows - base < 64 ? nrows - base : 64;
                    const int got = n > 0 ? xch_poll<1>(xthr + base, n, n, tag, a.xwait, lane, v) : 0;
                    if (n > 0 && got < n && lane == 0 && a.xwait > 0) atomicAdd(a.xto, 1u);
                    thr[base + lane] = xch_key(n > 0 ? v[0] : 0u);
                }
                __syncthreads();
            }
            uint64_t ovf[kLNB];
            static_for<kLNB>([&](auto nc) {
                constexpr int n = decltype(nc)::value;
                const int row = rw0 + 32 * n + jl;
                const uint64_t tk = thr[row];
                uint64_t pend = stage_block(nc, tk ? key_value(tk) : -__builtin_inff());
                pend = (b0 + row < B) ? (pend & vmask) : 0ull;
                ovf[n] = append(nc, pend);
            });
            if (__syncthreads_or((ovf[0] | ovf[1] | ovf[2] | ovf[3]) != 0)) {
                // Rare: some row segments are full.  Block by block: compact the
                // full segments to their top k (which raises their thresholds),
                // drop the pending scores now below threshold, append the rest;
                // repeat until nothing is pending.
                static_for<kLNB>([&](auto nc) {
                    constexpr int n = decltype(nc)::value;
                    const int row = rw0 + 32 * n + jl;
                    uint64_t pend = ovf[n];
                    if (!__syncthreads_or(pend != 0)) return;
                    stage_block(nc, 0.f);   // this block's scores back into the staging area
                    for (int it = 0;; ++it) {
                        if (it >= a.max_rounds) {
                            // unreachable by the bound's argument (kMainLMaxRounds):
                            // the pending scores are lost, so the result is marked
                            if (tid == 0) __hip_atomic_store(a.err, (uint64_t)tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                            break;
                        }
                        __threadfence_block();   // this thread's segment stores are complete
                        __syncthreads();
                        compact_full_rows<kLargeRows / kLWaves>(cnt, thr, cscr + wave * cap,
                                                               [&](int r) { return qrow[r]; }, cap, k, wave, lane);
                        __threadfence_block();
                        __syncthreads();
                        // drop pending scores that fell below the raised threshold
                        const uint64_t tk = thr[row];
                        uint64_t mm2 = pend;
                        while (mm2) {
                            const int bit = __builtin_ctzll(mm2);
                            mm2 &= mm2 - 1u;
                            const int off = (bit >> 4) * 32 + ((bit & 15) >> 2) * 8 + (bit & 3);
                            if (!(make_key(stage_at(lane, bit), lat0 + off) > tk)) pend &= ~(1ull << bit);
                        }
                        pend = append(nc, pend);
                        if (!__syncthreads_or(pend != 0)) break;
                    }
                });
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
    hipError_t e = ensure_lds((const void*)kern, lds);
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
