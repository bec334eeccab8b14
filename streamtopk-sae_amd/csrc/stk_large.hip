// stk_large.hip -- the streaming kernel for large batches (compute-bound).
//
// mainl_kernel: one workgroup of 4 waves (one per SIMD, up to 512 registers
// each) owns 256 rows and a contiguous range of 256-latent tiles.  The waves
// form a 2 x 2 grid: each scores 128 latents x 128 rows per tile as 8 x 8
// blocks of v_mfma_f32_16x16x32, with the 256 accumulators per lane in AGPRs.
// Both operands come from LDS; each 16-byte operand read feeds 8 MFMAs.
//   - W and X: whole 128-byte lines loaded straight from global memory into
//     2-stage LDS rings (buffer loads with the lds flag: no staging
//     registers, no LDS-store instructions), one d-step ahead; 128-byte rows
//     with the 16-byte chunks swizzled, so the MFMA-layout reads hit no bank
//     conflicts.  One barrier per d-step.  The W lines are shared through L2
//     by the row blocks of the W range.
//   - The next step's LDS loads are spread through the MFMAs (one per MFMA),
//     not issued as a burst: with one wave per SIMD, a vector-memory
//     instruction that cannot issue stalls the MFMAs behind it.
//   - Each d-step's last 16 MFMAs are issued after the next step's barrier,
//     between the reads of its first operands, so that the MFMAs do not sit
//     idle while those reads land (the sums are unchanged: every
//     accumulator still takes its products in d order).
//   - The pipeline restarts at every tile, so the epilogue holds no prefetch.
//   - bias: the tile's 256 values are loaded at the tile start and staged in
//     LDS for the epilogue.
//   - epilogue, two 16-row blocks at a time and no barrier between them: the
//     accumulators are read once, biased, compared with the row thresholds
//     and staged in LDS; each lane reserves its survivors' slots in the rows'
//     queue segments in global memory (counters in LDS), and the wave's
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
// (w & 1) * 128 .. +127 for rows (w >> 1) * 128 .. +127, as 8 x 8 blocks of
// 16 x 16.  Each operand block read from LDS feeds 8 MFMAs.
constexpr int kLNB = 8;                      // 16-row blocks per wave
constexpr int kLLat = 8;                     // 16-latent blocks per wave
constexpr int kLPairs = kLNB / 2;            // epilogue rounds: two row blocks each
constexpr int kLTile = 256;                  // latents per tile
constexpr int kLDefer = 16;                  // MFMAs of each d-step issued after the next step's barrier
static_assert(kLDefer <= kLLat + kLNB, "one deferred MFMA per phase-0 operand read");
static_assert(2 * 16 * kLLat == kLTile && 2 * 16 * kLNB == kLargeRows, "2 x 2 wave grid");
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

// One 16 x 16 block through the k = 32 MFMA (fp16/bf16), or element e of
// the operands through the k = 4 one (fp32), accumulating into acc in place.
// Lane l supplies A[l % 16][8 (l / 16) + e'] in a and B[8 (l / 16) + e'][l % 16]
// in b (fp32: 4 (l / 16) + e'), e' over the 16 bytes; register r of lane l
// receives D[4 (l / 16) + r][l % 16].  On MI355X this form sustains ~12 % more
// FLOP/s than the 32x32 one under the power limit (1.99-2.01 against
// 1.73-1.81 PF/s in an MFMA loop on random operands): the same products with
// half the accumulator traffic per product.
// Written as volatile asm with the accumulator tied to its AGPRs: through the
// builtin, the compiler gives each of the 64 4-register accumulators a new
// register per MFMA and copies them back around every d-step (hundreds of
// AGPR/VGPR moves and spills per step), and volatile keeps the MFMAs in
// program order with the reads and loads woven between them.  The compiler's
// hazard checks do not look inside the asm: the operands are only ever
// written by LDS reads (whose waits the compiler counts) or zeroed before a
// tile's first loads and barrier (2 wait states needed), an MFMA's
// accumulator is next read by an MFMA 64 MFMAs later, the zeros written into
// the accumulators at a tile's start are separated from its first MFMA by the
// tile's first loads, barrier and operand reads (2 wait states needed), and
// the reads of the results wait for mfma_drain (tests/test_isa.py checks each
// of these on the compiled code).
template <int DT>
__device__ __forceinline__ void mfma16_tied(f32x4& acc, const u32x4& a, const u32x4& b, int e)
{
    if constexpr (DT == DT_BF16)
        asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
    else if constexpr (DT == DT_F16)
        asm volatile("v_mfma_f32_16x16x32_f16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
    else
        asm volatile("v_mfma_f32_16x16x4_f32 %0, %1, %2, %0" : "+a"(acc) : "v"(a[e]), "v"(b[e]));
}

// Wait states between the last MFMA of a tile and the first read of its
// results (a VALU read of an MFMA result needs up to passes + 4 = 20 on
// gfx950; 3 x 8 here).  Volatile, so that it stays between the MFMAs and the
// (volatile) accumulator reads.
__device__ __forceinline__ void mfma_drain()
{
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7");
}

template <int DT, bool SAMPLE, bool TAILK>
struct BigStream {
    static constexpr int E = DT == DT_F32 ? 4 : 1;   // MFMA rounds per phase
    const unsigned char* W;
    int64_t row_bytes;           // bytes of a W row and of an X row (d elements)
    const unsigned char* X;
    int64_t B, b0, F;
    int64_t tile_begin;
    int ntiles, nds, nds2;
    int tail;                    // elements of d in the last d-step when it is partial, else 0
    int s_lo, s_hi;              // d-steps [s_lo, s_hi) of every tile
    int samp_log2;               // SAMPLE: tile t covers sampled latents t*256 ..
    int tid, lane, wave;

    // load cursors (absolute d-steps), uniform
    int ws, xs;
    __amdgpu_buffer_rsrc_t wres, xres, zres;      // wres: this wave's 64-row run of the tile
    // LDS load i of a wave reads rows 8 i + lane / 8 of the wave's 64-row run
    // (W: of the tile; X: of the row block), chunk lane % 8 ^ xswz(row).
    // xswz(row) depends on row % 16 only, so loads i and i + 2 share their
    // chunk and lie 16 rows apart: load i's source offset is vb[i % 2] +
    // (i / 2) * rows16 (X: + xrun).
    int vb[2];                   // this lane's source offsets of loads 0 and 1
    int vbt[2];                  // the same in the partial last d-step: beyond every resource past d
    int rows16;                  // bytes of 16 rows
    int xrun;                    // bytes of the wave's 64-row X run into the row block
    int rd[2];                   // operand read offset of MFMA step m (row lane % 16 of block 0)

    __device__ __forceinline__ void init()
    {
        // LDS load i of wave w fills rows 64 w + 8 i .. +7 of a stage (W: the
        // wave's 64-row run of the tile; X: of the row block): lane -> row +
        // lane / 8, slot lane % 8, which holds chunk slot ^ xswz(row)
#pragma unroll
        for (int p = 0; p < 2; ++p) {
            const int r = 8 * p + (lane >> 3);   // row within the wave's 64
            const int chunk = (lane & 7) ^ xswz(r);
            vb[p] = r * (int)row_bytes + chunk * 16;
            vbt[p] = chunk * (16 / Dt<DT>::esize) < tail ? vb[p] : 0x40000000;
        }
        rows16 = 16 * (int)row_bytes;
        xrun = wave * 64 * (int)row_bytes;
        // lanes 16 g .. 16 g + 15 of MFMA step m read chunk 4 m + g of rows
        // 0 .. 15 of a block (rows 16 j + i share swizzle xswz(i))
        const int i = lane & 15, g = lane >> 4;
#pragma unroll
        for (int m = 0; m < 2; ++m) rd[m] = i * kStepBytes + (((4 * m + g) ^ xswz(i)) * 16);
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

    // Source offset of LDS load i from the pair of offsets b (vb, or vbt in
    // the partial last d-step (tail != 0), where a lane whose source chunk
    // lies past d takes an offset beyond every resource's size, so the load
    // returns zeros).
    __device__ __forceinline__ int load_off(const int (&b)[2], int i) const { return b[i & 1] + (i >> 1) * rows16; }

    // W of step ws (zeros past s_hi) straight into the W stage, whole 128-byte
    // lines: this wave's 64-row run.
    __device__ __forceinline__ void issue_w(unsigned char* wst)
    {
        const int w = __builtin_amdgcn_readfirstlane(ws);
        const bool live = w < s_hi;
        const __amdgpu_buffer_rsrc_t r = live ? wres : zres;
        const int so = live ? w * kStepBytes : 0;
        const bool tl = tail != 0 && w == nds - 1;
        const int b[2] = {tl ? vbt[0] : vb[0], tl ? vbt[1] : vb[1]};
#pragma unroll
        for (int i = 0; i < kLWChunks; ++i) lds_load16(r, wst + (wave * 64 + 8 * i) * kStepBytes, load_off(b, i), so);
        ++ws;
    }

    // X of step xs (zeros past s_hi and for rows past B) straight into the X stage.
    __device__ __forceinline__ void issue_x(unsigned char* xst)
    {
        const int x = __builtin_amdgcn_readfirstlane(xs);
        const bool live = x < s_hi;
        const __amdgpu_buffer_rsrc_t r = live ? xres : zres;
        const int so = live ? x * kStepBytes : 0;
        const bool tl = tail != 0 && x == nds - 1;
        const int b[2] = {tl ? vbt[0] : vb[0], tl ? vbt[1] : vb[1]};
#pragma unroll
        for (int i = 0; i < kLXChunks; ++i)
            lds_load16(r, xst + (wave * 64 + 8 * i) * kStepBytes, load_off(b, i) + xrun, so);
        ++xs;
    }

    // One d-step from LDS stages wst / xst: two MFMA phases m of k = 32 (half
    // the step's d each), 64 MFMAs apiece (fp32: 4 x 64 of k = 4, one element
    // of the 16-byte operands per round of 64).  The operands of phase 0 are
    // read at the step's start, after the barrier; the previous
    // step's last kLDefer MFMAs (whose operands a1 / b1 still hold) go between
    // those reads, so that the MFMAs are busy while the reads land (deferring
    // 16 took c4's kernel from ~1735 to ~1700 us on one box; 8 did as well,
    // 24 and 32 were slower).  Phase 1's operands are read during phase 0's
    // MFMAs, one read between MFMAs, and its last kLDefer MFMAs are left to
    // the next step (or to finish()).  Every accumulator still receives its
    // products in d order, so the sums are those of the undeferred order.
    // The next d-step's LDS loads are folded into the stream too -- W(s+1)
    // into wnx with the first reads after the barrier, X(s+1) into xnx at the
    // start of phase 1, one load instruction between MFMAs -- so that the
    // texture path works in the background instead of stalling the wave's
    // in-order issue.
    // The MFMAs are volatile asm (mfma16_tied), so this program order is the
    // issue order.
    __device__ __forceinline__ void step(f32x4 (&acc)[kLLat][kLNB], u32x4 (&a1)[kLLat], u32x4 (&b1)[kLNB],
                                         const unsigned char* wst, const unsigned char* xst, unsigned char* wnx,
                                         unsigned char* xnx)
    {
        const unsigned char* wl = wst + (wave & 1) * (16 * kLLat) * kStepBytes;
        const unsigned char* xl = xst + (wave >> 1) * (16 * kLNB) * kStepBytes;
        const int w = __builtin_amdgcn_readfirstlane(ws);   // the next d-step (ws == xs)
        const bool live = w < s_hi;
        const __amdgpu_buffer_rsrc_t wr = live ? wres : zres, xr = live ? xres : zres;
        const int so = live ? w * kStepBytes : 0;
        // the next d-step is the partial last one (only kernels built for a
        // partial last step look)
        const bool tl = TAILK && w == nds - 1;
        // the loads' offsets are formed in the step from two registers: opaque
        // here, so that the compiler does not keep all 16 alive across the loop
        int ob[2] = {tl ? vbt[0] : vb[0], tl ? vbt[1] : vb[1]};
        asm volatile("" : "+v"(ob[0]), "+v"(ob[1]));
        u32x4 a0[kLLat], b0[kLNB];
        // operand read r of a phase, in first-use order: W block 0, the X
        // blocks, W blocks 1 .. 7
        auto rd_op = [&](u32x4 (&av)[kLLat], u32x4 (&bv)[kLNB], int m, auto rc) {
            constexpr int r = decltype(rc)::value;
            if constexpr (r == 0) av[0] = *(const u32x4*)(wl + rd[m]);
            else if constexpr (r <= kLNB) bv[r - 1] = *(const u32x4*)(xl + rd[m] + (16 * (r - 1)) * kStepBytes);
            else av[r - kLNB] = *(const u32x4*)(wl + rd[m] + (16 * (r - kLNB)) * kStepBytes);
        };
        // after the barrier: (DS read, deferred MFMA, W load) x 8, (DS read,
        // deferred MFMA) x 8.  W comes from HBM: its loads go first, to land by
        // the step's end (W loads later in the step, or X loads in phase 0,
        // measured 1-10 % slower at B = 1024).
        static_for<kLLat + kLNB>([&](auto rc) {
            rd_op(a0, b0, 0, rc);
            if constexpr (decltype(rc)::value < kLDefer) deferred(acc, a1, b1, rc);
            if constexpr (decltype(rc)::value < kLWChunks) {
                constexpr int q = decltype(rc)::value;
                lds_load16(wr, wnx + (wave * 64 + 8 * q) * kStepBytes, load_off(ob, q), so);
            }
        });
        // phase 0: (MFMA, DS read) x 16, MFMA x the rest
        static_for<E * kLLat * kLNB>([&](auto jc) {
            constexpr int j = decltype(jc)::value;
            constexpr int e = j / (kLLat * kLNB), la = (j / kLNB) % kLLat, n = j % kLNB;
            mfma16_tied<DT>(acc[la][n], a0[la], b0[n], e);
            if constexpr (j < kLLat + kLNB) rd_op(a1, b1, 1, jc);
        });
        // phase 1: (MFMA, X load) x 8, MFMA x the rest but the last kLDefer
        static_for<E * kLLat * kLNB - kLDefer>([&](auto jc) {
            constexpr int j = decltype(jc)::value;
            constexpr int e = j / (kLLat * kLNB), la = (j / kLNB) % kLLat, n = j % kLNB;
            mfma16_tied<DT>(acc[la][n], a1[la], b1[n], e);
            if constexpr (j < kLXChunks)
                lds_load16(xr, xnx + (wave * 64 + 8 * j) * kStepBytes, load_off(ob, j) + xrun, so);
        });
        ++ws;
        ++xs;
    }

    // Deferred MFMA r of a step: its phase-1 MFMA E * 64 - kLDefer + r.
    template <class RC>
    __device__ __forceinline__ static void deferred(f32x4 (&acc)[kLLat][kLNB], const u32x4 (&a1)[kLLat],
                                                    const u32x4 (&b1)[kLNB], RC)
    {
        constexpr int j = E * kLLat * kLNB - kLDefer + RC::value;
        constexpr int e = j / (kLLat * kLNB), la = (j / kLNB) % kLLat, n = j % kLNB;
        mfma16_tied<DT>(acc[la][n], a1[la], b1[n], e);
    }

    // The last step's deferred MFMAs.
    __device__ __forceinline__ static void finish(f32x4 (&acc)[kLLat][kLNB], const u32x4 (&a1)[kLLat],
                                                  const u32x4 (&b1)[kLNB])
    {
        static_for<kLDefer>([&](auto rc) { deferred(acc, a1, b1, rc); });
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
           (size_t)kLWaves * cap * 8 + (size_t)kLargeRows * sizeof(uint64_t*) + 2 * kLWaves * sizeof(uint32_t);
}

// TAILK: built for a partial last d-step (d not a multiple of the step's elements)
template <int DT, bool SAMPLE, bool TAILK>
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
    uint32_t* vote = (uint32_t*)(cscr + kLWaves * a.cap);            // [2][waves] block_any slots (cap even)
    uint32_t vpar = 0;
    const int cap = a.cap, k = a.k;

    // wave is read into a scalar register so that the compiler knows it is
    // uniform: the per-wave buffer resources then stay in scalar registers
    // (a resource the compiler takes for divergent costs a waterfall loop
    // around every load).
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // MFMA result layout: register r of block (la, n) of lane 16 g + i is
    // latent lw0 + 16 la + 4 g + r of row rw0 + 16 n + i
    const int i16 = lane & 15, g = lane >> 4;
    const int lw0 = (wave & 1) * (16 * kLLat);   // this wave's first latent of the tile
    const int rw0 = (wave >> 1) * (16 * kLNB);   // this wave's first row of the row block

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

    BigStream<DT, SAMPLE, TAILK> bs;
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

    if (bs.ntiles > 0) {
        bs.init();

        f32x4 acc[kLLat][kLNB];
#pragma unroll
        for (int la = 0; la < kLLat; ++la)
#pragma unroll
            for (int n = 0; n < kLNB; ++n) acc[la][n] = f32x4{0.f, 0.f, 0.f, 0.f};

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
            // a padded last step (s >= nds) reads zeros: every step computes
            // unconditionally.  Every step takes the previous one's deferred
            // MFMAs: the first step's operands a1 / b1 are zeros, which add
            // exact zeros to the zero accumulators (a first step without them
            // left the compiler free to place the accumulators' zeroing, and it
            // moved live accumulators between registers).  The last step's
            // deferred MFMAs run in finish().  The zeros pass through an empty
            // asm, so that they are written here, before the first barrier
            // (a VALU write of an MFMA operand needs 2 wait states before the
            // MFMA), and so that the compiler does not take them from the
            // zeroed accumulators.
            u32x4 a1[kLLat], b1[kLNB];   // phase-1 operands, live into the next step
#pragma unroll
            for (int la = 0; la < kLLat; ++la) {
                a1[la] = u32x4{0u, 0u, 0u, 0u};
                asm volatile("" : "+v"(a1[la]));
            }
#pragma unroll
            for (int n = 0; n < kLNB; ++n) {
                b1[n] = u32x4{0u, 0u, 0u, 0u};
                asm volatile("" : "+v"(b1[n]));
            }
            // nds2 >= 2 (d >= 1, and a sample-mode d range holds at least one
            // step: ksplit <= nds): a loop that cannot run zero times, so that
            // no path around it joins the accumulators at finish() (the join
            // made the compiler move accumulators between registers)
            int s = 0;
            do {
                __builtin_amdgcn_s_waitcnt(0x0070);   // vmcnt(0) lgkmcnt(0): W/X(s) in stage 0
                __builtin_amdgcn_s_barrier();         // ... for every wave; stage 1 free
                bs.step(acc, a1, b1, wst0, xs0, wst1, xs1);   // loads W/X(s+1) into stage 1
                __builtin_amdgcn_s_waitcnt(0x0070);
                __builtin_amdgcn_s_barrier();
                bs.step(acc, a1, b1, wst1, xs1, wst0, xs0);   // loads W/X(s+2) into stage 0
                s += 2;
            } while (s < bs.nds2);
            bs.finish(acc, a1, b1);
            mfma_drain();
            // the loads past the last step (zeros) land before the rings are reused
            __builtin_amdgcn_s_waitcnt(0x0070);   // vmcnt(0) lgkmcnt(0)
            __syncthreads();
            if (SAMPLE) {
                // raw partial scores of this d range (split ks)
                float* P = a.P + (int64_t)ks * a.p_split;
#pragma unroll
                for (int n = 0; n < kLNB; ++n) {
                    const int64_t row = b0 + rw0 + 16 * n + i16;
                    if (row < B) {
#pragma unroll
                        for (int la = 0; la < kLLat; ++la) {
                            const int64_t f = tile0 + lw0 + 16 * la + 4 * g;
                            f32x4 v;
#pragma unroll
                            for (int e = 0; e < 4; ++e) v[e] = agpr_read(acc[la][n][e]);
                            *(f32x4*)(P + row * a.p_row + f) = flush_denorm4(v);
                        }
                    }
                }
                continue;
            }
            bias_s[tid] = bnext;
            __syncthreads();

            // ---- epilogue: bias, threshold filter, append to the row segments ----
            // Two row blocks (2 p, 2 p + 1) per round, with no barrier between
            // rounds.  Their 64 scores per lane are read from the accumulators
            // once, in straight-line code, biased and compared with the rows'
            // thresholds; they go to this wave's LDS staging area ([bit][lane],
            // in the idle W ring), where the survivor walk reads them back.  Bit
            // 32 s + 4 la + r of a round's mask is latent lat0 + 16 la + r of
            // row rw0 + 16 (2 p + s) + i16.  Survivors that find their row
            // segment full are kept in ovf[p] and handled after one barrier for
            // the whole tile.
            const bool edge = tile0 + kLTile > F ||
                              (a.sampled && (is_sampled(tile0, a.samp_log2, a.samp_blocks) ||
                                             is_sampled(tile0 + kLTile - 1, a.samp_log2, a.samp_blocks)));
            const int lat0 = (int)tile0 + lw0 + 4 * g;
            // latents past F or in the sample are never candidates here
            uint64_t vmask = ~0ull;
            if (edge) {
                uint32_t vm = 0;
#pragma unroll
                for (int bit = 0; bit < 32; ++bit) {
                    const int64_t f = lat0 + 16 * (bit >> 2) + (bit & 3);
                    const bool ok = f < F && !(a.sampled && is_sampled(f, a.samp_log2, a.samp_blocks));
                    vm |= ok ? (1u << bit) : 0u;
                }
                vmask = ((uint64_t)vm << 32) | vm;
            }
            // This wave's staging area: [lane][64 scores]; 16-byte chunk c of a
            // lane's 256 bytes sits in slot c ^ (lane & 15), so that the b128
            // writes of 16 consecutive lanes hit distinct banks.
            float* stage = (float*)wst0 + wave * (64 * 64);
            // This wave's survivor descriptors (the X ring is idle): up to 64 per lane.
            uint32_t* dlist = (uint32_t*)xs0 + wave * (64 * 64);
            auto stage_at = [&](int ln, int bit) -> float {
                return stage[ln * 64 + ((((bit >> 2) ^ (ln & 15))) << 2) + (bit & 3)];
            };
            // this lane's 32 bias values, in registers for all rounds
            f32x4 bias_r[kLLat];
#pragma unroll
            for (int la = 0; la < kLLat; ++la) bias_r[la] = *(const f32x4*)(bias_s + lw0 + 16 * la + 4 * g);
            // Stages round p's biased scores; returns the mask of those not
            // below their row's threshold (t0: row block 2 p, t1: 2 p + 1).
            auto stage_pair = [&](auto pc, float t0, float t1) -> uint64_t {
                constexpr int p = decltype(pc)::value;
                uint64_t msk = 0;
#pragma unroll
                for (int s2 = 0; s2 < 2; ++s2) {
                    const float tv = s2 ? t1 : t0;
                    uint32_t m = 0;
#pragma unroll
                    for (int la = kLLat - 1; la >= 0; --la) {
                        const f32x4 bv = bias_r[la];
                        f32x4 v;
#pragma unroll
                        for (int e = 0; e < 4; ++e) v[e] = agpr_read(acc[la][2 * p + s2][e]) + bv[e];
                        *(f32x4*)(stage + lane * 64 + (((8 * s2 + la) ^ (lane & 15)) << 2)) = v;
#pragma unroll
                        for (int e = 3; e >= 0; --e) m = mask_step(m, v[e], tv);   // bits 31 .. 0
                    }
                    msk |= (uint64_t)m << (32 * s2);
                }
                return msk;
            };
            // Appends the staged scores of the bits of pend (round p) to the
            // rows' segments; returns the bits that found their segment full.
            // The lanes' survivors are spread over the whole wave: each lane
            // lists its own as descriptors (slot, bit, lane) at its offset in the
            // wave's list, then every lane stores one listed survivor per round.
            auto append = [&](auto pc, uint64_t pend) -> uint64_t {
                constexpr int p = decltype(pc)::value;
                const int row0 = rw0 + 32 * p + i16;   // row of bits 0 .. 31; + 16 for 32 .. 63
                const uint32_t lo = (uint32_t)pend, hi = (uint32_t)(pend >> 32);
                const int c0 = __popc(lo), c1 = __popc(hi);
                const int base0 = c0 ? atomicAdd(&cnt[row0], c0) : 0;
                const int base1 = c1 ? atomicAdd(&cnt[row0 + 16], c1) : 0;
                __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0)
                int nf0 = cap - base0, nf1 = cap - base1;
                nf0 = nf0 < 0 ? 0 : (nf0 > c0 ? c0 : nf0);
                nf1 = nf1 < 0 ? 0 : (nf1 > c1 ? c1 : nf1);
                const int nfit = nf0 + nf1;
                // exclusive prefix sum of nfit (<= 64) over the wave, from its bit planes
                int off = 0, total = 0;
#pragma unroll
                for (int bp = 0; bp < 7; ++bp) {
                    const uint64_t bal = __ballot((nfit >> bp) & 1);
                    off += (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(bal >> 32),
                                                          __builtin_amdgcn_mbcnt_lo((uint32_t)bal, 0u)) << bp;
                    total += __popcll(bal) << bp;
                }
                uint32_t m0 = lo, m1 = hi;
                for (int j = 0; j < nf0; ++j) {
                    const int bit = __builtin_ctz(m0);
                    m0 &= m0 - 1u;
                    dlist[off + j] = ((uint32_t)(base0 + j) << 12) | ((uint32_t)bit << 6) | (uint32_t)lane;
                }
                for (int j = 0; j < nf1; ++j) {
                    const int bit = __builtin_ctz(m1);
                    m1 &= m1 - 1u;
                    dlist[off + nf0 + j] =
                        ((uint32_t)(base1 + j) << 12) | ((uint32_t)(32 + bit) << 6) | (uint32_t)lane;
                }
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                for (int j = lane; j < total; j += 64) {
                    const uint32_t dsc = dlist[j];
                    const int ln = dsc & 63, bit = (dsc >> 6) & 63, slot = (int)(dsc >> 12);
                    const int lat = (int)tile0 + lw0 + 4 * (ln >> 4) + 16 * ((bit >> 2) & 7) + (bit & 3);
                    qrow[rw0 + 32 * p + 16 * (bit >> 5) + (ln & 15)][slot] = make_key(stage_at(ln, bit), lat);
                }
                __builtin_amdgcn_wave_barrier();
                return ((uint64_t)m1 << 32) | m0;
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
                //    each 64-latent half of its 128 latents: latent blocks
                //    4 q .. 4 q + 3, over the four lane groups
                static_for<kLNB>([&](auto nc) {
                    constexpr int n = decltype(nc)::value;
                    const int row = rw0 + 16 * n + i16;
#pragma unroll
                    for (int q = 0; q < 2; ++q) {
                        float m = -__builtin_inff();
#pragma unroll
                        for (int l4 = 0; l4 < 4; ++l4) {
                            const int la = 4 * q + l4;
#pragma unroll
                            for (int r = 0; r < 4; ++r) {
                                const float v = agpr_read(acc[la][n][r]) + bias_r[la][r];
                                m = __builtin_fmaxf(m, ((vmask >> (4 * la + r)) & 1ull) ? v : -__builtin_inff());
                            }
                        }
                        uint32_t o = ordered_u32(m);
                        uint32_t o2 = __shfl_xor(o, 16);
                        o = o2 > o ? o2 : o;
                        o2 = __shfl_xor(o, 32);
                        o = o2 > o ? o2 : o;
                        if (g == 0 && row < nrows)
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
            uint64_t ovf[kLPairs];
            static_for<kLPairs>([&](auto pc) {
                constexpr int p = decltype(pc)::value;
                const int row0 = rw0 + 32 * p + i16;
                const uint64_t tk0 = thr[row0], tk1 = thr[row0 + 16];
                uint64_t pend = stage_pair(pc, tk0 ? key_value(tk0) : -__builtin_inff(),
                                           tk1 ? key_value(tk1) : -__builtin_inff());
                const uint64_t rows_ok = (b0 + row0 < B ? 0xFFFFFFFFull : 0ull) |
                                         (b0 + row0 + 16 < B ? 0xFFFFFFFF00000000ull : 0ull);
                ovf[p] = append(pc, pend & vmask & rows_ok);
            });
            if (block_any<kLWaves>((ovf[0] | ovf[1] | ovf[2] | ovf[3]) != 0, vote, vpar, wave, lane)) {
                // Rare: some row segments are full.  Round by round: compact the
                // full segments to their top k (which raises their thresholds),
                // drop the pending scores now below threshold, append the rest;
                // repeat until nothing is pending.
                static_for<kLPairs>([&](auto pc) {
                    constexpr int p = decltype(pc)::value;
                    const int row0 = rw0 + 32 * p + i16;
                    uint64_t pend = ovf[p];
                    if (!block_any<kLWaves>(pend != 0, vote, vpar, wave, lane)) return;
                    stage_pair(pc, 0.f, 0.f);   // this pair's scores back into the staging area
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
                        // drop pending scores that fell below the raised thresholds
                        const uint64_t tk0 = thr[row0], tk1 = thr[row0 + 16];
                        uint64_t mm2 = pend;
                        while (mm2) {
                            const int bit = __builtin_ctzll(mm2);
                            mm2 &= mm2 - 1u;
                            const int off = 16 * ((bit >> 2) & 7) + (bit & 3);
                            if (!(make_key(stage_at(lane, bit), lat0 + off) > ((bit >> 5) ? tk1 : tk0)))
                                pend &= ~(1ull << bit);
                        }
                        pend = append(pc, pend);
                        if (!block_any<kLWaves>(pend != 0, vote, vpar, wave, lane)) break;
                    }
                });
            }
#pragma unroll
            for (int la = 0; la < kLLat; ++la)
#pragma unroll
                for (int n = 0; n < kLNB; ++n) acc[la][n] = f32x4{0.f, 0.f, 0.f, 0.f};
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

template <int DT, bool SAMPLE, bool TAILK>
static hipError_t launch_mainl_k(const MainLArgs& a, int grid, hipStream_t st)
{
    const size_t lds = mainl_lds_bytes(a.cap);
    auto kern = mainl_kernel<DT, SAMPLE, TAILK>;
    hipError_t e = ensure_lds((const void*)kern, lds);
    if (e != hipSuccess) return e;
    launch(kern, dim3((unsigned)grid), dim3(kLargeThreads), lds, st, a);
    return hipGetLastError();
}

template <int DT, bool SAMPLE>
static hipError_t launch_mainl_t(const MainLArgs& a, int grid, hipStream_t st)
{
    if (a.d % Dt<DT>::DS != 0) return launch_mainl_k<DT, SAMPLE, true>(a, grid, st);
    return launch_mainl_k<DT, SAMPLE, false>(a, grid, st);
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
