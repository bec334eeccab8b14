// stk_kernels.hip -- the exact streaming top-k encoder on gfx950.
//
//   main_kernel    : streams W once; MFMA scores for 256 latents x up to 128
//                    rows per tile; scores not below the row threshold go to
//                    a short per-row LDS queue, which spills to the
//                    workgroup's segment of the row's list when it fills; a
//                    full segment is rank-compacted to its top-k.  At the end
//                    every queue is flushed to its segment.  The row
//                    thresholds come from the workgroups' first tiles
//                    (xch_thresholds: each row's k-th largest of the
//                    workgroups' maxima), or, for grids too small for that,
//                    from the two passes below (then the sampled latents are
//                    skipped here: each latent is scored by exactly one kernel).
//   sample_kernel  : fp32 partial sums (one per d range) of the scores of the
//                    sampled latents (blocks of 128 consecutive latents spread
//                    over F) for every row.
//   thr_kernel     : per row, the k-th largest sampled key: a lower bound of
//                    the row's k-th key; the sample's top k open the row's
//                    candidate list.
//   merge_seg_kernel / merge_kernel : per row, top-k of its candidate list
//                    (the head, if any, and one segment per workgroup).
//
// The reference's pass 1 / pass 2 split (streamtopk_exact.cu:58-187 tile
// kernel, :429-499 merge kernel) maps to main_kernel / merge_kernel; its
// per-thread insertion buffers (topk_buffer.cuh) are replaced by threshold
// filtering against a row threshold that only ever rises, so almost no
// selection work is done in the streaming kernel.
#include "stk_kernels.h"

namespace stk {

// Register r (0..15, varying per lane) of a lane's 16 accumulators, by a
// four-level tree of bitwise selects: a lane cannot index its own registers
// (written as masks so the compiler cannot turn the tree back into an
// indexed array, which would live in scratch memory).
__device__ __forceinline__ float sel_bit(uint32_t r, uint32_t bit, float hi, float lo)
{
    const uint32_t m = 0u - ((r >> bit) & 1u);
    return __uint_as_float((m & __float_as_uint(hi)) | (~m & __float_as_uint(lo)));
}

__device__ __forceinline__ float pick16(const f32x16& v, uint32_t r)
{
    const float a0 = sel_bit(r, 0, v[1], v[0]), a1 = sel_bit(r, 0, v[3], v[2]);
    const float a2 = sel_bit(r, 0, v[5], v[4]), a3 = sel_bit(r, 0, v[7], v[6]);
    const float a4 = sel_bit(r, 0, v[9], v[8]), a5 = sel_bit(r, 0, v[11], v[10]);
    const float a6 = sel_bit(r, 0, v[13], v[12]), a7 = sel_bit(r, 0, v[15], v[14]);
    const float b0 = sel_bit(r, 1, a1, a0), b1 = sel_bit(r, 1, a3, a2);
    const float b2 = sel_bit(r, 1, a5, a4), b3 = sel_bit(r, 1, a7, a6);
    const float c0 = sel_bit(r, 2, b1, b0), c1 = sel_bit(r, 2, b3, b2);
    return sel_bit(r, 3, c1, c0);
}

// ---------------------------------------------------------------------------
// main_kernel
// ---------------------------------------------------------------------------
// Spills the LDS queues of the rows `sel` selects among this wave's rows (bit
// i: row wave*R + i) to their global segments (row r's at seg + r *
// seg_stride, cap keys).  A segment without room for the queue's keys is
// first rank-compacted to its top k (raising the row threshold), then the LDS
// keys above the threshold are appended.  Every global access of a row is
// made by the wave that owns the row.  Ends with the wave's stores complete.
template <int R>
__device__ __forceinline__ void spill_sel(uint64_t full, int* cnt, int* gcnt, uint64_t* thr, const uint64_t* lqk,
                                          uint64_t* seg, int64_t seg_stride, uint64_t* scr, int lq, int cap,
                                          int k, int wave, int lane)
{
    while (full) {
        const int i = __builtin_ctzll(full);
        full &= full - 1;
        const int row = wave * R + i;
        uint64_t* q = seg + row * seg_stride;
        const int nl = cnt[row] < lq ? cnt[row] : lq;
        int g = gcnt[row];
        uint64_t t = thr[row];
        if (g + nl > cap) {
            t = compact_row(q, g, scr, cap, k, lane);
            g = k;
        }
        // lq <= 64: one key per lane
        const uint64_t key = lane < nl ? lqk[row * lq + lane] : 0ull;
        const bool f = key > t;
        const uint64_t bal = __ballot(f);
        const int pos = (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(bal >> 32),
                                                       __builtin_amdgcn_mbcnt_lo((uint32_t)bal, 0u));
        if (f) q[g + pos] = key;
        if (lane == 0) {
            thr[row] = t;
            gcnt[row] = g + __popcll(bal);
            cnt[row] = 0;
        }
        __builtin_amdgcn_wave_barrier();
    }
    __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0): the segment stores are complete
}

// spill_sel over this wave's full queues.
template <int R>
__device__ __forceinline__ void spill_rows(int* cnt, int* gcnt, uint64_t* thr, const uint64_t* lqk,
                                           uint64_t* seg, int64_t seg_stride, uint64_t* scr, int lq, int cap,
                                           int k, int wave, int lane)
{
    const int myrow = wave * R + (lane < R ? lane : 0);
    const uint64_t full = __ballot(lane < R && cnt[myrow] >= lq);
    spill_sel<R>(full, cnt, gcnt, thr, lqk, seg, seg_stride, scr, lq, cap, k, wave, lane);
}

// End of main_kernel: moves the LDS queue keys of this wave's rows into their
// segments.  Rows whose segment lacks room go through spill_sel (compacted
// first); the others' keys are copied as they are, one row per round with a
// key per lane and no round waiting for another (a queued key at or below
// the final threshold is only an extra candidate, which the merge drops).
// Afterwards gcnt holds each segment's key count.  Ends with the stores
// complete.
template <int R>
__device__ __forceinline__ void flush_rows(int* cnt, int* gcnt, uint64_t* thr, const uint64_t* lqk,
                                           uint64_t* seg, int64_t seg_stride, uint64_t* scr, int lq, int cap,
                                           int k, int wave, int lane)
{
    const int myrow = wave * R + (lane < R ? lane : 0);
    int c = lane < R ? (cnt[myrow] < lq ? cnt[myrow] : lq) : 0;
    int g = lane < R ? gcnt[myrow] : 0;
    const uint64_t tight = __ballot(c > 0 && g + c > cap);
    if (tight) {
        spill_sel<R>(tight, cnt, gcnt, thr, lqk, seg, seg_stride, scr, lq, cap, k, wave, lane);
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        c = lane < R ? (cnt[myrow] < lq ? cnt[myrow] : lq) : 0;   // 0 for the rows just spilled
        g = lane < R ? gcnt[myrow] : 0;
    }
#pragma unroll
    for (int i = 0; i < R; ++i) {
        const int ci = __shfl(c, i), gi = __shfl(g, i);
        const int row = wave * R + i;
        if (lane < ci) seg[row * seg_stride + gi + lane] = lqk[row * lq + lane];   // lq <= 64
    }
    if (lane < R) {
        gcnt[myrow] = g + c;
        cnt[myrow] = 0;
    }
    __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0): the segment stores are complete
}

// ---------------------------------------------------------------------------
// Threshold exchange (main_kernel, MainArgs::xch)
// ---------------------------------------------------------------------------
// After the first tile's scores (bias included) are in ac: fills thr[0..BT)
// with the row thresholds of the exchange.
//   1. Each workgroup publishes, per row, the score image (ordered_u32) of
//      the largest score of its first tile (NaN scores left out).
//   2. Workgroup x owns rows x, x + nwg, ... of its row block (one wave per
//      row): once max(k, 3/4 nwg) of the row's maxima have arrived, it takes
//      the k-th largest of those: at least k distinct latents of the row
//      score at least that value, so it is a lower bound of the row's k-th
//      score, whichever maxima arrived first (the result does not depend on
//      it, only the number of candidates).  Not waiting for the last quarter
//      spares the workgroups of the slowest XCDs most of the wait.  The
//      threshold key is the largest key below every key of that score.
//   3. Every workgroup polls its block's thresholds.
// A poll that runs out (some workgroup never became resident) leaves the
// affected thresholds at 0, which accepts every score: the result stays
// exact, the call only slower.  scr: 8 * BT LDS words, free while the
// epilogue runs.
template <int NB>
__device__ __forceinline__ void xch_thresholds(const MainArgs& a, const f32x16 (&ac)[NB], uint32_t vmask,
                                               uint64_t* thr, uint32_t* scr, int64_t b0, int tid, uint32_t tag)
{
    constexpr int BT = 32 * NB;
    const int lane = tid & 63, wave = tid >> 6, h = lane >> 5, jl = lane & 31;
    const int nwg = (int)gridDim.x, x = (int)blockIdx.x;
    const int nrows = (int)(a.B - b0 < BT ? a.B - b0 : BT);
    const int nown = nwg < nrows ? nwg : nrows;
    // the row block passes through an empty asm so that no address derived
    // from it is hoisted out of the tile loop (kept live, it would spill)
    int64_t yb = blockIdx.y;
    asm volatile("" : "+s"(yb));
    uint64_t* xmax = a.xmax + yb * BT * nwg;   // [BT][nwg]
    uint64_t* xthr = a.xthr + yb * BT;         // [BT]

#pragma unroll
    for (int n = 0; n < NB; ++n) {
        float m = -__builtin_inff();
#pragma unroll
        for (int r = 0; r < 16; ++r) m = __builtin_fmaxf(m, ((vmask >> r) & 1u) ? ac[n][r] : -__builtin_inff());
        const uint32_t o = ordered_u32(m);
        const uint32_t q = __shfl_xor(o, 32);
        if (h == 0) scr[wave * BT + 32 * n + jl] = q > o ? q : o;
    }
    __syncthreads();
    if (tid < nrows) {
        uint32_t m = scr[tid];
#pragma unroll
        for (int w = 1; w < kMainWaves; ++w) {
            const uint32_t o = scr[w * BT + tid];
            m = o > m ? o : m;
        }
        xch_put(xmax + (int64_t)tid * nwg + x, tag, m);
    }

    const int row = x + wave * nwg;
    if (x < nown && row < nrows) {
        uint32_t v[4];
        uint32_t T = 0;
        const int quorum = (3 * nwg + 3) / 4;
        const int need = a.k > quorum ? a.k : quorum;
        const int got = xch_poll<4>(xmax + (int64_t)row * nwg, nwg, need, tag, a.xwait, lane, v);
        // any k arrived maxima bound the k-th score, a quorum or not
        if (got >= a.k) T = xch_kth<4>(v, a.k);
        if (got < need && lane == 0 && a.xwait > 0) atomicAdd(a.xto, 1u);
        if (lane == 0) xch_put(xthr + row, tag, T);
    }

    // waves 0 and 1 poll the block's thresholds, a row per lane; a row whose
    // threshold has not arrived when the wait runs out reads 0 (key 0:
    // every score passes), the others keep theirs
    if (wave < 2) {
        uint32_t v[1];
        const int base = 64 * wave;
        const int n = nrows - base < 64 ? nrows - base : 64;
        const int got = n > 0 ? xch_poll<1>(xthr + base, n, n, tag, a.xwait, lane, v) : 0;
        if (n > 0 && got < n && lane == 0 && a.xwait > 0) atomicAdd(a.xto, 1u);
        if (base + lane < BT) thr[base + lane] = xch_key(n > 0 ? v[0] : 0u);
    }
    __syncthreads();
}

template <int DT, int NB>
__global__ __launch_bounds__(kMainThreads, 2) void main_kernel(MainArgs a)
{
    constexpr int BT = 32 * NB;
    constexpr int WAVES = kMainWaves;
    constexpr int R = BT / WAVES;   // rows each wave spills and flushes
    using TS = TileStream<DT, NB, WAVES>;
    extern __shared__ __align__(16) unsigned char smem[];
    const int cap = a.cap, lq = a.lq;
    uint64_t* thr = (uint64_t*)(smem + TS::kRingBytes);          // [BT] row threshold keys
    int* cnt = (int*)(thr + BT);                                   // [BT] LDS queue fill counts
    int* gcnt = cnt + BT;                                          // [BT] global segment fill counts
    float* bias_lds = (float*)(gcnt + BT);                         // [2][kTileLatents]
    uint64_t* lqk = (uint64_t*)(bias_lds + 2 * kTileLatents);      // [BT][lq] LDS queues
    uint64_t* cscr = lqk + BT * lq;                                // [WAVES][cap] compaction scratch
    uint32_t* vote = (uint32_t*)(cscr + WAVES * cap);              // [2][WAVES] block_any slots (cap even: 16-byte aligned)
    uint32_t vpar = 0;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int h = lane >> 5, jl = lane & 31;
    const int64_t b0 = (int64_t)blockIdx.y * BT;
    const int64_t B = a.B, F = a.F;
    const int k = a.k;
    // this call's tag: the workspace's epoch (advanced by the previous call's
    // merge) + 1, recorded for this call's merge after the first tile (the
    // epoch's load overlaps the first tile's)
    const uint32_t epoch = load_epoch(a.epoch);
    // this workgroup's global segments: cap keys in each row's list (row
    // b0 + r at seg + r * list_cap; rows past B are never written)
    uint64_t* seg = a.list_keys + b0 * a.list_cap + a.head_span + (int64_t)blockIdx.x * cap;

    for (int i = tid; i < BT; i += kMainThreads) {
        thr[i] = (a.thr0 != nullptr && b0 + i < B) ? a.thr0[b0 + i] : 0ull;
        cnt[i] = 0;
        gcnt[i] = 0;
    }

    TS ts;
    ts.W = (const unsigned char*)a.W;
    ts.w_row_bytes = a.d * Dt<DT>::esize;
    ts.bias = a.bias;
    ts.F = F;
    ts.tile_begin = (int64_t)blockIdx.x * a.tiles_per_wg;
    {
        const int64_t t1 = ts.tile_begin + a.tiles_per_wg;
        ts.ntiles = (int)((t1 < a.num_tiles ? t1 : a.num_tiles) - ts.tile_begin);
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
    // the accumulators start at the bias: ac holds the scores at the epilogue
    uint32_t tag = 0;
    ts.template run<true>(acc, smem, bias_lds, [&](int t, f32x16 (&ac)[NB], const float (&)[16]) {
        if (t == 0) {
            tag = call_tag_of(epoch);
            if (tid == 0) *a.cur = tag;
            if (tid == 0 && blockIdx.x == 0 && blockIdx.y == 0) clear_stale_err(a.err, tag);
        }
        // latent of accumulator register r of this lane: fl + 8*(r/4) + r%4
        const int64_t tile0 = (ts.tile_begin + t) * (int64_t)kTileLatents;
        const int64_t fl = tile0 + wave * 32 + h * 4;
        // latents past F or in the sample are never candidates here
        uint32_t vmask = 0xFFFFu;
        if (tile0 + kTileLatents > F || (a.sampled && (is_sampled(tile0, a.samp_log2, a.samp_blocks) ||
                                                       is_sampled(tile0 + kTileLatents - 1, a.samp_log2, a.samp_blocks)))) {
            vmask = 0;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int64_t f = fl + (r >> 2) * 8 + (r & 3);
                const bool ok = f < F && !(a.sampled && is_sampled(f, a.samp_log2, a.samp_blocks));
                vmask |= ok ? (1u << r) : 0u;
            }
        }
        if (a.xch && t == 0) xch_thresholds<NB>(a, ac, vmask, thr, (uint32_t*)(smem + TS::kWBuf), b0, tid, tag);
        // ---- scores not below the row threshold ----
        // The float test keeps every score whose key beats the threshold key
        // (and possibly a few equal to its value: harmless extra candidates).
        uint32_t pend[NB];
#pragma unroll
        for (int n = 0; n < NB; ++n) {
            const int j = 32 * n + jl;
            const uint64_t tk = thr[j];
            const float tv = tk ? key_value(tk) : -__builtin_inff();
            uint32_t m = 0;
#pragma unroll
            for (int r = 0; r < 16; ++r) m |= (!(ac[n][r] < tv)) ? (1u << r) : 0u;
            pend[n] = (b0 + j < B) ? (m & vmask) : 0u;
        }

        // ---- append to the LDS queues; spill full ones and retry while anything overflowed ----
        // A survivor's score comes out of its register by pick16 (a lane
        // cannot index its own registers; survivors are a few per cent of the
        // scores, so selecting beats staging every score in LDS).  The second
        // X ring buffer is idle during the epilogue: a slot per thread there
        // absorbs the writes of overflowing survivors.
        uint64_t* dump = (uint64_t*)(smem + 2 * TS::kWBuf + TS::kXBuf) + tid;
        for (int it = 0;; ++it) {
            bool overflow = false;
            // reserve the slots of every row block first, then wait once
            int base[NB];
#pragma unroll
            for (int n = 0; n < NB; ++n)
                base[n] = pend[n] ? atomicAdd(&cnt[32 * n + jl], __builtin_popcount(pend[n])) : 0;
#pragma unroll
            for (int n = 0; n < NB; ++n) {
                // this lane's survivors only, lowest register first
                uint64_t* qj = lqk + (32 * n + jl) * lq;
                uint32_t m = pend[n], keep = 0;
                int slot = base[n];
                while (m) {
                    const uint32_t r = (uint32_t)__builtin_ctz(m);
                    m &= m - 1u;
                    const bool ok = slot < lq;
                    *(ok ? qj + slot : dump) = make_key(pick16(ac[n], r), fl + (r >> 2) * 8 + (r & 3));
                    keep |= ok ? 0u : (1u << r);
                    ++slot;
                }
                pend[n] = keep;
                overflow |= keep != 0;
            }
            if (!block_any<WAVES>(overflow, vote, vpar, wave, lane)) break;
            if (it >= a.max_rounds) {
                // unreachable by the bound's argument (kMainMaxRounds): the
                // pending scores are lost, so the call's result is marked
                if (tid == 0) __hip_atomic_store(a.err, (uint64_t)tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                break;
            }
            __syncthreads();   // the LDS queues are complete
            spill_rows<R>(cnt, gcnt, thr, lqk, seg, a.list_cap, cscr + wave * cap, lq, cap, k, wave, lane);
            __syncthreads();
            // drop pending scores that fell below a raised threshold
#pragma unroll
            for (int n = 0; n < NB; ++n) {
                const uint64_t tk = thr[32 * n + jl];
                uint32_t m = pend[n];
                while (m) {
                    const uint32_t r = (uint32_t)__builtin_ctz(m);
                    m &= m - 1u;
                    if (!(make_key(pick16(ac[n], r), fl + (r >> 2) * 8 + (r & 3)) > tk)) pend[n] &= ~(1u << r);
                }
            }
        }
    });

    // ---- flush: every wave moves its R rows' LDS queues into their global
    // segments (compacting a segment without room), then publishes how many
    // keys each of its segments holds ----
    __syncthreads();
    flush_rows<R>(cnt, gcnt, thr, lqk, seg, a.list_cap, cscr + wave * cap, lq, cap, k, wave, lane);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const int myrow = wave * R + lane;
    if (lane < R && b0 + myrow < B) a.seg_cnt[(b0 + myrow) * gridDim.x + blockIdx.x] = gcnt[myrow];
}

// ---------------------------------------------------------------------------
// sample_kernel: partial sums P[split][row][i] = X[row] . W[f] over the d-steps
// of one split, f = sample_latent(i), for the nsamp sampled latents (the bias
// is added by thr_kernel, after the splits).  A workgroup owns 64 sampled
// latents x 32*NB rows x one d range of at most kSampleSteps steps: W is read
// once per row block, straight to registers in the MFMA layout; the X rows of
// the range are staged in LDS with whole 128-byte row steps per load (X lives
// in L2 and is read once per 64 latents).  Wave (g, sl) scores latent group g
// (32 latents) over the range's steps sl and sl + 4; the four step lanes'
// sums are added in a fixed order through LDS and written as whole rows
// (denormal sums as zero: flush_denorm4).
// ---------------------------------------------------------------------------
constexpr int kSampleStride = 68;   // floats per LDS-staged row of sums: 64 latents + pad (16-byte aligned)

size_t sample_lds_bytes(int NB)
{
    const size_t BT = 32 * (size_t)NB;
    const size_t x = (size_t)kSampleSteps * BT * kXRowStride;
    const size_t r = (size_t)4 * BT * kSampleStride * 4;
    return x > r ? x : r;
}

template <int DT, int NB>
__global__ __launch_bounds__(kSampleThreads) void sample_kernel(SampleArgs a)
{
    constexpr int ES = Dt<DT>::esize;
    constexpr int DS = Dt<DT>::DS;
    constexpr int BT = 32 * NB;
    constexpr int kChunks = kSampleSteps * BT * 8 / kSampleThreads;   // 16-byte X chunks per thread
    extern __shared__ __align__(16) unsigned char smem[];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int h = lane >> 5, jl = lane & 31;
    const int g = wave >> 2, sl = wave & 3;
    const int nlb = a.nsamp / kSampleLat;
    const int lb = (int)(blockIdx.x % nlb);
    const int sp = (int)(blockIdx.x / nlb);
    const int64_t ib = (int64_t)lb * kSampleLat;
    const int64_t b0 = (int64_t)blockIdx.y * BT;
    const int64_t d = a.d;
    constexpr int QE = 16 / ES;   // elements per 16-byte chunk
    const int64_t nds = (d + DS - 1) / DS;   // the last step may be partial: its chunks past d read as zeros
    const int64_t sb = sp * nds / a.nsplit;
    const int ns = (int)((sp + 1) * nds / a.nsplit - sb);   // 1 .. kSampleSteps (host)

    // X: chunk c is 16 bytes of row (c / 8) % BT at step c / (8 * BT); rows
    // past B and steps past the range are staged as zeros.  The X loads go
    // out first and W's after them, so waiting for X (in order) leaves the W
    // loads in flight until the MFMAs.
    const unsigned char* wp =
        (const unsigned char*)a.W + (sample_latent(ib + 32 * g + jl, a.samp_log2) * d + sb * DS) * ES + h * 64;
    u32x4 w[2][4];
    {
        u32x4 xr[kChunks];
        uint32_t okm = 0;
#pragma unroll
        for (int p = 0; p < kChunks; ++p) {
            // every load is in bounds (clamped row and step); a select at the
            // store keeps branches, and the register copies they cause, out
            const int c = tid + kSampleThreads * p;
            const int c16 = c & 7, row = (c >> 3) % BT, st = (c >> 3) / BT;
            const int64_t j = b0 + row;
            const int stc = st < ns ? st : ns - 1;
            const bool in_d = (sb + stc) * DS + c16 * QE < d;   // a chunk past d reads the step's first
            okm |= (j < a.B && st < ns && in_d) ? (1u << p) : 0u;
            const int64_t jc = j < a.B ? j : a.B - 1;
            xr[p] = *(const u32x4*)((const unsigned char*)a.X + (jc * d + (sb + stc) * DS) * ES +
                                    (in_d ? c16 * 16 : 0));
        }
        __builtin_amdgcn_sched_barrier(0);
        // W of steps sl and sl + 4 (a step past the range reloads step 0; its X
        // is zero); chunks past d read the step's first chunk and are zeroed
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            const int st = sl + 4 * t < ns ? sl + 4 * t : 0;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const bool in_d = (sb + st) * DS + h * (DS / 2) + q * QE < d;
                const u32x4 v = *(const u32x4*)(wp + st * kStepBytes + (in_d ? q * 16 : -h * 64));
                w[t][q] = in_d ? v : u32x4{0u, 0u, 0u, 0u};
            }
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int p = 0; p < kChunks; ++p) {
            const int c = tid + kSampleThreads * p;
            const int c16 = c & 7, row = (c >> 3) % BT, st = (c >> 3) / BT;
            *(u32x4*)(smem + (st * BT + row) * kXRowStride + c16 * 16) =
                (okm >> p & 1u) ? xr[p] : u32x4{0u, 0u, 0u, 0u};
        }
    }
    __syncthreads();

    f32x16 acc[NB];
#pragma unroll
    for (int n = 0; n < NB; ++n)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[n][r] = 0.f;
    // steps past the range multiply the zeros staged for them (no branch
    // around the MFMAs, whose accumulators would be copied at the join)
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        const int st = sl + 4 * t;
#pragma unroll
        for (int n = 0; n < NB; ++n)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const u32x4 bx = *(const u32x4*)(smem + (st * BT + 32 * n + jl) * kXRowStride + h * 64 + q * 16);
                mfma_quad<DT>(acc[n], w[t][q], bx);
            }
    }
    __syncthreads();   // the X area becomes the staging area of the sums

    // registers 4e..4e+3 of a lane hold latents 32g + 8e + 4h + 0..3 of row 32n + jl
    float* T = (float*)smem;   // [sl][BT][kSampleStride]
#pragma unroll
    for (int n = 0; n < NB; ++n)
#pragma unroll
        for (int e = 0; e < 4; ++e)
            *(f32x4*)(T + (sl * BT + 32 * n + jl) * kSampleStride + 32 * g + 8 * e + 4 * h) =
                f32x4{acc[n][4 * e], acc[n][4 * e + 1], acc[n][4 * e + 2], acc[n][4 * e + 3]};
    __syncthreads();
    float* Ps = a.P + (int64_t)sp * a.p_split;
    constexpr int WS = BT * kSampleStride;
    for (int c = tid; c < BT * 16; c += kSampleThreads) {
        const int row = c >> 4, c4 = (c & 15) * 4;
        const int64_t j = b0 + row;
        if (j < a.B) {
            const float* t0 = T + row * kSampleStride + c4;
            const f32x4 v = ((*(const f32x4*)t0 + *(const f32x4*)(t0 + WS)) + *(const f32x4*)(t0 + 2 * WS)) +
                            *(const f32x4*)(t0 + 3 * WS);
            *(f32x4*)(Ps + j * a.p_row + ib + c4) = flush_denorm4(v);
        }
    }
}

// ---------------------------------------------------------------------------
// Selection kernels (one workgroup per row).
// ---------------------------------------------------------------------------
// Per row: the threshold key main_kernel starts from and the head of the
// row's candidate list.  The threshold is the k-th largest sampled key (k
// real scores reach it, so it never exceeds the row's final k-th key); the
// sampled keys that reach it -- the sample's top k -- are written to the
// list, since main_kernel skips the sampled latents.
template <int kItems, int NT>
__global__ __launch_bounds__(NT) void thr_kernel(ThrArgs a)
{
    __shared__ SelSharedT<NT> S;
    const int tid = threadIdx.x;
    const int64_t row = blockIdx.x;
    if (a.P == nullptr) {
        if (tid == 0) { a.thr[row] = 0; a.list_cnt[row * kCntStride] = 0; }
        return;
    }
    // item t of this thread is sampled latent 4 * tid + NT * 4 * (t / 4) + t % 4:
    // four consecutive sampled latents (one 16-byte load of P) per quad
    constexpr int kQuads = kItems / 4;
    auto item = [&](int t) { return 4 * tid + NT * 4 * (t >> 2) + (t & 3); };
    const float* prow = a.P + row * a.p_row;
    const int64_t split_stride = a.p_split;
    // With up to 16 items per thread (both launches) the bias of the sampled
    // latents goes out first (it does not depend on P) and the splits' partial
    // sums four splits at a time with all their loads in flight; with more,
    // whose keys fill the registers, one split at a time and the bias last, as
    // more loads in flight would cost occupancy.  Either way the sums are added
    // in split order, then the bias.
    constexpr bool kEarly = kItems <= 16;
    constexpr int kSplitBatch = kEarly ? 4 : 1;
    float bsv[kEarly ? kItems : 1];
    if constexpr (kEarly) {
        if (a.bias != nullptr) {
#pragma unroll
            for (int t = 0; t < kItems; ++t) bsv[t] = a.bias[sample_latent(item(t), a.samp_log2)];   // 4-byte aligned only
        } else {
#pragma unroll
            for (int t = 0; t < kItems; ++t) bsv[t] = 0.f;
        }
    }
    f32x4 v[kQuads];
    for (int sp0 = 0; sp0 < a.nsplit; sp0 += kSplitBatch) {
        f32x4 p[kSplitBatch][kQuads];
#pragma unroll
        for (int j = 0; j < kSplitBatch; ++j) {
            const int sp = sp0 + j < a.nsplit ? sp0 + j : sp0;   // past the last split: reloaded, not added
#pragma unroll
            for (int u = 0; u < kQuads; ++u) p[j][u] = *(const f32x4*)(prow + sp * split_stride + item(4 * u));
        }
#pragma unroll
        for (int j = 0; j < kSplitBatch; ++j) {
            if (sp0 + j < a.nsplit) {
#pragma unroll
                for (int u = 0; u < kQuads; ++u) v[u] = (sp0 + j == 0) ? p[j][u] : v[u] + p[j][u];
            }
        }
    }
    if (a.bias != nullptr) {
#pragma unroll
        for (int t = 0; t < kItems; ++t)
            v[t >> 2][t & 3] += kEarly ? bsv[kEarly ? t : 0] : a.bias[sample_latent(item(t), a.samp_log2)];
    }
    uint64_t key[kItems];
    uint64_t m = 0;
#pragma unroll
    for (int t = 0; t < kItems; ++t) {
        key[t] = make_key(v[t >> 2][t & 3], sample_latent(item(t), a.samp_log2));
        m = key[t] > m ? key[t] : m;
    }
    if (tid == 0) { S.cnt = 0; S.sel_cnt = 0; }
    // T0 <= the sample's k-th key; the keys that reach it are few (about
    // 2-4% of the sample) and include the sample's k largest, whose k-th key
    // is the threshold: a lower bound of the row's k-th key (k real scores
    // reach it) and the tightest one the sample gives.
    const uint64_t T0 = kth_of_maxima(S, m, a.k, tid);
    uint32_t pass = 0;
#pragma unroll
    for (int t = 0; t < kItems; ++t) pass |= (key[t] >= T0) ? (1u << t) : 0u;
    const int base = wave_reserve(&S.cnt, __builtin_popcount(pass));
#pragma unroll
    for (int t = 0; t < kItems; ++t) {
        const int pos = base + __builtin_popcount(pass & ((1u << t) - 1u));
        if ((pass >> t & 1u) && pos < kSelCap) S.buf[pos] = key[t];
    }
    __syncthreads();
    const int n = S.cnt;   // >= k: at least k sampled keys reach T0
    uint64_t T = T0;
    uint64_t* out = a.list_keys + row * a.list_cap;
    if (n <= NT) {
        // the sample's k largest keys by rank, counted (thread t ranks key
        // t): the key of rank k - 1 is the threshold
        if (tid < n) {
            const uint64_t key = S.buf[tid];
            const int r = rank_desc<false>(S, n, key, tid);
            if (r < a.k) out[r] = key;
            if (r == a.k - 1) S.thr = key;
        }
        if (tid == 0) S.sel_cnt = a.k;
        __syncthreads();
        T = S.thr;
    } else if (n <= kSelCap) {
        // the sample's k largest keys (unordered): the k-th is the threshold
        select_compact(S, n, a.k, tid);
        if (tid < a.k) out[tid] = S.buf[tid];
        if (tid == 0) S.sel_cnt = a.k;
        T = S.thr;
    } else {
        // (only a sample larger than the selection buffer gets here: the head
        // then holds every sampled key that reaches T0, up to nsamp)
        uint32_t hit = 0;
#pragma unroll
        for (int t = 0; t < kItems; ++t) hit |= (key[t] >= T) ? (1u << t) : 0u;
        const int hb = wave_reserve(&S.sel_cnt, __builtin_popcount(hit));
#pragma unroll
        for (int t = 0; t < kItems; ++t)
            if (hit >> t & 1u) out[hb + __builtin_popcount(hit & ((1u << t) - 1u))] = key[t];
    }
    __syncthreads();
    if (tid == 0) {
        a.thr[row] = T;
        a.list_cnt[row * kCntStride] = S.sel_cnt;
    }
}

// One pass of the per-row selection: every thread holds N keys in v (0 for
// none).  The keys that reach the larger of the pass's bound (the k-th of the
// per-thread maxima: k of the pass's keys reach it) and `run` (the k-th key of
// the last compaction) go to S.buf; when it fills, it is compacted to its top
// k, which raises `run`.  Every thread of the workgroup takes part.
template <int N, int NT>
__device__ __forceinline__ void merge_pass(SelSharedT<NT>& S, const uint64_t (&v)[N], int k, int tid, uint64_t& run,
                                           uint32_t& vpar)
{
    static_assert(N <= 64, "pending mask");
    using Mask = std::conditional_t<(N > 32), uint64_t, uint32_t>;
    constexpr Mask one = 1;
    uint64_t m = 0;
#pragma unroll
    for (int u = 0; u < N; ++u) m = v[u] > m ? v[u] : m;
    const uint64_t T = kth_of_maxima(S, m, k, tid);
    const uint64_t thr = T > run ? T : run;
    Mask pend = 0;
#pragma unroll
    for (int u = 0; u < N; ++u) pend |= (v[u] != 0 && v[u] >= thr) ? (one << u) : Mask(0);
    for (;;) {
        bool stalled = false;
        const Mask pm = pend;
        const int base = wave_reserve(&S.cnt, __popcll((uint64_t)pm));
#pragma unroll
        for (int u = 0; u < N; ++u) {
            if (pm >> u & one) {
                const int pos = base + __popcll((uint64_t)(pm & ((one << u) - one)));
                if (pos < kSelCap) {
                    S.buf[pos] = v[u];
                    pend &= ~(one << u);
                } else {
                    stalled = true;
                }
            }
        }
        if (!block_any<NT / 64>(stalled, S.vote, vpar, tid >> 6, tid & 63)) break;
        select_compact(S, kSelCap, k, tid);   // S.cnt = k, S.thr = k-th key
        const uint64_t r2 = S.thr;
        run = r2;
        Mask keep = 0;
#pragma unroll
        for (int u = 0; u < N; ++u) keep |= (v[u] > r2) ? (one << u) : Mask(0);
        pend &= keep;
    }
}

// Per row: top-k of its candidates (MergeArgs: a dense head, then optional
// fixed-size segments), read in chunks of kPer slots per thread.  Each chunk
// is filtered against the larger of its own k-th of the per-thread maxima and
// the k-th key of the last compaction.
// kPer: candidate slots per thread and chunk.  kSpec > 0 (dense lists
// expected to fill a whole chunk): the first kSpec slots per thread are loaded
// at once, unconditionally (clamped into the row's list, masked afterwards),
// together with the row's count; every other slot is loaded only if it holds
// a candidate.
// Whether the error word holds this call's tag (a streaming kernel of the
// call lost candidates); if so, row `row` of the output is marked: indices
// -1, values NaN.  The word is the same for every thread, so the whole
// workgroup returns together.  Workgroup 0 also advances the workspace's
// epoch for the next call (no other kernel of this call reads it; the
// streaming kernel has recorded this call's tag in *cur), and every
// workgroup zeroes its row's threshold-exchange words.
template <int NT = kThreads>
__device__ __forceinline__ bool merge_marked(const MergeArgs& a, int64_t row, int tid)
{
    if (a.epoch != nullptr && blockIdx.x == 0 && tid == 0) *a.epoch = (*a.epoch % kTagPeriod + 1u) % kTagPeriod;
    if (a.xmax != nullptr) {
        // this row's exchange words: no later call may meet them
        uint64_t* xm = a.xmax + row * a.xmax_row;
        for (int64_t i = tid; i < a.xmax_row; i += NT) xm[i] = 0ull;
        if (tid == 0) a.xthr[row] = 0ull;
    }
    if (a.err == nullptr || *a.err != *a.cur) return false;
    for (int r = tid; r < a.k; r += NT) {
        a.V[row * a.k + r] = __builtin_nanf("");
        a.I[row * a.k + r] = -1;
    }
    return true;
}

// At most kMergeMaxSeg segments per row (host), one count per thread.
// kWaves: the waves per SIMD the registers must allow (1: no bound); the LDS
// and registers of the 16-slot instance leave room for four workgroups per
// CU, so a large batch's rows run in one round.
template <int kPer, int kSpec, int NT, int kWaves>
__global__ __launch_bounds__(NT, kWaves) void merge_kernel(MergeArgs a)
{
    constexpr int NW = NT / 64;
    static_assert(kMergeMaxSeg <= NT, "one segment count per thread");
    __shared__ SelSharedT<NT> S;
    __shared__ int spre[kMergeMaxSeg];   // inclusive prefix sums of the segment counts
    __shared__ int wsum[NW];
    const int tid = threadIdx.x;
    const int64_t row = blockIdx.x;
    if (merge_marked<NT>(a, row, tid)) return;
    const int k = a.k;
    const int nseg = a.nseg;
    const int64_t hc = a.head_span > 0 ? a.list_cnt[row * kCntStride] : 0;   // no head: no count either
    const uint64_t* keys = a.list_keys + row * a.list_cap;
    uint64_t v[kPer];
#pragma unroll
    for (int u = 0; u < kSpec; ++u) {
        const int64_t i = tid + (int64_t)u * NT;
        v[u] = keys[i < a.list_cap ? i : a.list_cap - 1];
    }
    // thread t holds the count of segment t; the inclusive prefix sums go to
    // spre (a scan over the lanes, then over the waves)
    const int cs = tid < nseg ? a.seg_cnt[row * nseg + tid] : 0;
    if (tid == 0) S.cnt = 0;
    // Candidate i (0 <= i < n) is head key i for i < hc, else key i - hc of
    // the segments' valid keys taken in order: the chunks run over valid keys
    // only, however full the segments are.
    int64_t n = hc;
    int top = 0;   // largest power of two <= nseg
    if (nseg > 0) {
        const int lane = tid & 63, wave = tid >> 6;
        int x = cs;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const int t = __shfl_up(x, o, 64);
            if (lane >= o) x += t;
        }
        if (lane == 63) wsum[wave] = x;
        __syncthreads();
#pragma unroll
        for (int w = 0; w < NW; ++w) x += w < wave ? wsum[w] : 0;
        if (tid < nseg) spre[tid] = x;
        __syncthreads();
        n = hc + spre[nseg - 1];
        top = 1 << (31 - __builtin_clz(nseg));
    } else {
        __syncthreads();
    }
    uint64_t run = 0;
    uint32_t vpar = 0;   // block_any's call parity
    for (int64_t c0 = 0; c0 < n; c0 += (int64_t)kPer * NT) {
        if (nseg > 0) {
            // segment of each segment candidate: the number of segments whose
            // inclusive prefix is <= its index (kGrp items searched in step;
            // a group's loads are in flight while the next group searches)
            constexpr int kGrp = kPer < 8 ? kPer : 8;
            static_assert(kPer % kGrp == 0, "whole groups");
#pragma unroll
            for (int g0 = 0; g0 < kPer; g0 += kGrp) {
                int j[kGrp], pos[kGrp];
#pragma unroll
                for (int u = 0; u < kGrp; ++u) {
                    j[u] = (int)(c0 + tid + (int64_t)(g0 + u) * NT - hc);
                    pos[u] = 0;
                }
                for (int st = top; st > 0; st >>= 1) {
#pragma unroll
                    for (int u = 0; u < kGrp; ++u) {
                        const int q = pos[u] + st - 1;
                        if (q < nseg && spre[q] <= j[u]) pos[u] += st;
                    }
                }
#pragma unroll
                for (int u = 0; u < kGrp; ++u) {
                    const int64_t i = c0 + tid + (int64_t)(g0 + u) * NT;
                    if (i >= n) {
                        v[g0 + u] = 0ull;
                    } else if (i < hc) {
                        v[g0 + u] = keys[i];
                    } else {
                        const int sg = pos[u];
                        const int off = j[u] - (sg > 0 ? spre[sg - 1] : 0);
                        v[g0 + u] = keys[a.head_span + (int64_t)sg * a.seg_cap + off];
                    }
                }
            }
        } else {
#pragma unroll
            for (int u = 0; u < kPer; ++u) {
                const int64_t i = c0 + tid + (int64_t)u * NT;
                const bool ok = i < n;
                if (u < kSpec && c0 == 0)
                    v[u] = ok ? v[u] : 0ull;
                else
                    v[u] = ok ? keys[i] : 0ull;
            }
        }
        merge_pass(S, v, k, tid, run, vpar);
    }
    auto out = [&](int r, uint64_t kk) {
        a.V[row * k + r] = key_value(kk);
        a.I[row * k + r] = key_index(kk) + a.f_offset;
    };
    if (a.ties)
        emit_topk<true>(S, k, tid, out);
    else
        emit_topk<false>(S, k, tid, out);
}

// Per row: top-k of a segmented list (main_kernel's, or mainl_kernel's
// without a head) -- a head of at most NT keys, then nseg segments of seg_cap
// slots, segment s holding seg_cnt[row * nseg + s] keys.  NT = SPLIT * kSlots
// threads; the SPLIT threads of slot t (threads SPLIT * t ..) read segments
// t, t + kSlots, ..., the keys in
// pairs dealt round-robin (pair j of a segment to thread j % SPLIT), kPer keys
// per thread and pass (16-byte loads, adjacent threads on adjacent pairs):
// no search for a key's segment, and every thread has its loads in flight at
// once.  Thread t also reads head key t.  The head key and the first kEager
// keys per thread of a segment (SPLIT * kEager keys) are loaded without
// waiting for the counts and masked afterwards.  A pass filters as
// merge_kernel's chunks.
// kWaves: the waves per SIMD the registers must allow (1: no bound).
// kHead false: the list has no head (head_span == 0, host).
template <int kPer, int kEager, int NT, int SPLIT, int kWaves, bool kHead>
__global__ __launch_bounds__(NT, kWaves) void merge_seg_kernel(MergeArgs a)
{
    static_assert(kPer % 2 == 0 && kEager % 2 == 0 && kEager <= kPer, "pairs of keys");
    static_assert(NT % SPLIT == 0, "whole slots");
    constexpr int kSlots = NT / SPLIT;
    constexpr int kStep = SPLIT * kPer;   // keys of a segment per pass
    __shared__ SelSharedT<NT> S;
    const int tid = threadIdx.x;
    const int slot = tid / SPLIT, part = tid % SPLIT;
    const int64_t row = blockIdx.x;
    if (merge_marked<NT>(a, row, tid)) return;
    const int k = a.k;
    const int nseg = a.nseg;
    const int64_t hs = kHead ? a.head_span : 0;   // <= NT (host)
    const uint64_t* keys = a.list_keys + row * a.list_cap;
    uint64_t v[kHead ? kPer + 1 : kPer];
    int hc = 0;
    if constexpr (kHead) {
        v[kPer] = tid < hs ? keys[tid] : 0ull;   // the head key rides in the first pass
        hc = hs > 0 ? a.list_cnt[row * kCntStride] : 0;
    }
    if (tid == 0) S.cnt = 0;
    uint64_t run = 0;
    uint32_t vpar = 0;   // block_any's call parity
    for (int s0 = 0; s0 < nseg || s0 == 0; s0 += kSlots) {
        const int sg = s0 + slot;
        const bool own = sg < nseg;
        // segment starts are 16-byte aligned (head_span and seg_cap even);
        // this thread's pair u / 2 of a pass starts at key base + SPLIT * u +
        // 2 * part of the segment
        const uint64_t* q = keys + hs + (int64_t)(own ? sg : 0) * a.seg_cap + 2 * part;
        u64x2 e[kEager / 2];
#pragma unroll
        for (int u = 0; u < kEager; u += 2) {
            e[u / 2] = u64x2{0ull, 0ull};
            if (own && SPLIT * u + 2 * part < a.seg_cap) e[u / 2] = *(const u64x2*)(q + SPLIT * u);
        }
        const int cnt = (own ? a.seg_cnt[row * nseg + sg] : 0) - 2 * part;
        if constexpr (kHead)
            if (s0 == 0 && tid >= hc) v[kPer] = 0ull;
        for (int base = 0;; base += kStep) {
#pragma unroll
            for (int u = 0; u < kPer; u += 2) {
                // a pair starting below the count lies inside the segment
                // (pair starts and seg_cap are even, the count <= seg_cap)
                const int o = base + SPLIT * u;
                u64x2 p = {0ull, 0ull};
                if (u < kEager && base == 0)
                    p = e[u / 2];
                else if (o < cnt)
                    p = *(const u64x2*)(q + o);
                v[u] = o < cnt ? p[0] : 0ull;
                v[u + 1] = o + 1 < cnt ? p[1] : 0ull;
            }
            merge_pass(S, v, k, tid, run, vpar);
            if constexpr (kHead) v[kPer] = 0ull;
            if (!block_any<NT / 64>(cnt > base + kStep - 2 * part, S.vote, vpar, tid >> 6, tid & 63)) break;
        }
    }
    emit_topk(S, k, tid, [&](int r, uint64_t kk) {
        a.V[row * k + r] = key_value(kk);
        a.I[row * k + r] = key_index(kk) + a.f_offset;
    });
}

// ---------------------------------------------------------------------------
// pack_kernel: the rows of nparts partial (B, k) results (values and global
// latent indices, e.g. one per W shard) as keys of a dense candidate list per
// row, for merge_kernel.  One workgroup per row.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kThreads) void pack_kernel(PackArgs a)
{
    const int64_t row = blockIdx.x;
    const int n = a.nparts * a.k;
    uint64_t* out = a.list_keys + row * a.list_cap;
    for (int j = threadIdx.x; j < n; j += kThreads) {
        const int part = j / a.k, r = j - part * a.k;
        const int64_t src = ((int64_t)part * a.B + row) * a.k + r;
        out[j] = make_key(a.V[src], a.I[src]);
    }
    if (threadIdx.x == 0) a.list_cnt[row * kCntStride] = n;
}

// ---------------------------------------------------------------------------
// fill_zero_kernel: n16 16-byte words at p set to zero, grid-stride.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kThreads) void fill_zero_kernel(u32x4* p, int64_t n16)
{
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n16; i += (int64_t)gridDim.x * kThreads)
        p[i] = u32x4{0u, 0u, 0u, 0u};
}

// ---------------------------------------------------------------------------
// read_probe_kernel: reads n16 16-byte words once and folds them (XOR) into
// *sink with one atomic per wave, so that no load can be elided.  The words
// are taken as 4 KiB rows; each workgroup owns a contiguous run of rows and
// reads them 256 rows at a time, one 128-byte line of each row per round (four
// nontemporal 16-byte loads per thread), two rounds in flight.  Of the plain
// read orders measured on MI355X (this one, 32 KiB contiguous per round, and
// 256-byte pieces of 128 rows), this one is the fastest, ~7.1 TB/s over 1 GiB:
// it is the HBM read rate the streaming kernels are compared with.  Words past
// the last whole row are read by workgroup 0.
// ---------------------------------------------------------------------------
constexpr int kProbeThreads = 512;
constexpr int kProbeRow = 256;   // 16-byte words per 4 KiB row

__global__ __launch_bounds__(kProbeThreads) void read_probe_kernel(const u32x4* p, int64_t n16, uint32_t* sink)
{
    const int tid = threadIdx.x;
    const int64_t nrows = n16 / kProbeRow;
    const int64_t per = (nrows + gridDim.x - 1) / gridDim.x;
    int64_t r0 = (int64_t)blockIdx.x * per, r1 = r0 + per;
    r0 = r0 < nrows ? r0 : nrows;
    r1 = r1 < nrows ? r1 : nrows;
    u32x4 acc = {0u, 0u, 0u, 0u};
    for (int64_t t0 = r0; t0 < r1; t0 += 256) {
        const int64_t nr = r1 - t0 < 256 ? r1 - t0 : 256;
        // round s: words 8s .. 8s+7 of each of the tile's rows; thread chunk c is
        // row c / 8, word c % 8 of the round.  Chunks of rows past the tile's end
        // load row 0 again (so that every load is unconditional) and are masked
        // out when folded.
        bool ok[4];
        int64_t off[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int c = tid + kProbeThreads * q;
            ok[q] = (c >> 3) < nr;
            off[q] = (t0 + (ok[q] ? (c >> 3) : 0)) * kProbeRow + (c & 7);
        }
        auto load = [&](u32x4 (&v)[4], int s) {
#pragma unroll
            for (int q = 0; q < 4; ++q) v[q] = __builtin_nontemporal_load(p + off[q] + 8 * s);
        };
        auto fold = [&](const u32x4 (&v)[4]) {
#pragma unroll
            for (int q = 0; q < 4; ++q) acc ^= ok[q] ? v[q] : u32x4{0u, 0u, 0u, 0u};
        };
        u32x4 va[4], vb[4];
        load(va, 0);
        load(vb, 1);
        for (int s = 2; s < kProbeRow / 8; s += 2) {
            fold(va);
            load(va, s);
            __syncthreads();
            fold(vb);
            load(vb, s + 1);
            __syncthreads();
        }
        fold(va);
        fold(vb);
    }
    if (blockIdx.x == 0)
        for (int64_t i = nrows * kProbeRow + tid; i < n16; i += kProbeThreads) acc ^= __builtin_nontemporal_load(p + i);
    uint32_t x = acc[0] ^ acc[1] ^ acc[2] ^ acc[3];
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) x ^= __shfl_xor(x, off, 64);
    if ((threadIdx.x & 63) == 0) atomicXor(sink, x);
}

// ---------------------------------------------------------------------------
// Host-side launch helpers
// ---------------------------------------------------------------------------
size_t main_lds_bytes(int NB, int cap, int lq)
{
    const size_t BT = 32 * (size_t)NB;
    const size_t rings = 2 * (size_t)kTileLatents * kXRowStride + 2 * BT * kXRowStride;   // TileStream rings
    return rings + BT * 8 + BT * 8 + 2 * kTileLatents * 4 + BT * (size_t)lq * 8 + (size_t)kMainWaves * cap * 8 +
           2 * kMainWaves * sizeof(uint32_t);
}

// LDS queue keys per row: the most (even, at most 64) whose LDS use, with
// global segments of cap = k + lq keys, fits 159 KiB of the workgroup's 160.
int main_lds_queue(int NB, int k)
{
    for (int lq = 64; lq >= 2; lq -= 2) {
        const int cap = (k + lq + 1) & ~1;
        if (main_lds_bytes(NB, cap, lq) <= 159 * 1024) return lq;
    }
    return 0;
}

template <int DT, int NB>
static hipError_t launch_main_t(const MainArgs& a, dim3 grid, hipStream_t st)
{
    const size_t lds = main_lds_bytes(NB, a.cap, a.lq);
    auto kern = main_kernel<DT, NB>;
    hipError_t e = ensure_lds((const void*)kern, lds);
    if (e != hipSuccess) return e;
    launch(kern, grid, dim3(kMainThreads), lds, st, a);
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

template <int DT, int NB>
static hipError_t launch_sample_t(const SampleArgs& a, dim3 grid, hipStream_t st)
{
    const size_t lds = sample_lds_bytes(NB);
    auto kern = sample_kernel<DT, NB>;
    hipError_t e = ensure_lds((const void*)kern, lds);
    if (e != hipSuccess) return e;
    launch(kern, grid, dim3(kSampleThreads), lds, st, a);
    return hipGetLastError();
}

hipError_t launch_sample(int dt, int NB, const SampleArgs& a, dim3 grid, hipStream_t st)
{
#define STK_CASE(DTV, NBV) \
    if (dt == DTV && NB == NBV) return launch_sample_t<DTV, NBV>(a, grid, st);
    STK_CASE(DT_BF16, 1) STK_CASE(DT_BF16, 2) STK_CASE(DT_BF16, 4)
    STK_CASE(DT_F16, 1) STK_CASE(DT_F16, 2) STK_CASE(DT_F16, 4)
    STK_CASE(DT_F32, 1) STK_CASE(DT_F32, 2) STK_CASE(DT_F32, 4)
#undef STK_CASE
    return hipErrorInvalidValue;
}

hipError_t launch_thr(const ThrArgs& a, int64_t rows, hipStream_t st)
{
    if (a.P != nullptr && a.nsamp == kSampleLarge) {
        // the larger sample on 512 threads (16 keys each): 27.9 -> 25.6 us
        // at B = 1024; the 4096-latent one gains nothing from it
        launch(thr_kernel<kSampleLarge / (2 * kThreads), 2 * kThreads>, dim3((unsigned)rows), dim3(2 * kThreads), 0, st, a);
        return hipGetLastError();
    }
    if (a.P != nullptr && a.nsamp != kSampleTarget) return hipErrorInvalidValue;
    launch(thr_kernel<kSampleTarget / kThreads, kThreads>, dim3((unsigned)rows), dim3(kThreads), 0, st, a);
    return hipGetLastError();
}

hipError_t launch_read_probe(const void* buf, int64_t n16, uint32_t* sink, int ncu, hipStream_t st)
{
    launch(read_probe_kernel, dim3((unsigned)ncu), dim3(kProbeThreads), 0, st, (const u32x4*)buf, n16, sink);
    return hipGetLastError();
}

hipError_t launch_fill_zero(void* p, size_t bytes, hipStream_t st)
{
    const int64_t n16 = (int64_t)(bytes / 16);
    int64_t wgs = (n16 + kThreads * 4 - 1) / (kThreads * 4);
    if (wgs > 4096) wgs = 4096;
    if (wgs < 1) wgs = 1;
    launch(fill_zero_kernel, dim3((unsigned)wgs), dim3(kThreads), 0, st, (u32x4*)p, n16);
    return hipGetLastError();
}

hipError_t launch_pack(const PackArgs& a, int64_t rows, hipStream_t st)
{
    launch(pack_kernel, dim3((unsigned)rows), dim3(kThreads), 0, st, a);
    return hipGetLastError();
}

hipError_t launch_merge(const MergeArgs& a, int64_t rows, hipStream_t st)
{
    // dense lists expected to exceed one 4096-slot chunk (spec 1): 32 slots
    // per thread (one chunk), the first 16 loaded ahead of the count; spec 0:
    // 16 slots per thread, which also keeps the registers low enough for four
    // workgroups per CU when the rows are many (large batches)
    if (a.spec == 1)
        launch(merge_kernel<32, 16, kThreads, 1>, dim3((unsigned)rows), dim3(kThreads), 0, st, a);
    else if (a.spec == 6)   // segments expected to hold up to ~3 keys: 8 per pass
        launch(merge_seg_kernel<4, 4, 2 * kThreads, 2, 1, true>, dim3((unsigned)rows), dim3(2 * kThreads), 0, st, a);
    else if (a.spec == 3)   // segments expected to hold up to ~12 keys: 32 per pass
        launch(merge_seg_kernel<16, 8, 2 * kThreads, 2, 1, true>, dim3((unsigned)rows), dim3(2 * kThreads), 0, st, a);
    else if (a.spec == 4)   // segments expected to hold up to ~24 keys: 48 per pass
        launch(merge_seg_kernel<24, 8, 2 * kThreads, 2, 1, true>, dim3((unsigned)rows), dim3(2 * kThreads), 0, st, a);
    else if (a.spec == 5)   // fuller segments: 64 per pass
        launch(merge_seg_kernel<32, 8, 2 * kThreads, 2, 1, true>, dim3((unsigned)rows), dim3(2 * kThreads), 0, st, a);
    else if (a.spec == 8)   // no head, few segments (a large batch's): 4 threads per segment, 64 keys
                            // per pass, four row workgroups per CU
        launch(merge_seg_kernel<16, 4, kThreads, 4, 4, false>, dim3((unsigned)rows), dim3(kThreads), 0, st, a);
    else
        launch(merge_kernel<16, 0, kThreads, 4>, dim3((unsigned)rows), dim3(kThreads), 0, st, a);
    return hipGetLastError();
}

}  // namespace stk
