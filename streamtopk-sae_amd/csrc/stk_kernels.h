// stk_kernels.h -- kernel argument blocks and host launch helpers shared by
// the kernels (stk_kernels.hip, stk_approx.hip) and the C ABI (stk_api.hip).
#pragma once
#include <hip/hip_ext.h>
#include "stk_select.h"

namespace stk {

// Events the next kernel launch of this thread records at the kernel's start
// and end, or null.  They ride in the kernel's dispatch packet
// (hipExtLaunchKernelGGL), so timing adds no packets, and no idle time,
// between kernels.
struct LaunchEvents {
    hipEvent_t start = nullptr, stop = nullptr;
};
LaunchEvents& launch_events();

// Raises `kern`'s dynamic-LDS limit to at least `lds` bytes on the current
// device.  The attribute call is made once per (kernel, device, larger size):
// later launches only look the pair up.
hipError_t ensure_lds(const void* kern, size_t lds);

// Every kernel of the library is launched through here.
template <class K, class... A>
inline void launch(K kern, dim3 grid, dim3 block, size_t lds, hipStream_t st, A... args)
{
    LaunchEvents& ev = launch_events();
    if (ev.start != nullptr) {
        hipExtLaunchKernelGGL(kern, grid, block, (uint32_t)lds, st, ev.start, ev.stop, 0u, args...);
        ev = LaunchEvents{};
    } else {
        hipLaunchKernelGGL(kern, grid, block, lds, st, args...);
    }
}

constexpr int kMainWaves = 8;        // wavefronts per main_kernel workgroup (2 per SIMD)
constexpr int kMainThreads = 64 * kMainWaves;
constexpr int kTileLatents = 32 * kMainWaves;   // latents per main_kernel tile
constexpr int kApproxGroup = 128;    // latent group of the approximate variant
constexpr int kGroupTile = 256;      // latents per group_kernel tile (two groups)
constexpr int kSampleTarget = 4096;  // sampled latents that seed the thresholds
constexpr int kSampleLarge = 8192;   //   (large batches with F >= kSampleLargeMinF)
constexpr int kSampleBlock = 128;    // consecutive latents per sampled block
constexpr int64_t kSampleMinF = 16384;
// The larger sample pays from F = 2^17: at B = 512, F = 65536 the 4096-latent
// sample makes the whole pass 4.5 % faster; at B = 1024..2048, F = 262144 the
// 8192-latent one does (its tighter threshold leaves half the candidates).
constexpr int64_t kSampleLargeMinF = 131072;

// Sampled latent i (0 <= i < nsamp) is latent
// (i / kSampleBlock) << blk_log2 + i % kSampleBlock: nsamp / kSampleBlock
// blocks of consecutive latents spread evenly over F.
__host__ __device__ inline int64_t sample_latent(int64_t i, int blk_log2)
{
    return ((i / kSampleBlock) << blk_log2) + (i % kSampleBlock);
}

// Whether latent f belongs to a sample of `nblocks` blocks.
__host__ __device__ inline bool is_sampled(int64_t f, int blk_log2, int nblocks)
{
    return (f & ((int64_t(1) << blk_log2) - 1)) < kSampleBlock && (f >> blk_log2) < nblocks;
}

struct MainArgs {
    const void* X;
    const void* W;
    const float* bias;
    int64_t B, d, F;
    int k, cap;
    int64_t num_tiles, tiles_per_wg;
    const uint64_t* thr0;        // per-row starting threshold keys, or null
    int sampled;                 // non-zero: the sampled latents (is_sampled) were
    int samp_log2, samp_blocks;  //   scored by the sample pass and are skipped here
    uint64_t* list_keys;         // [B][list_cap]: row r's head (head_span slots, the
    int64_t list_cap, head_span; //   sample's top k; none with the exchange), then one
                                 //   segment of cap keys per workgroup (gridDim.x of them)
    int32_t* seg_cnt;            // [B][gridDim.x] keys each workgroup left in its segment
    int lq;                      // LDS queue keys per row (even, <= 64; cap >= k + lq)
    int max_rounds;              // bound of the epilogue's spill-and-retry loop
    uint64_t* err;               // set to the call's tag if that bound is ever reached
    const uint32_t* epoch;       // the workspace's call count: this call's tag is *epoch + 1
    uint64_t* cur;               // receives the call's tag (for the merge's error check)
    // Threshold exchange (xch != 0; then thr0 is null and nothing is sampled):
    // after its first tile every workgroup publishes each row's largest score
    // of that tile, the owner of a row takes the k-th largest of those maxima
    // as the row's threshold, and every workgroup reads its rows' thresholds
    // before its first epilogue filters anything.  Each word: the call's tag
    // tag << 32 | a score image (ordered_u32).
    int xch;
    uint64_t* xmax;              // [nbc][32*NB][gridDim.x] each workgroup's row maxima
    uint64_t* xthr;              // [nbc][32*NB] row thresholds (owner x: rows x, x + gridDim.x, ...)
    int64_t xwait;               // s_memrealtime ticks a wave polls for words before going
                                 //   on without the exchanged thresholds (threshold 0)
    uint32_t* xto;               // incremented by every poll that runs out with xwait > 0
                                 //   (the word after the error word; never reset)
};

// Row blocks of main_kernel whose workgroups exchange thresholds need at
// least this many workgroups (an owner workgroup handles its rows one wave
// each: at most 128 / kXchMinWg <= kMainWaves rows).
constexpr int kXchMinWg = 16;
// Every workspace starts with a control line (kCtlBytes): the epoch (u32 at
// 0: calls completed on this workspace, advanced by each exact call's merge),
// the exchange's count of polls that ran out (u32 at 4), the error word (u64
// at 8) and the running call's tag (u64 at 16).  Only the exact path's
// kernels write it; every other buffer of every entry point (the shard
// merge's lists, the candidate path's group heads) starts past it.
//
// A call's tag is epoch + 1, in [1, kTagPeriod]: the epoch runs modulo
// kTagPeriod, so a tag is never 0 and differs from the tags of the previous
// kTagPeriod - 1 calls on the workspace, whatever their shapes, also when the
// call is a replay of a captured graph (whose kernel arguments never change).
// A tag sits in the high half of a 64-bit word, and every such half any
// kernel writes to a workspace is either a tag or outside [1, kTagPeriod]:
//   - sort keys: the image of an fp32 score (ordered_u32), at least
//     0x007FFFFF (-inf) for every value, or 0 (empty);
//   - counts (lists, segments): at most 2^20, and the high half of a word
//     only where another count is its low half, which, read as a score
//     image, lies below every real score (a maximum or threshold that low
//     only admits more candidates);
//   - the sample pass's partial sums (fp32): denormals are stored as zero,
//     so a positive one is at least 0x00800000.
// The merge zeroes the exchange words its call used, so a tag that comes
// round again after kTagPeriod calls meets no word of its earlier use; the
// streaming kernel clears an error word that holds another call's tag.
constexpr size_t kCtlBytes = 256;
constexpr uint32_t kTagPeriod = (1u << 22) - 1;

// This call's tag from the workspace's epoch (reduced modulo the period, so
// that even a corrupted epoch yields a tag in range).
__device__ __forceinline__ uint32_t call_tag(const uint32_t* epoch)
{
    return *epoch % kTagPeriod + 1u;
}

// The epoch as a vector load, for kernels that need the tag only after
// their first tile: issued at the start, it overlaps the first loads of W
// instead of stalling the first wait on the scalar counter, which every
// kernel-argument load shares.  call_tag_of turns it into the tag.
__device__ __forceinline__ uint32_t load_epoch(const uint32_t* epoch)
{
    return __hip_atomic_load(epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ uint32_t call_tag_of(uint32_t epoch)
{
    return (uint32_t)__builtin_amdgcn_readfirstlane((int)(epoch % kTagPeriod + 1u));
}

// Clears an error word that holds another call's tag (it may come round
// again); a workgroup of this call that sets the word meanwhile keeps it.
__device__ __forceinline__ void clear_stale_err(uint64_t* err, uint32_t tag)
{
    const uint64_t e = __hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (e != 0ull && e != (uint64_t)tag) atomicCAS((unsigned long long*)err, (unsigned long long)e, 0ull);
}

// 500 us at the 100 MHz s_memrealtime clock: ~30x the longest wait measured
// (the skew of the first tile's end over the grid plus two round trips,
// under 15 us), so reached only if some workgroups were not resident (another
// kernel holding CUs).  The exchange's words are read only after
// their tag matches the call's; a workspace must therefore be zero-filled
// before its first use (tag 0 is never a call's).
constexpr int64_t kXchWaitTicks = 50000;

// Row r's head count is list_cnt[r * kCntStride]: one 128-byte line per row.
constexpr int kCntStride = 32;

// The spill-and-retry loops of the streaming kernels end after a bounded
// number of rounds.  The bounds are never reached (main_kernel places at least
// lq >= 8 of a row's <= 256 pending scores per round, mainl_kernel at least
// cap - k >= 64), so they only guard against a broken invariant: reaching one
// sets the workspace's error word to the call's tag, and the merge of that
// call then marks every row of its output (indices -1, values NaN) instead of
// returning a silently wrong result.  A word holding another call's tag (or
// zero) means no error: nothing has to clear it between calls.
// The test-only stk_test_set_hooks(max_rounds = n) allows n spill rounds
// instead (it forces that path from the host; 0: none).
constexpr int kMainMaxRounds = 4096;
constexpr int kMainLMaxRounds = 1 << 20;

constexpr int kSampleWaves = 8;      // wavefronts per sample_kernel workgroup
constexpr int kSampleThreads = 64 * kSampleWaves;
constexpr int kSampleSteps = 8;      // d-steps per sample_kernel workgroup (at most)
constexpr int kSampleLat = 64;       // sampled latents per sample_kernel workgroup

struct SampleArgs {
    const void* X;
    const void* W;
    int64_t B, d;
    int samp_log2, nsamp;
    int nsplit;                  // d ranges (splits) of the sample pass
    float* P;                    // partial scores of the sampled latents: split s,
    int64_t p_row, p_split;      //   row j, sample i at P[j * p_row + s * p_split + i]
};

struct ThrArgs {
    const float* P;              // sampled scores, or null (no sample: threshold 0):
    int64_t p_row, p_split;      //   nsplit partial sums (layout as in SampleArgs)
    int nsplit;                  //   added in split order, then
    const float* bias;           //   + bias[latent] if non-null
    int samp_log2, nsamp, k;
    uint64_t* thr;               // [B] row threshold keys
    uint64_t* list_keys;         // [B][list_cap]: receives the sampled keys >= thr
    int32_t* list_cnt;           // [B * kCntStride] set to the number of those keys
    int64_t list_cap;
};

// Large-batch streaming kernel: 256 rows x 256 latents per tile, queues in
// global memory (one segment of `cap` keys per row and W range).
constexpr int kLargeRows = 256;
constexpr int kLargeThreads = 256;
constexpr int64_t kLargeMinB = 512;   // batches from this size use mainl_kernel
constexpr int kLXchPerWg = 4;         // exchanged maxima per row and mainl_kernel workgroup

struct MainLArgs {
    const void* X;
    const void* W;
    const float* bias;
    int64_t B, d, F;
    int k, cap;
    int64_t num_tiles, tiles_per_wg;
    int nbc, nr;                 // row blocks, W ranges (grid = nbc * nr)
    const uint64_t* thr0;        // per-row starting threshold keys
    int sampled, samp_log2, samp_blocks;
    uint64_t* list_keys;         // [B][list_cap]: head_span head slots, then nr segments of cap
    int64_t list_cap, head_span;
    int32_t* seg_cnt;            // [B][nr] keys in each segment
    int max_rounds;              // bound of the overflow loop (see kMainLMaxRounds)
    uint64_t* err;               // set to the call's tag if that bound is ever reached
    const uint32_t* epoch;       // as MainArgs's
    uint64_t* cur;
    // Threshold exchange (xch != 0; then thr0 is null and nothing is sampled),
    // as MainArgs's, with kLXchPerWg maxima per row and workgroup (one per 64
    // latents of the first tile).  Tagged words as MainArgs's.
    int xch;
    int xnr;                     // W ranges that hold tiles (the first xnr; the rest are empty
                                 //   when F is small): only they publish and own rows
    uint64_t* xmax;              // [nbc][kLargeRows][xnr * kLXchPerWg]
    uint64_t* xthr;              // [nbc][kLargeRows]
    int64_t xwait;
    uint32_t* xto;
    // sample mode (mainl_sample_kernel): 256-latent tiles of the sampled
    // latents, d split in ksplit ranges; raw partial scores to P
    int ksplit, nsamp;
    float* P;                    // split s, row j, sample i at P[j * p_row + s * p_split + i]
    int64_t p_row, p_split;
};

// A row's candidates: slots [0, head_span) hold list_cnt[row * kCntStride] keys at their
// front; then nseg segments of seg_cap slots, segment s holding
// seg_cnt[row * nseg + s] keys at its front.  With nseg == 0 the row is the
// dense list [0, list_cnt[row * kCntStride]).
constexpr int kMergeMaxSeg = 256;   // merge_kernel's segments per row (mainl_kernel's W ranges)

struct MergeArgs {
    const uint64_t* list_keys;   // [B][list_cap]
    const int32_t* list_cnt;     // [B * kCntStride]
    int64_t list_cap, head_span;
    int nseg, seg_cap;
    const int32_t* seg_cnt;      // [B][nseg]
    int k;
    int spec;                    // 0: merge_kernel, chunks of 16 candidates per thread;
                                 //   1: merge_kernel for a dense list expected to hold more
                                 //   than 4096 candidates (32 per thread and chunk);
                                 //   6, 3, 4, 5: merge_seg_kernel (head <= 256 keys, two
                                 //   threads per segment; 8, 32, 48 or 64 keys per pass);
                                 //   8: merge_seg_kernel for a list without a head, four
                                 //   threads per segment, 64 keys per pass, 256 threads
    int32_t f_offset;            // added to every emitted index (a shard's first latent)
    int ties;                    // non-zero: keys may repeat (stk_topk_merge's parts); equal keys
                                 //   take consecutive ranks
    const uint64_t* err;         // equal to *cur (this call's tag): mark the output rows
    const uint64_t* cur;         //   (-1, NaN); both null for stk_topk_merge
    uint32_t* epoch;             // advanced by one modulo kTagPeriod (workgroup 0), or null
    uint64_t* xmax;              // the threshold exchange's words of this call, zeroed by
    int64_t xmax_row;            //   the merge: row r's maxima xmax[r * xmax_row ..
    uint64_t* xthr;              //   + xmax_row) and its threshold xthr[r]; null without
    float* V;
    int32_t* I;
};

struct PackArgs {                // partial top-k results -> dense candidate lists
    const float* V;              // [nparts][B][k]
    const int32_t* I;            // [nparts][B][k] latent indices
    int64_t B;
    int k, nparts;
    uint64_t* list_keys;         // [B][list_cap]
    int32_t* list_cnt;           // [B * kCntStride]
    int64_t list_cap;
};

struct GroupArgs {               // approximate variant, per-group top-c candidates
    const void* X;
    const void* W;
    const float* bias;
    int64_t B, d, F;
    int c;
    int64_t num_groups, tiles_per_wg;
    float* cand_vals;            // [B][num_groups][c]
    int32_t* cand_idxs;          // [B][num_groups][c]
    uint64_t* heads;             // [B][num_groups] each group's first candidate as a key (0: none)
};

struct CandArgs {                // approximate variant, top-k over the candidates
    const float* cand_vals;
    const int32_t* cand_idxs;
    const uint64_t* heads;       // [B][num_groups] as GroupArgs::heads
    int64_t num_groups;          // candidates per row: num_groups * c, each group's in descending order
    int c, k;
    float* V;
    int32_t* I;
};

size_t main_lds_bytes(int NB, int cap, int lq);
int main_lds_queue(int NB, int k);
size_t mainl_lds_bytes(int cap);
size_t group_lds_bytes(int NB);

hipError_t launch_main(int dt, int NB, const MainArgs& a, dim3 grid, hipStream_t st);
hipError_t launch_mainl(int dt, const MainLArgs& a, int grid, hipStream_t st);
hipError_t launch_mainl_sample(int dt, const MainLArgs& a, int grid, hipStream_t st);
hipError_t launch_sample(int dt, int NB, const SampleArgs& a, dim3 grid, hipStream_t st);
hipError_t launch_thr(const ThrArgs& a, int64_t rows, hipStream_t st);
hipError_t launch_merge(const MergeArgs& a, int64_t rows, hipStream_t st);
hipError_t launch_pack(const PackArgs& a, int64_t rows, hipStream_t st);
hipError_t launch_group(int dt, int NB, const GroupArgs& a, dim3 grid, hipStream_t st);
hipError_t launch_cand(const CandArgs& a, int64_t rows, hipStream_t st);
hipError_t launch_read_probe(const void* buf, int64_t n16, uint32_t* sink, int ncu, hipStream_t st);
// Zero-fills `bytes` (a multiple of 16) at 16-byte aligned `p` with a kernel (no memset node).
hipError_t launch_fill_zero(void* p, size_t bytes, hipStream_t st);

}  // namespace stk
