// stk_api.hip -- the C ABI (include/streamtopk.h): argument validation with the
// reference's error wording, launch planning for the current device, and the
// kernel sequence of each entry point.  No device memory is allocated here:
// every temporary lives in the caller's workspace.
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <atomic>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/streamtopk.h"
#include "stk_internal.h"
#include "stk_kernels.h"

namespace stk {

static thread_local std::string g_err;

int set_error(int code, const char* fmt, ...)
{
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}

void clear_error() { g_err.clear(); }

bool k_supported(int64_t k)
{
    return k == 1 || k == 2 || k == 4 || k == 8 || k == 16 || k == 32 || k == 64 || k == 128;
}

static int hip_fail(hipError_t e, const char* what)
{
    return set_error(STK_E_HIP, "%s failed: %s", what, hipGetErrorString(e));
}

// ---------------------------------------------------------------------------
// Optional per-kernel event timing (stk_profile_enable / stk_profile_read).
// ---------------------------------------------------------------------------
struct ProfRec {
    const char* name;
    hipEvent_t a, b;
};
static thread_local int g_prof = 0;   // 0 off, 1 every kernel, 2 streaming kernels only
static thread_local std::vector<ProfRec> g_recs;
static thread_local std::vector<hipEvent_t> g_pool;

static hipEvent_t prof_event()
{
    if (!g_pool.empty()) {
        hipEvent_t e = g_pool.back();
        g_pool.pop_back();
        return e;
    }
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    return e;
}

LaunchEvents& launch_events()
{
    static thread_local LaunchEvents ev;
    return ev;
}

// Arms the next kernel launch to record a start/stop event pair (in its own
// dispatch packet) under `name`.
static int prof_begin(const char* name, hipStream_t)
{
    if (!g_prof) return -1;
    if (g_prof == 2 && std::strcmp(name, "main_kernel") != 0 && std::strcmp(name, "group_kernel") != 0) return -1;
    ProfRec r{name, prof_event(), prof_event()};
    if (!r.a || !r.b) return -1;
    launch_events() = LaunchEvents{r.a, r.b};
    g_recs.push_back(r);
    return (int)g_recs.size() - 1;
}

// Disarms the events if the launch did not take them (it failed first): the
// record is dropped so reading it cannot wait on an event never recorded.
static void prof_end(int idx, hipStream_t)
{
    LaunchEvents& ev = launch_events();
    if (ev.start != nullptr) {
        ev = LaunchEvents{};
        if (idx >= 0 && idx + 1 == (int)g_recs.size()) {
            g_pool.push_back(g_recs.back().a);
            g_pool.push_back(g_recs.back().b);
            g_recs.pop_back();
        }
    }
}

static void prof_release()
{
    for (auto& r : g_recs) { g_pool.push_back(r.a); g_pool.push_back(r.b); }
    g_recs.clear();
}

// Dynamic-LDS limits already raised, per (kernel, device).
struct LdsLimit {
    const void* kern;
    int dev;
    size_t lds;
};
static std::mutex g_lds_mu;
static std::vector<LdsLimit> g_lds;

hipError_t ensure_lds(const void* kern, size_t lds)
{
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    std::lock_guard<std::mutex> lock(g_lds_mu);
    for (LdsLimit& l : g_lds) {
        if (l.kern != kern || l.dev != dev) continue;
        if (l.lds >= lds) return hipSuccess;
        e = hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e == hipSuccess) l.lds = lds;
        return e;
    }
    e = hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e == hipSuccess) g_lds.push_back(LdsLimit{kern, dev, lds});
    return e;
}

// Compute units of the current device (queried once per device).
static int cu_count(int* out)
{
    static int cache[64] = {0};
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
    if (dev >= 0 && dev < 64 && cache[dev] > 0) { *out = cache[dev]; return 0; }
    int n = 0;
    e = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev);
    if (e != hipSuccess) return hip_fail(e, "hipDeviceGetAttribute");
    if (n <= 0) n = 1;
    if (dev >= 0 && dev < 64) cache[dev] = n;
    *out = n;
    return 0;
}

// ---------------------------------------------------------------------------
// Test hooks (stk_test_set_hooks, exported for the test suite and not
// declared in include/streamtopk.h): they force paths that real inputs never
// take -- the sample pass at shapes that would exchange thresholds, a retry
// bound low enough to be reached, exchange waits that run out.  Set from the
// host, read once per call; the defaults are the product's behaviour.
// ---------------------------------------------------------------------------
struct TestHooks {
    int no_xch = 0;              // non-zero: never take the threshold exchange
    int max_rounds = -1;         // >= 0: the streaming kernels' retry bound
    int64_t xch_wait = kXchWaitTicks;   // the exchange's poll bound in ticks (0: one
                                        // poll; < 0: none, every threshold 0)
};
static std::mutex g_hooks_mu;
static TestHooks g_hooks;

static TestHooks test_hooks()
{
    std::lock_guard<std::mutex> lock(g_hooks_mu);
    return g_hooks;
}

static int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }
static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }
static int ilog2_floor(int64_t x) { int l = 0; while ((x >> (l + 1)) > 0) ++l; return l; }

// ---------------------------------------------------------------------------
// Exact-path plan
// ---------------------------------------------------------------------------
struct ExactPlan {
    bool large;                  // mainl_kernel (B >= kLargeMinB) instead of main_kernel
    bool xch;                    // main_kernel exchanges thresholds after its first tile (no sample pass)
    int NB, cap, lq;             // lq: main_kernel's LDS queue keys per row
    int64_t nbc, num_tiles, tpw;
    int nwg;                     // main_kernel: W ranges; mainl_kernel: nr (grid = nbc * nr)
    bool sample;
    int samp_log2, nsamp;        // sampled latents: nsamp / kSampleBlock blocks, 1 << samp_log2 apart
    int ksplit;                  // d ranges (splits) of the sample pass
    int snb;                     // sample_kernel: 32-row tiles per workgroup
    int64_t list_cap, head_span;
    int64_t expect_seg;          // keys a segment is expected to receive (merge pass width)
    size_t off_thr, off_list, off_lcnt, off_seg, off_xmax, off_xthr, total;
};

static ExactPlan make_exact_plan(int64_t B, int64_t d, int64_t F, int64_t k, int dtype, int ncu,
                                 const TestHooks& hooks)
{
    ExactPlan p;
    p.num_tiles = cdiv(F, kTileLatents);
    p.large = B >= kLargeMinB;
    p.lq = 0;
    if (p.large) {
        // 256-row blocks; W ranges a multiple of 8 so each range's row blocks share an XCD
        p.NB = kLargeRows / 32;
        p.cap = (int)(k + 64 < 192 ? k + 64 : 192);
        if (p.cap & 1) ++p.cap;
        p.nbc = cdiv(B, kLargeRows);
        int64_t nr = ncu / p.nbc;
        if (nr < 1) nr = 1;
        if (nr >= 8) nr &= ~(int64_t)7;
        if (nr > kMergeMaxSeg) nr = kMergeMaxSeg;   // merge_kernel's segments per row
        p.tpw = cdiv(p.num_tiles, nr);
        p.nwg = (int)nr;
    } else {
        const int64_t bblocks = cdiv(B > 0 ? B : 1, 32);
        p.NB = (int)(bblocks < 4 ? bblocks : 4);
        if (p.NB == 3) p.NB = 4;
        p.nbc = cdiv(B, 32 * p.NB);
        int64_t nwg = ncu / (p.nbc > 0 ? p.nbc : 1);
        if (nwg < 1) nwg = 1;
        if (nwg > p.num_tiles) nwg = p.num_tiles;
        p.tpw = cdiv(p.num_tiles, nwg);
        p.nwg = (int)cdiv(p.num_tiles, p.tpw);
    }

    // The thresholds come from the streaming kernel's own first tiles (each
    // row's k-th largest of the n maxima its workgroups publish, each over m
    // latents: n = nwg, m = 256 below 512 rows; n = kLXchPerWg * W ranges,
    // m = 64 above) or from a sample pass of nsamp latents (whose k-th is the
    // threshold).  A latent passes the exchange's threshold with probability
    // about -ln(1 - k / n) / m and the sample's about k / nsamp.  The exchange
    // is taken when it passes at most as many (up to twice as many below 512
    // rows, where it also saves the two launches of the sample and threshold
    // passes, a larger share of the call); it needs n > k (n = k is the
    // minimum of all maxima) and, below 512 rows, at least kXchMinWg
    // workgroups.  Measured (B = 512-2048, d = 2048-4096, k = 64-128): the
    // exchange was 3-8 % faster where it passes fewer latents, 1-4 % slower
    // where it passes ~1.4x as many, and up to 2x slower at n = k.
    // (The no_xch test hook selects the sample pass.)
    const int samp_n = (p.large && F >= kSampleLargeMinF) ? kSampleLarge : kSampleTarget;
    {
        // mainl_kernel: the W ranges that hold tiles (main_kernel has no empty workgroup)
        const int64_t nfull = p.large ? cdiv(p.num_tiles, p.tpw) : p.nwg;
        const int64_t n = p.large ? nfull * kLXchPerWg : p.nwg;
        const double m = p.large ? 64.0 : 256.0;
        // n = k still bounds the k-th score; without a sample pass (small F)
        // that weak bound beats none.  Only workgroups with a first tile take
        // part (mainl_kernel's W ranges past the last tile are empty when F is
        // small); they publish the maxima and own the rows.
        bool ok = (F < kSampleMinF ? n >= k : n > k) &&
                  (p.large ? n <= 512 : (p.nwg >= kXchMinWg && p.nwg <= 256));
        if (ok && F >= kSampleMinF) {
            const double px = -std::log1p(-(double)k / (double)n) / m;
            const double ps = (double)k / (double)samp_n;
            ok = px <= (p.large ? 1.0 : 2.0) * ps;
        }
        p.xch = ok && !hooks.no_xch;
    }
    p.sample = F >= kSampleMinF && !p.xch;
    p.samp_log2 = 0;
    p.nsamp = 0;
    if (p.sample) {
        // large batches take a twice larger sample: a tighter threshold halves
        // the candidates their (compute-bound) epilogue and merge handle
        p.nsamp = samp_n;
        p.samp_log2 = ilog2_floor(F / (p.nsamp / kSampleBlock));
    }
    // large batches score the sample with mainl_kernel's sample mode: one
    // workgroup per (row block, 256 sampled latents, d range), enough d
    // ranges to fill the device
    p.ksplit = 1;
    p.snb = 1;
    const int64_t nds = cdiv(d, dtype == STK_DTYPE_F32 ? 32 : 64);   // d-steps, the last maybe partial
    if (p.large && p.sample) {
        const int64_t wgs = p.nbc * (p.nsamp / kTileLatents);
        int64_t ks = cdiv(ncu, wgs);
        if (ks > nds) ks = nds;
        if (ks < 1) ks = 1;
        p.ksplit = (int)ks;
    } else if (p.sample) {
        // small batches: sample_kernel, one workgroup per (64 sampled
        // latents, row block of up to 128 rows, d range of at most
        // kSampleSteps steps); more d ranges while that leaves CUs idle
        const int64_t bblocks = cdiv(B, 32);
        p.snb = bblocks >= 3 ? 4 : (int)bblocks;
        const int64_t wgs = (p.nsamp / kSampleLat) * cdiv(B, 32 * p.snb);
        int64_t ks = cdiv(ncu, wgs);
        if (ks > nds) ks = nds;
        if (ks < cdiv(nds, kSampleSteps)) ks = cdiv(nds, kSampleSteps);
        p.ksplit = (int)ks;
    }
    if (!p.large) {
        // main_kernel's LDS queue: room for about twice the survivors a
        // workgroup expects per row (the scores above the sample's k-th,
        // k * F / nsamp per row, spread over the workgroups), up to what fits
        // next to its rings; without a sample every score passes at first and
        // the queue takes all the room there is.
        // With the exchange, a row's threshold is the k-th largest of nwg
        // maxima over 256 latents each: a latent passes with probability
        // about -ln(1 - k / nwg) / 256, so a workgroup expects
        // -ln(1 - k / nwg) * tpw survivors per row.
        const int lq_max = main_lds_queue(p.NB, (int)k);
        int lq = lq_max;
        p.expect_seg = p.cap;
        if (p.sample || p.xch) {
            int64_t expect;
            if (p.xch) {
                const double q = std::fmin((double)k / (double)p.nwg, 0.9);
                expect = (int64_t)std::ceil(-std::log1p(-q) * (double)p.tpw);
            } else {
                expect = cdiv(k * F / p.nsamp, p.nwg);
            }
            p.expect_seg = expect;
            const int64_t want = (2 * expect + 8 + 1) & ~(int64_t)1;
            if (want < lq) lq = (int)want;
        }
        p.lq = lq;
        p.cap = (int)((k + p.lq + 1) & ~(int64_t)1);
        if (!p.sample && !p.xch) p.expect_seg = p.cap;
    } else {
        p.expect_seg = p.cap;
    }
    // Each row's list: a head (the sample's top k; with a sample larger than
    // the selection buffer, every sampled key that reaches its first bound),
    // then one segment of cap keys per workgroup of the streaming kernel.
    // The sample pass's partial sums of the row live in the segment area:
    // they are dead (read by thr_kernel) before the first segment is written.
    if (!p.sample)
        p.head_span = 0;
    else if (p.nsamp <= kSelCap)
        p.head_span = (k + 1) & ~(int64_t)1;
    else
        p.head_span = p.nsamp;
    int64_t seg_keys = (int64_t)p.nwg * p.cap;
    const int64_t p_keys = p.sample ? ((int64_t)p.ksplit * p.nsamp + 1) / 2 : 0;
    if (p_keys > seg_keys) seg_keys = p_keys;
    p.list_cap = (p.head_span + seg_keys + 1) & ~(int64_t)1;
    size_t off = kCtlBytes;   // the control line (epoch, timeouts, error word, tag) at 0
    p.off_thr = off;
    off = align256(off + (size_t)B * 8);
    p.off_lcnt = off;
    off = align256(off + (size_t)B * 4 * kCntStride);
    p.off_seg = off;
    off = align256(off + (size_t)B * p.nwg * 4);
    p.off_list = off;
    off = align256(off + (size_t)B * p.list_cap * 8);
    p.off_xmax = p.off_xthr = off;
    if (p.xch) {
        // [nbc][bt][words per row]
        const size_t bt = p.large ? (size_t)kLargeRows : 32 * (size_t)p.NB;
        const size_t per_row = p.large ? (size_t)cdiv(p.num_tiles, p.tpw) * kLXchPerWg : (size_t)p.nwg;
        p.off_xmax = off;
        off = align256(off + (size_t)p.nbc * bt * per_row * 8);
        p.off_xthr = off;
        off = align256(off + (size_t)p.nbc * bt * 8);
    }
    p.total = off;
    return p;
}

static int check_dtype(int dtype)
{
    if (dtype != STK_DTYPE_F32 && dtype != STK_DTYPE_F16 && dtype != STK_DTYPE_BF16)
        return set_error(STK_E_INVALID, "X dtype must be fp32, fp16, or bf16");
    return 0;
}

static int check_shape_common(int64_t B, int64_t d, int64_t F, int dtype)
{
    if (B < 0 || d < 1 || F < 1) return set_error(STK_E_INVALID, "invalid shape: B=%lld d=%lld F=%lld",
                                                  (long long)B, (long long)d, (long long)F);
    if (F > 0x7FFFFFFELL) return set_error(STK_E_INVALID, "F=%lld exceeds the int32 index range", (long long)F);
    // rows are read in 16-byte chunks (8 fp16/bf16 or 4 fp32 elements); a d
    // that is not a whole number of 128-byte d-steps ends in a partial step
    // whose chunks past d read as zeros
    const int64_t q = (dtype == STK_DTYPE_F32) ? 4 : 8;
    if (d % q)
        return set_error(STK_E_INVALID,
                         "d=%lld must be a multiple of %lld for %s inputs (pad X and W_enc with zero columns)",
                         (long long)d, (long long)q, dtype == STK_DTYPE_F32 ? "fp32" : "fp16/bf16");
    return 0;
}

static int check_ptrs(const void* X, const void* W, const void* b, const void* V, const void* I)
{
    if (!X || !W || !b || !V || !I) return set_error(STK_E_INVALID, "null tensor pointer");
    if (((uintptr_t)X | (uintptr_t)W) & 15) return set_error(STK_E_INVALID, "X and W_enc must be 16-byte aligned");
    if ((uintptr_t)b & 3) return set_error(STK_E_INVALID, "b_enc must be 4-byte aligned");
    return 0;
}

static int validate_exact(int64_t B, int64_t d, int64_t F, int64_t k, int dtype)
{
    int rc;
    if ((rc = check_dtype(dtype))) return rc;
    if (B < 0 || d < 1 || F < 1) return check_shape_common(B, d, F, dtype);
    if (k < 1 || k > F) return set_error(STK_E_INVALID, "k out of range");
    if (d > 4096) return set_error(STK_E_INVALID, "d exceeds D_MAX=4096");
    if (!k_supported(k))
        return set_error(STK_E_INVALID, "streamtopk_cuda_exact: unsupported k=%lld. Supported: 1,2,4,8,16,32,64,128.",
                         (long long)k);
    return check_shape_common(B, d, F, dtype);
}

// Runs sample -> thr -> main -> merge on `st`.
static int run_exact(const ExactPlan& p, const TestHooks& hooks, const void* X, const void* W, const float* b,
                     float* V, int32_t* I, int64_t B, int64_t d, int64_t F, int64_t k, int dtype, unsigned char* ws,
                     hipStream_t st, int64_t f_offset = 0)
{
    const int dt = dtype;   // STK_DTYPE_* and DT_* share values
    hipError_t e;
    uint64_t* thr = (uint64_t*)(ws + p.off_thr);
    uint64_t* list_keys = (uint64_t*)(ws + p.off_list);
    int32_t* list_cnt = (int32_t*)(ws + p.off_lcnt);
    int32_t* seg_cnt = (int32_t*)(ws + p.off_seg);
    // the control line: epoch (u32), poll timeouts (u32), error word, call tag
    uint32_t* epoch = (uint32_t*)ws;
    uint32_t* xto = epoch + 1;
    uint64_t* err = (uint64_t*)(ws + 8);
    uint64_t* cur = (uint64_t*)(ws + 16);
    // test hooks: a lower retry bound; the exchange's wait in ticks (0: one
    // poll, < 0: none -- the paths of workgroups that were never resident)
    const int max_rounds = hooks.max_rounds;
    const int64_t xwait = hooks.xch_wait;
    // the sample's partial sums: in each row's segment area, split after split
    float* P = p.sample ? (float*)(list_keys + p.head_span) : nullptr;
    const int64_t p_row = 2 * p.list_cap, p_split = p.nsamp;
    if (p.sample && p.large) {
        MainLArgs sl;
        std::memset(&sl, 0, sizeof sl);
        sl.X = X; sl.W = W; sl.bias = b; sl.B = B; sl.d = d; sl.F = F;
        sl.k = (int)k; sl.cap = p.cap;
        sl.nbc = (int)p.nbc;
        sl.samp_log2 = p.samp_log2;
        sl.ksplit = p.ksplit;
        sl.nsamp = p.nsamp;
        sl.P = P;
        sl.p_row = p_row;
        sl.p_split = p_split;
        const int grid = (int)(p.nbc * (p.nsamp / kTileLatents) * p.ksplit);
        int pi = prof_begin("sample_kernel", st);
        e = launch_mainl_sample(dt, sl, grid, st);
        prof_end(pi, st);
        if (e != hipSuccess) return hip_fail(e, "sample launch");
    } else if (p.sample) {
        SampleArgs sa;
        sa.X = X; sa.W = W; sa.B = B; sa.d = d;
        sa.samp_log2 = p.samp_log2;
        sa.nsamp = p.nsamp;
        sa.nsplit = p.ksplit;
        sa.P = P;
        sa.p_row = p_row;
        sa.p_split = p_split;
        const dim3 grid((unsigned)(p.nsamp / kSampleLat * p.ksplit), (unsigned)cdiv(B, 32 * p.snb));
        int pi = prof_begin("sample_kernel", st);
        e = launch_sample(dt, p.snb, sa, grid, st);
        prof_end(pi, st);
        if (e != hipSuccess) return hip_fail(e, "sample_kernel launch");
    }
    if (!p.xch) {
        ThrArgs ta;
        ta.P = P;
        ta.p_row = p_row;
        ta.p_split = p_split;
        ta.nsplit = p.ksplit;
        ta.bias = b;
        ta.samp_log2 = p.samp_log2; ta.nsamp = p.nsamp; ta.k = (int)k;
        ta.thr = thr; ta.list_keys = list_keys; ta.list_cnt = list_cnt; ta.list_cap = p.list_cap;
        int pt = prof_begin("thr_kernel", st);
        e = launch_thr(ta, B, st);
        prof_end(pt, st);
        if (e != hipSuccess) return hip_fail(e, "thr_kernel launch");
    }
    MergeArgs mg;
    if (p.large) {
        MainLArgs ml;
        std::memset(&ml, 0, sizeof ml);
        ml.X = X; ml.W = W; ml.bias = b; ml.B = B; ml.d = d; ml.F = F;
        ml.k = (int)k; ml.cap = p.cap;
        ml.num_tiles = p.num_tiles; ml.tiles_per_wg = p.tpw;
        ml.nbc = (int)p.nbc; ml.nr = p.nwg;
        ml.thr0 = p.xch ? nullptr : thr;
        ml.sampled = p.sample ? 1 : 0;
        ml.samp_log2 = p.samp_log2;
        ml.samp_blocks = p.nsamp / kSampleBlock;
        ml.list_keys = list_keys; ml.list_cap = p.list_cap; ml.head_span = p.head_span;
        ml.seg_cnt = seg_cnt;
        ml.max_rounds = max_rounds >= 0 ? max_rounds : kMainLMaxRounds;
        ml.err = err;
        ml.epoch = epoch;
        ml.cur = cur;
        ml.xch = p.xch ? 1 : 0;
        ml.xnr = (int)cdiv(p.num_tiles, p.tpw);
        ml.xmax = (uint64_t*)(ws + p.off_xmax);
        ml.xthr = (uint64_t*)(ws + p.off_xthr);
        ml.xwait = xwait;
        ml.xto = xto;
        int pm = prof_begin("main_kernel", st);
        e = launch_mainl(dt, ml, (int)(p.nbc * p.nwg), st);
        prof_end(pm, st);
        if (e != hipSuccess) return hip_fail(e, "mainl_kernel launch");
        mg.list_keys = list_keys; mg.list_cnt = list_cnt; mg.list_cap = p.list_cap;
        mg.head_span = p.head_span; mg.nseg = p.nwg; mg.seg_cap = p.cap; mg.seg_cnt = ml.seg_cnt;
        // without a head (the exchange) the segments are read in place, four
        // threads each; else each key's segment is searched for over the
        // counts' prefix sums
        mg.spec = p.head_span == 0 ? 8 : 0;
    } else {
        MainArgs ma;
        std::memset(&ma, 0, sizeof ma);
        ma.X = X; ma.W = W; ma.bias = b; ma.B = B; ma.d = d; ma.F = F;
        ma.k = (int)k; ma.cap = p.cap;
        ma.num_tiles = p.num_tiles; ma.tiles_per_wg = p.tpw;
        ma.thr0 = p.xch ? nullptr : thr;
        ma.sampled = p.sample ? 1 : 0;
        ma.samp_log2 = p.samp_log2;
        ma.samp_blocks = p.nsamp / kSampleBlock;
        ma.list_keys = list_keys; ma.list_cap = p.list_cap; ma.head_span = p.head_span;
        ma.seg_cnt = seg_cnt;
        ma.lq = p.lq;
        ma.max_rounds = max_rounds >= 0 ? max_rounds : kMainMaxRounds;
        ma.err = err;
        ma.epoch = epoch;
        ma.cur = cur;
        ma.xch = p.xch ? 1 : 0;
        ma.xmax = (uint64_t*)(ws + p.off_xmax);
        ma.xthr = (uint64_t*)(ws + p.off_xthr);
        ma.xwait = xwait;
        ma.xto = xto;
        int pm = prof_begin("main_kernel", st);
        e = launch_main(dt, p.NB, ma, dim3((unsigned)p.nwg, (unsigned)p.nbc), st);
        prof_end(pm, st);
        if (e != hipSuccess) return hip_fail(e, "main_kernel launch");
        mg.list_keys = list_keys; mg.list_cnt = list_cnt; mg.list_cap = p.list_cap;
        mg.head_span = p.head_span; mg.nseg = p.nwg; mg.seg_cap = p.cap; mg.seg_cnt = seg_cnt;
        // the head holds at most k keys (nsamp <= kSelCap) or none: two
        // merge threads per segment, read in place, in passes of 8 keys where
        // a segment expects at most ~3 (the exchange at c1 and c2), of 32 up
        // to ~12, of 48 up to ~24, else of 64
        const int64_t per_seg = p.expect_seg;
        mg.spec = per_seg <= 3 ? 6 : per_seg <= 12 ? 3 : per_seg <= 24 ? 4 : 5;
    }
    mg.k = (int)k;
    mg.f_offset = (int32_t)f_offset;
    mg.err = err;
    mg.cur = cur;
    mg.epoch = epoch;
    // the exchange's words of this call, zeroed by the merge: row r's maxima
    // at xmax + r * (words per row), its threshold at xthr + r
    mg.xmax = p.xch ? (uint64_t*)(ws + p.off_xmax) : nullptr;
    mg.xthr = p.xch ? (uint64_t*)(ws + p.off_xthr) : nullptr;
    mg.xmax_row = p.xch ? (p.large ? cdiv(p.num_tiles, p.tpw) * kLXchPerWg : (int64_t)p.nwg) : 0;
    mg.ties = 0;   // one encode's keys are distinct
    mg.V = V; mg.I = I;
    const int pg = prof_begin("merge_kernel", st);
    e = launch_merge(mg, B, st);
    prof_end(pg, st);
    if (e != hipSuccess) return hip_fail(e, "merge_kernel launch");
    return 0;
}

// ---------------------------------------------------------------------------
// Approximate-path plan (candidate buffer requested)
// ---------------------------------------------------------------------------
struct GroupPlan {
    int NB;
    int64_t nbc, num_groups, tpw;
    int nwg;
};

static GroupPlan make_group_plan(int64_t B, int64_t F, int ncu)
{
    GroupPlan p;
    const int64_t bblocks = cdiv(B > 0 ? B : 1, 32);
    p.NB = (int)(bblocks < 4 ? bblocks : 4);
    if (p.NB == 3) p.NB = 4;
    p.nbc = cdiv(B, 32 * p.NB);
    p.num_groups = cdiv(F, kApproxGroup);
    const int64_t num_tiles = cdiv(p.num_groups, 2);
    int64_t nwg = ncu / (p.nbc > 0 ? p.nbc : 1);
    if (nwg < 1) nwg = 1;
    if (nwg > num_tiles) nwg = num_tiles;
    p.tpw = cdiv(num_tiles, nwg);
    p.nwg = (int)cdiv(num_tiles, p.tpw);
    return p;
}

static int validate_approx(int64_t B, int64_t d, int64_t F, int64_t k, int64_t c, int dtype)
{
    int rc;
    if ((rc = check_dtype(dtype))) return rc;
    if (k < 1 || k > c) return set_error(STK_E_INVALID, "k must be <= c");
    if (c != 16 && c != 32 && c != 64 && c != 128)
        return set_error(STK_E_INVALID, "streamtopk_cuda_approx: unsupported c=%lld. Supported: 16,32,64,128.",
                         (long long)c);
    if ((rc = check_shape_common(B, d, F, dtype))) return rc;
    if (k > F) return set_error(STK_E_INVALID, "k out of range");
    return 0;
}

// ---------------------------------------------------------------------------
// Static scratch of stk_exact_forward_noalloc
// ---------------------------------------------------------------------------
// The exact path's workspace for callers that cannot allocate: a file-scope
// array in the code object, so every device that runs the entry point holds
// its own copy until the process ends.  In host code `scratch` names a
// host-side stand-in, not a device address: each device's address comes from
// hipGetSymbolAddress, resolved once per device with that device current,
// and only that address is handed to kernels.  Nothing in it needs to start
// at zero: every count and key a kernel reads is written earlier in the same
// call (thr_kernel or the exchange each row's threshold, thr_kernel the head
// counts, main_kernel every segment count), and the words compared with the
// call's tag (the exchange's words, the error word) never hold it before the
// call writes them: the tag is the epoch of the control line + 1, zero at
// load, advanced by every call.
__attribute__((used)) static __device__ __align__(256) unsigned char scratch[STK_NOALLOC_SCRATCH_BYTES];

static std::mutex g_scratch_mu;
static void* g_scratch_ptr[64];   // per device
static std::atomic<bool> g_scratch_dirty[64];   // per device: zero-fill before the next call

static int scratch_ptr(void** out, int* out_dev)
{
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
    if (dev < 0 || dev >= 64) return set_error(STK_E_INVALID, "device %d out of range", dev);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch_ptr[dev] == nullptr) {
        void* ptr = nullptr;
        e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(scratch)");
        if (ptr == nullptr || ((uintptr_t)ptr & 255))
            return set_error(STK_E_HIP, "hipGetSymbolAddress(scratch) returned an unusable address %p", ptr);
        g_scratch_ptr[dev] = ptr;
    }
    *out = g_scratch_ptr[dev];
    *out_dev = dev;
    return 0;
}

}  // namespace stk

using namespace stk;

extern "C" {

int stk_abi_version(void) { return STK_ABI_VERSION; }

const char* stk_last_error(void) { return g_err.c_str(); }

int stk_exact_workspace_bytes(int64_t B, int64_t d, int64_t F, int64_t k, int dtype, size_t* out_bytes)
{
    clear_error();
    if (!out_bytes) return set_error(STK_E_INVALID, "null out_bytes");
    int rc = validate_exact(B, d, F, k, dtype);
    if (rc) return rc;
    int ncu = 0;
    if ((rc = cu_count(&ncu))) return rc;
    *out_bytes = (B == 0) ? 0 : make_exact_plan(B, d, F, k, dtype, ncu, test_hooks()).total;
    return 0;
}

int stk_exact_forward(const void* X, const void* W, const float* b, float* V, int32_t* I,
                      int64_t B, int64_t d, int64_t F, int64_t k, int dtype,
                      void* workspace, size_t workspace_bytes, void* stream)
{
    clear_error();
    int rc = validate_exact(B, d, F, k, dtype);
    if (rc) return rc;
    if (B == 0) return 0;
    if ((rc = check_ptrs(X, W, b, V, I))) return rc;
    int ncu = 0;
    if ((rc = cu_count(&ncu))) return rc;
    const TestHooks hooks = test_hooks();
    const ExactPlan p = make_exact_plan(B, d, F, k, dtype, ncu, hooks);
    if (!workspace || workspace_bytes < p.total)
        return set_error(STK_E_WORKSPACE, "workspace of %zu bytes is smaller than the %zu bytes required",
                         workspace ? workspace_bytes : (size_t)0, p.total);
    if ((uintptr_t)workspace & 255) return set_error(STK_E_INVALID, "workspace must be 256-byte aligned");
    return run_exact(p, hooks, X, W, b, V, I, B, d, F, k, dtype, (unsigned char*)workspace, (hipStream_t)stream);
}

int stk_exact_forward_noalloc(const void* X, const void* W, const float* b, float* V, int32_t* I,
                              int64_t B, int64_t d, int64_t F, int64_t k, int dtype, void* stream)
{
    clear_error();
    int rc = validate_exact(B, d, F, k, dtype);
    if (rc) return rc;
    if (B == 0) return 0;
    if ((rc = check_ptrs(X, W, b, V, I))) return rc;
    int ncu = 0;
    if ((rc = cu_count(&ncu))) return rc;
    const TestHooks hooks = test_hooks();
    const ExactPlan p = make_exact_plan(B, d, F, k, dtype, ncu, hooks);
    if (p.total > (size_t)STK_NOALLOC_SCRATCH_BYTES)
        return set_error(STK_E_WORKSPACE,
                         "this problem needs %zu bytes of workspace, more than the %zu-byte static scratch of "
                         "stk_exact_forward_noalloc; call stk_exact_forward with a workspace",
                         p.total, (size_t)STK_NOALLOC_SCRATCH_BYTES);
    void* ws = nullptr;
    int dev = 0;
    if ((rc = scratch_ptr(&ws, &dev))) return rc;
    const hipStream_t st = (hipStream_t)stream;
    // A call that failed after its first launch may have left words tagged
    // with a tag its merge never retired (the epoch did not advance): the
    // scratch is zero-filled (a fill kernel, no memset node) before it is
    // used again.
    if (g_scratch_dirty[dev].load()) {
        const hipError_t e = launch_fill_zero(ws, STK_NOALLOC_SCRATCH_BYTES, st);
        if (e != hipSuccess) return hip_fail(e, "scratch fill launch");
        g_scratch_dirty[dev].store(false);
    }
    // no profiling events either (creating one may allocate)
    const int prof = g_prof;
    g_prof = 0;
    rc = run_exact(p, hooks, X, W, b, V, I, B, d, F, k, dtype, (unsigned char*)ws, st);
    g_prof = prof;
    if (rc) g_scratch_dirty[dev].store(true);
    return rc;
}

int stk_exact_forward_shard(const void* X, const void* W, const float* b, float* V, int32_t* I,
                            int64_t B, int64_t d, int64_t F, int64_t k, int dtype, int64_t f_offset,
                            void* workspace, size_t workspace_bytes, void* stream)
{
    clear_error();
    if (f_offset < 0 || f_offset > 0x7FFFFFFELL)
        return set_error(STK_E_INVALID, "f_offset=%lld out of range", (long long)f_offset);
    int rc = validate_exact(B, d, F, k, dtype);
    if (rc) return rc;
    if (f_offset + F > 0x7FFFFFFFLL)
        return set_error(STK_E_INVALID, "f_offset + F = %lld exceeds the int32 index range",
                         (long long)(f_offset + F));
    if (B == 0) return 0;
    if ((rc = check_ptrs(X, W, b, V, I))) return rc;
    int ncu = 0;
    if ((rc = cu_count(&ncu))) return rc;
    const TestHooks hooks = test_hooks();
    const ExactPlan p = make_exact_plan(B, d, F, k, dtype, ncu, hooks);
    if (!workspace || workspace_bytes < p.total)
        return set_error(STK_E_WORKSPACE, "workspace of %zu bytes is smaller than the %zu bytes required",
                         workspace ? workspace_bytes : (size_t)0, p.total);
    if ((uintptr_t)workspace & 255) return set_error(STK_E_INVALID, "workspace must be 256-byte aligned");
    return run_exact(p, hooks, X, W, b, V, I, B, d, F, k, dtype, (unsigned char*)workspace, (hipStream_t)stream,
                     f_offset);
}

static int validate_merge(int64_t B, int64_t k, int64_t nparts)
{
    if (B < 0) return set_error(STK_E_INVALID, "invalid shape: B=%lld", (long long)B);
    if (k < 1 || !k_supported(k))
        return set_error(STK_E_INVALID, "unsupported k=%lld. Supported: 1,2,4,8,16,32,64,128.", (long long)k);
    if (nparts < 1 || nparts * k > (1 << 20))
        return set_error(STK_E_INVALID, "nparts=%lld out of range (1 <= nparts, nparts * k <= 2^20)",
                         (long long)nparts);
    return 0;
}

// Merge workspace: past the control line (which only the exact path
// writes: a workspace shared with exact calls keeps its epoch), the dense
// candidate lists (nparts*k keys per row), then the per-row counts.
static size_t merge_ws_lcnt(int64_t B, int64_t k, int64_t nparts)
{
    return kCtlBytes + (((size_t)B * (size_t)(nparts * k) * 8 + 255) & ~(size_t)255);
}

int stk_topk_merge_workspace_bytes(int64_t B, int64_t k, int64_t nparts, size_t* out_bytes)
{
    clear_error();
    if (!out_bytes) return set_error(STK_E_INVALID, "null out_bytes");
    int rc = validate_merge(B, k, nparts);
    if (rc) return rc;
    *out_bytes = (B == 0) ? 0 : merge_ws_lcnt(B, k, nparts) + (size_t)B * kCntStride * 4;
    return 0;
}

int stk_topk_merge(const float* Vp, const int32_t* Ip, int64_t nparts, int64_t B, int64_t k,
                   float* V, int32_t* I, void* workspace, size_t workspace_bytes, void* stream)
{
    clear_error();
    int rc = validate_merge(B, k, nparts);
    if (rc) return rc;
    if (B == 0) return 0;
    if (!Vp || !Ip || !V || !I) return set_error(STK_E_INVALID, "null tensor pointer");
    if (((uintptr_t)Vp | (uintptr_t)Ip | (uintptr_t)V | (uintptr_t)I) & 3)
        return set_error(STK_E_INVALID, "values and indices must be 4-byte aligned");
    const size_t need = merge_ws_lcnt(B, k, nparts) + (size_t)B * kCntStride * 4;
    if (!workspace || workspace_bytes < need)
        return set_error(STK_E_WORKSPACE, "workspace of %zu bytes is smaller than the %zu bytes required",
                         workspace ? workspace_bytes : (size_t)0, need);
    if ((uintptr_t)workspace & 255) return set_error(STK_E_INVALID, "workspace must be 256-byte aligned");
    unsigned char* ws = (unsigned char*)workspace;
    const hipStream_t st = (hipStream_t)stream;
    PackArgs pa;
    pa.V = Vp; pa.I = Ip; pa.B = B; pa.k = (int)k; pa.nparts = (int)nparts;
    pa.list_keys = (uint64_t*)(ws + kCtlBytes);
    pa.list_cnt = (int32_t*)(ws + merge_ws_lcnt(B, k, nparts));
    pa.list_cap = nparts * k;
    hipError_t e = launch_pack(pa, B, st);
    if (e != hipSuccess) return hip_fail(e, "pack_kernel launch");
    MergeArgs mg;
    std::memset(&mg, 0, sizeof mg);
    mg.list_keys = pa.list_keys; mg.list_cnt = pa.list_cnt; mg.list_cap = pa.list_cap;
    mg.head_span = pa.list_cap; mg.nseg = 0; mg.seg_cap = 1; mg.seg_cnt = nullptr;
    mg.spec = nparts * k > 4096 ? 1 : 0;
    mg.k = (int)k;
    mg.f_offset = 0;
    mg.err = nullptr;
    mg.ties = 1;   // the parts may repeat a latent
    mg.V = V; mg.I = I;
    const int pg = prof_begin("merge_kernel", st);
    e = launch_merge(mg, B, st);
    prof_end(pg, st);
    if (e != hipSuccess) return hip_fail(e, "merge_kernel launch");
    return 0;
}

int stk_approx_workspace_bytes(int64_t B, int64_t d, int64_t F, int64_t k, int64_t c, int dtype,
                               int with_candidates, size_t* out_bytes)
{
    clear_error();
    if (!out_bytes) return set_error(STK_E_INVALID, "null out_bytes");
    int rc = validate_approx(B, d, F, k, c, dtype);
    if (rc) return rc;
    if (B == 0) { *out_bytes = 0; return 0; }
    // with a candidate buffer: past the control line, the groups' head keys,
    // B x ceil(F / 128) words
    if (with_candidates) {
        *out_bytes = kCtlBytes + align256((size_t)B * cdiv(F, kApproxGroup) * 8);
        return 0;
    }
    int ncu = 0;
    if ((rc = cu_count(&ncu))) return rc;
    *out_bytes = make_exact_plan(B, d, F, k, dtype, ncu, test_hooks()).total;
    return 0;
}

int stk_approx_forward(const void* X, const void* W, const float* b, float* V, int32_t* I,
                       int64_t B, int64_t d, int64_t F, int64_t k, int64_t c, int dtype,
                       float* cand_vals, int32_t* cand_idxs,
                       void* workspace, size_t workspace_bytes, void* stream)
{
    clear_error();
    int rc = validate_approx(B, d, F, k, c, dtype);
    if (rc) return rc;
    if (B == 0) return 0;
    if ((rc = check_ptrs(X, W, b, V, I))) return rc;
    if ((cand_vals == nullptr) != (cand_idxs == nullptr))
        return set_error(STK_E_INVALID, "cand_vals and cand_idxs must both be given or both be NULL");
    // group_kernel writes each group's candidates as 16-byte vectors
    if (((uintptr_t)cand_vals | (uintptr_t)cand_idxs) & 15)
        return set_error(STK_E_INVALID, "cand_vals and cand_idxs must be 16-byte aligned");
    int ncu = 0;
    if ((rc = cu_count(&ncu))) return rc;
    hipStream_t st = (hipStream_t)stream;
    if (cand_vals == nullptr) {
        // With k <= c, every one of the k best latents of a row is within the
        // top-c of its own group (fewer than k <= c latents of the row beat
        // it), so the union of the per-group top-c holds the exact top-k and
        // its top-k is exactly that set: the exact streaming path computes the
        // approximate result without materialising any candidate.
        const TestHooks hooks = test_hooks();
        const ExactPlan p = make_exact_plan(B, d, F, k, dtype, ncu, hooks);
        if (!workspace || workspace_bytes < p.total)
            return set_error(STK_E_WORKSPACE, "workspace of %zu bytes is smaller than the %zu bytes required",
                             workspace ? workspace_bytes : (size_t)0, p.total);
        if ((uintptr_t)workspace & 255) return set_error(STK_E_INVALID, "workspace must be 256-byte aligned");
        return run_exact(p, hooks, X, W, b, V, I, B, d, F, k, dtype, (unsigned char*)workspace, st);
    }
    const GroupPlan p = make_group_plan(B, F, ncu);
    // the group heads start past the control line (only the exact path
    // writes it: a workspace shared with exact calls keeps its epoch)
    const size_t heads_bytes = kCtlBytes + (size_t)B * p.num_groups * 8;
    if (!workspace || workspace_bytes < heads_bytes)
        return set_error(STK_E_WORKSPACE, "workspace of %zu bytes is smaller than the %zu bytes required",
                         workspace ? workspace_bytes : (size_t)0, heads_bytes);
    if ((uintptr_t)workspace & 255) return set_error(STK_E_INVALID, "workspace must be 256-byte aligned");
    GroupArgs ga;
    ga.X = X; ga.W = W; ga.bias = b; ga.B = B; ga.d = d; ga.F = F; ga.c = (int)c;
    ga.num_groups = p.num_groups; ga.tiles_per_wg = p.tpw;
    ga.cand_vals = cand_vals; ga.cand_idxs = cand_idxs;
    ga.heads = (uint64_t*)((unsigned char*)workspace + kCtlBytes);
    int pg = prof_begin("group_kernel", st);
    hipError_t e = launch_group(dtype, p.NB, ga, dim3((unsigned)p.nwg, (unsigned)p.nbc), st);
    prof_end(pg, st);
    if (e != hipSuccess) return hip_fail(e, "group_kernel launch");
    CandArgs ca;
    ca.cand_vals = cand_vals; ca.cand_idxs = cand_idxs;
    ca.heads = (const uint64_t*)((unsigned char*)workspace + kCtlBytes);
    ca.num_groups = p.num_groups; ca.c = (int)c; ca.k = (int)k; ca.V = V; ca.I = I;
    pg = prof_begin("cand_kernel", st);
    e = launch_cand(ca, B, st);
    prof_end(pg, st);
    if (e != hipSuccess) return hip_fail(e, "cand_kernel launch");
    return 0;
}

int stk_read_probe(const void* buf, size_t bytes, uint32_t* sink, void* stream)
{
    clear_error();
    if (!buf || !sink) return set_error(STK_E_INVALID, "null pointer");
    if (((uintptr_t)buf & 15) || (bytes & 15)) return set_error(STK_E_INVALID, "buf and bytes must be 16-byte aligned");
    if (bytes == 0) return 0;
    int ncu = 0;
    int rc;
    if ((rc = cu_count(&ncu))) return rc;
    hipStream_t st = (hipStream_t)stream;
    const int pi = prof_begin("read_probe", st);
    const hipError_t e = launch_read_probe(buf, (int64_t)(bytes / 16), sink, ncu, st);
    prof_end(pi, st);
    if (e != hipSuccess) return hip_fail(e, "read_probe launch");
    return 0;
}

// Test-only (not declared in include/streamtopk.h): sets the test hooks
// (TestHooks) for later calls of every thread.  no_xch != 0 never takes the
// threshold exchange; max_rounds >= 0 bounds the streaming kernels' retry
// loops (-1: the default bound); xch_wait is the exchange's poll bound in
// ticks of the 100 MHz counter (0: one poll, < 0: none).
int stk_test_set_hooks(int no_xch, int max_rounds, int64_t xch_wait)
{
    clear_error();
    std::lock_guard<std::mutex> lock(g_hooks_mu);
    g_hooks.no_xch = no_xch;
    g_hooks.max_rounds = max_rounds;
    g_hooks.xch_wait = xch_wait;
    return 0;
}

// Test-only (not declared in include/streamtopk.h): copies `bytes` between
// host memory and the current device's no-allocation scratch at byte offset
// `off` (write != 0: host -> scratch), synchronously, so that a test can
// plant stale contents and read the control line.
int stk_test_scratch_io(size_t off, void* host, size_t bytes, int write)
{
    clear_error();
    if (!host || off > (size_t)STK_NOALLOC_SCRATCH_BYTES || bytes > (size_t)STK_NOALLOC_SCRATCH_BYTES - off)
        return set_error(STK_E_INVALID, "scratch range out of bounds");
    void* ws = nullptr;
    int dev = 0;
    int rc = scratch_ptr(&ws, &dev);
    if (rc) return rc;
    unsigned char* p = (unsigned char*)ws + off;
    const hipError_t e = write ? hipMemcpy(p, host, bytes, hipMemcpyHostToDevice)
                               : hipMemcpy(host, p, bytes, hipMemcpyDeviceToHost);
    if (e != hipSuccess) return hip_fail(e, "hipMemcpy(scratch)");
    return 0;
}

int stk_profile_enable(int on)
{
    clear_error();
    if (on < 0 || on > 2) return set_error(STK_E_INVALID, "stk_profile_enable: mode must be 0, 1 or 2");
    prof_release();
    g_prof = on;
    if (!g_prof) {
        for (hipEvent_t e : g_pool) (void)hipEventDestroy(e);
        g_pool.clear();
    }
    return 0;
}

int stk_profile_read(const char* kernel, double* total_ms, int64_t* launches)
{
    clear_error();
    if (!kernel || !total_ms || !launches) return set_error(STK_E_INVALID, "null argument");
    double tot = 0.0;
    int64_t n = 0;
    for (auto& r : g_recs) {
        if (std::strcmp(r.name, kernel) != 0) continue;
        hipError_t e = hipEventSynchronize(r.b);
        if (e != hipSuccess) return hip_fail(e, "hipEventSynchronize");
        float ms = 0.f;
        e = hipEventElapsedTime(&ms, r.a, r.b);
        if (e != hipSuccess) return hip_fail(e, "hipEventElapsedTime");
        tot += ms;
        ++n;
    }
    *total_ms = tot;
    *launches = n;
    return 0;
}

}  // extern "C"
