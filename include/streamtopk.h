/*
 * streamtopk.h -- C ABI of libstreamtopk_hip.so, the MI355X (gfx950) streaming
 * fused top-k SAE encoder.
 *
 * It replaces the reference's pybind11 module `streamtopk_sae_native`
 * (streamtopk_sae/csrc/bindings.cpp:28-51) and the CUDA/C++ sources behind it.
 * Plain pointers and sizes only: the caller owns every buffer (inputs, outputs
 * and the device workspace), so the library never allocates device memory.
 *
 * Conventions shared by every entry point:
 *   - Return 0 on success; a non-zero STK_E_* code on failure, with a
 *     thread-local message from stk_last_error().  Argument errors carry the
 *     reference's TORCH_CHECK wording (streamtopk_exact.cu:794-830,
 *     streamtopk_approx.cu:243-284, streamtopk_cpu.cpp:87-122).
 *   - X is (B, d) row-major, W is (F, d) row-major, both of `dtype`; b is (F,)
 *     fp32.  V is (B, k) fp32 and I is (B, k) int32, each row sorted by value
 *     descending; equal values are ordered by lower latent index first.
 *   - Device entry points run asynchronously on `stream` (a hipStream_t, NULL
 *     for the legacy default stream) on the current HIP device; all pointers
 *     must be device pointers on that device, 16-byte aligned.
 *   - A workspace must be zero-filled before its first use (hipMemset once,
 *     when it is allocated), and again after a call on it returned an error;
 *     every successful call leaves it valid for the next call of any shape,
 *     also when the calls are replays of a captured HIP graph.  Calls that
 *     overlap in time must not share a workspace.  One workspace may serve
 *     exact, approximate and shard-merge calls in turn.  (The exact path's
 *     workgroups exchange per-row thresholds through words tagged with the
 *     call's number, kept in the workspace's first 256 bytes -- which only
 *     exact calls write -- and advanced by each exact call on the device,
 *     modulo 2^22 - 1; zero is never a call's tag, and each call's merge
 *     zeroes the words it tagged.)
 */
#ifndef STREAMTOPK_H
#define STREAMTOPK_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define STK_ABI_VERSION 1

/* dtype codes for X and W */
#define STK_DTYPE_F32 0
#define STK_DTYPE_F16 1
#define STK_DTYPE_BF16 2

/* return codes */
#define STK_OK 0
#define STK_E_INVALID 1      /* argument rejected before any device work */
#define STK_E_HIP 2          /* a HIP runtime call or launch failed */
#define STK_E_WORKSPACE 3    /* workspace missing or smaller than required */

/* ABI version of the loaded library (STK_ABI_VERSION it was built with). */
int stk_abi_version(void);

/* Message of the last failed call on this thread ("" if none). */
const char* stk_last_error(void);

/* Device workspace (bytes) that stk_exact_forward needs for this problem on
 * the current device.  Replaces the temporaries the reference allocates with
 * libtorch inside launch_exact (streamtopk_exact.cu:686-689). */
int stk_exact_workspace_bytes(int64_t B, int64_t d, int64_t F, int64_t k, int dtype,
                              size_t* out_bytes);

/* Exact encode: V, I = top_k(X @ W.T + b, k) without a (B, F) buffer.
 * Replaces streamtopk_cuda_exact_forward (streamtopk_exact.cu:788-833),
 * bound in the reference at bindings.cpp:33 and called from ops.py:57.
 * k must be one of 1,2,4,8,16,32,64,128 and <= F; d <= 4096; d must be a
 * multiple of 8 (fp16/bf16) or 4 (fp32), so that rows are 16-byte aligned (the
 * kernels mask a partial last 128-byte d-step; the Python op zero-pads other
 * d).  If a streaming kernel ever exhausted its bounded spill-and-retry loop
 * (which its bounds rule out), every output row is marked instead of being
 * returned short: indices -1, values NaN. */
int stk_exact_forward(const void* X, const void* W, const float* b, float* V, int32_t* I,
                      int64_t B, int64_t d, int64_t F, int64_t k, int dtype,
                      void* workspace, size_t workspace_bytes, void* stream);

/* Bytes of the static device scratch stk_exact_forward_noalloc works in. */
#define STK_NOALLOC_SCRATCH_BYTES (64u << 20)

/* stk_exact_forward without a workspace, for callers that cannot allocate
 * device memory: code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc.  No counterpart in the reference.  The workspace is
 * a static device array of STK_NOALLOC_SCRATCH_BYTES in the library's code
 * object, held by every device that runs this entry point until the process
 * ends; the call allocates nothing and records no profiling events.  A
 * problem whose stk_exact_workspace_bytes exceeds the array is rejected with
 * STK_E_WORKSPACE before any device work: batches of up to 256 rows fit for
 * any d <= 4096, k <= 128 and F (BASELINE configs 1-3 need 12-28 MB);
 * batches of 512 rows and more (config 4) do not.  All calls on one device
 * share its array, so calls that overlap on one device race: serialise them
 * (one stream, or events between streams).  Results are identical to
 * stk_exact_forward's. */
int stk_exact_forward_noalloc(const void* X, const void* W, const float* b, float* V, int32_t* I,
                              int64_t B, int64_t d, int64_t F, int64_t k, int dtype, void* stream);

/* Exact encode of one shard of W: W and b hold latents f_offset ..
 * f_offset + F - 1 of a larger dictionary, and I receives those global
 * indices (local index + f_offset).  Otherwise identical to
 * stk_exact_forward, with the same workspace (stk_exact_workspace_bytes for
 * the shard's F).  No counterpart in the reference, which runs one device
 * (device 0's attributes, streamtopk_exact.cu:658): it is the per-GPU part of
 * an F-sharded encoder, whose per-shard results stk_topk_merge combines.
 * Requires 0 <= f_offset and f_offset + F <= 2^31 - 1. */
int stk_exact_forward_shard(const void* X, const void* W, const float* b, float* V, int32_t* I,
                            int64_t B, int64_t d, int64_t F, int64_t k, int dtype, int64_t f_offset,
                            void* workspace, size_t workspace_bytes, void* stream);

/* Device workspace (bytes) for stk_topk_merge. */
int stk_topk_merge_workspace_bytes(int64_t B, int64_t k, int64_t nparts, size_t* out_bytes);

/* Top-k of nparts partial top-k results: Vp / Ip are (nparts, B, k) fp32
 * values and int32 global indices, e.g. the stk_exact_forward_shard outputs
 * of W's shards gathered on one device; V / I receive each row's top k of
 * the nparts * k candidates, in the library's order (value descending, then
 * lower index first).  No counterpart in the reference (see
 * stk_exact_forward_shard).  k as for stk_exact_forward; nparts >= 1 and
 * nparts * k <= 2^20. */
int stk_topk_merge(const float* Vp, const int32_t* Ip, int64_t nparts, int64_t B, int64_t k,
                   float* V, int32_t* I, void* workspace, size_t workspace_bytes, void* stream);

/* Device workspace (bytes) for stk_approx_forward.  `with_candidates` is
 * non-zero when the caller passes a candidate buffer (then the workspace holds
 * 256 bytes, then each group's first candidate as an 8-byte key:
 * 256 + B * ceil(F/128) * 8 bytes). */
int stk_approx_workspace_bytes(int64_t B, int64_t d, int64_t F, int64_t k, int64_t c, int dtype,
                               int with_candidates, size_t* out_bytes);

/* Approximate encode: top-k of the union of each 128-latent group's top-c.
 * Replaces streamtopk_cuda_approx_forward (streamtopk_approx.cu:234-291) plus
 * the final torch.topk/gather the reference runs in Python (ops.py:75-81).
 * c must be one of 16,32,64,128 and k <= c.  cand_vals / cand_idxs are
 * optional (B, ceil(F/128), c) outputs (NULL to skip): each group's top-c,
 * descending, padded with (-FLT_MAX, -1) -- the reference's candidate_buffer
 * side effect (streamtopk_approx.cu:264-274). */
int stk_approx_forward(const void* X, const void* W, const float* b, float* V, int32_t* I,
                       int64_t B, int64_t d, int64_t F, int64_t k, int64_t c, int dtype,
                       float* cand_vals, int32_t* cand_idxs,
                       void* workspace, size_t workspace_bytes, void* stream);

/* CPU encode on host memory, fp32 only, OpenMP over rows (num_threads <= 0:
 * the OpenMP default).  Replaces streamtopk_cpu_forward
 * (streamtopk_cpu.cpp:81-125), bound at bindings.cpp:29 and called from
 * ops.py:40.  Output rows are sorted descending (the reference leaves k=128
 * rows in heap order, topk_buffer.hpp:9). */
int stk_cpu_forward(const float* X, const float* W, const float* b, float* V, int32_t* I,
                    int64_t B, int64_t d, int64_t F, int64_t k, int num_threads);

/* Plain HBM read stream (no counterpart in the reference; used by bench.py to
 * report the streaming kernels' bandwidth as a fraction of a measured read
 * stream): reads `bytes` (a multiple of 16) from the 16-byte aligned device
 * buffer `buf` once (as 4 KiB rows, one 128-byte line of each of 256 rows
 * per round, nontemporal loads: the fastest plain read order measured), and XORs a digest of
 * it into *sink (a device uint32), asynchronously on `stream`.  Timed under
 * the name "read_probe". */
int stk_read_probe(const void* buf, size_t bytes, uint32_t* sink, void* stream);

/* Per-kernel timing (no counterpart in the reference; used by bench.py).
 * While enabled, every device entry point called on this thread records the
 * start and end of the kernels it launches with a HIP event pair carried in
 * each kernel's own dispatch packet (hipExtLaunchKernelGGL), which adds no
 * work or idle time between kernels: every kernel for on=1, only the
 * streaming kernels (main_kernel, mainl_kernel, group_kernel; read back as
 * "main_kernel" / "group_kernel") for on=2.  Enabling discards earlier
 * records; on=0 stops recording and frees the events. */
int stk_profile_enable(int on);

/* Total milliseconds and number of launches recorded for `kernel`
 * ("sample_kernel", "thr_kernel", "main_kernel", "merge_kernel",
 * "group_kernel", "cand_kernel", "read_probe") since profiling was enabled.
 * Waits for the recorded events to complete. */
int stk_profile_read(const char* kernel, double* total_ms, int64_t* launches);

#ifdef __cplusplus
}
#endif

#endif /* STREAMTOPK_H */
