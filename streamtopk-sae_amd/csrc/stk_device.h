// stk_device.h -- device-side building blocks for the streaming top-k encoder
// on gfx950 (CDNA4): sort keys, the MFMA score main loop, and the LDS layout
// of the staged X tile.
//
// Score layout.  A workgroup is 4 wavefronts of 64 lanes.  Each wavefront owns
// FRAGS blocks of 32 latents (W rows, the MFMA "A" operand) and NB blocks of
// 32 batch rows (X rows, the MFMA "B" operand), and accumulates the fp32
// scores W_blk . X_blk^T with v_mfma_f32_32x32x{16 bf16|16 f16|2 f32}.
//
// Permuted reduction axis.  One "d-step" covers 128 bytes of every W row
// (64 bf16/fp16 or 32 fp32 elements).  Lane l holds row (l % 32) of its block
// and the contiguous half h = l / 32 of the d-step: 64 bytes, fetched as four
// 16-byte loads ("quads").  The MFMA's reduction index k is paired with the
// physical d index through the same (lane-half, quad, element) map for both
// operands, so every product W[f,d]*X[j,d] is formed exactly once; only the
// order of the fp32 sum differs from a plain left-to-right dot product.
//
// Accumulator layout (checked on the GPU by tests/test_gpu_layout.py):
// register r of lane l holds row 8*(r/4) + 4*(l/32) + (r%4), column l % 32.
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
// Score main loop over d-steps [s_begin, s_end).
//   wrow[a]  : byte pointer to this lane's W row of block a, already offset by
//              the lane-half (h * 64 bytes); rows past F are clamped by the
//              caller to a valid row.
//   X        : batch rows b0 .. b0 + 32*NB - 1 (rows >= B staged as zeros).
//   xs0/xs1  : two LDS buffers of 32*NB rows x kXRowStride bytes.
// The caller's accumulators are added to (not cleared).
// Ends with a workgroup barrier, so the LDS buffers are free on return.
// ---------------------------------------------------------------------------
template <int DT, int NB, int FRAGS>
struct MainLoop {
    static constexpr int DS = Dt<DT>::DS;
    static constexpr int ES = Dt<DT>::esize;
    static constexpr int kQuadElems = DS / 8;       // elements per 16-byte quad
    static constexpr int kXChunks = NB;             // 16-byte X chunks per thread per d-step

    const unsigned char* wrow[FRAGS];
    const unsigned char* X;
    int64_t B, d, b0;
    int lane, h;

    __device__ __forceinline__ void load_w(u32x4 (&w)[FRAGS][4], int64_t s) const
    {
        const bool full = (s + 1) * DS <= d;
#pragma unroll
        for (int a = 0; a < FRAGS; ++a)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int64_t e0 = s * DS + h * (DS / 2) + q * kQuadElems;
                if (full || e0 < d)
                    w[a][q] = *(const u32x4*)(wrow[a] + s * kStepBytes + q * 16);
                else
                    w[a][q] = u32x4{0u, 0u, 0u, 0u};
            }
    }

    __device__ __forceinline__ void load_x(u32x4 (&xr)[kXChunks], int64_t s, int tid) const
    {
#pragma unroll
        for (int p = 0; p < kXChunks; ++p) {
            const int c = tid + kThreads * p;
            const int row = c >> 3, c16 = c & 7;
            const int64_t e0 = s * DS + c16 * kQuadElems;
            if (b0 + row < B && e0 < d)
                xr[p] = *(const u32x4*)(X + ((b0 + row) * d + e0) * ES);
            else
                xr[p] = u32x4{0u, 0u, 0u, 0u};
        }
    }

    __device__ __forceinline__ static void store_x(const u32x4 (&xr)[kXChunks], unsigned char* xs, int tid)
    {
#pragma unroll
        for (int p = 0; p < kXChunks; ++p) {
            const int c = tid + kThreads * p;
            const int row = c >> 3, c16 = c & 7;
            *(u32x4*)(xs + row * kXRowStride + c16 * 16) = xr[p];
        }
    }

    __device__ __forceinline__ void compute(f32x16 (&acc)[FRAGS][NB], const u32x4 (&w)[FRAGS][4],
                                            const unsigned char* xs) const
    {
#pragma unroll
        for (int n = 0; n < NB; ++n)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const u32x4 bx = *(const u32x4*)(xs + (32 * n + (lane & 31)) * kXRowStride + h * 64 + q * 16);
#pragma unroll
                for (int a = 0; a < FRAGS; ++a) mfma_quad<DT>(acc[a][n], w[a][q], bx);
            }
    }

    __device__ __forceinline__ void run(f32x16 (&acc)[FRAGS][NB], int64_t s_begin, int64_t s_end,
                                        unsigned char* xs0, unsigned char* xs1, int tid) const
    {
        if (s_begin >= s_end) return;
        u32x4 wA[FRAGS][4], wB[FRAGS][4];
        u32x4 xr[kXChunks];
        load_w(wA, s_begin);
        load_x(xr, s_begin, tid);
        store_x(xr, xs0, tid);
        if (s_begin + 1 < s_end) {
            load_w(wB, s_begin + 1);
            load_x(xr, s_begin + 1, tid);
        }
        __syncthreads();
        for (int64_t s = s_begin; s < s_end; s += 2) {
            if (s + 1 < s_end) store_x(xr, xs1, tid);
            if (s + 2 < s_end) load_x(xr, s + 2, tid);
            compute(acc, wA, xs0);
            if (s + 2 < s_end) load_w(wA, s + 2);
            __syncthreads();
            if (s + 1 < s_end) {
                if (s + 2 < s_end) store_x(xr, xs0, tid);
                if (s + 3 < s_end) load_x(xr, s + 3, tid);
                compute(acc, wB, xs1);
                if (s + 3 < s_end) load_w(wB, s + 3);
                __syncthreads();
            }
        }
    }
};

}  // namespace stk
