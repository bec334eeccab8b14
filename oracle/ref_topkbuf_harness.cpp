// Harness that drives the reference's own CPU TopKBuffer
// (streamtopk_sae/csrc/cpu/topk_buffer.hpp, compiled from where it lies in the
// reference checkout) over a score stream with the reference's insertion loop
// (streamtopk_sae/csrc/cpu/streamtopk_cpu.cpp:49-55).  Built into oracle/_ref/
// only; it checks the oracle's restatement of the selection rule, never the
// product.
#include <cstdint>
#include "topk_buffer.hpp"

template <int K>
static void run(const float* s, int64_t n, float* V, int32_t* I)
{
    TopKBuffer<K> buf;
    buf.init();
    float thr = buf.threshold();
    for (int64_t j = 0; j < n; ++j) {
        if (s[j] > thr) {
            buf.try_insert(s[j], (int)j);
            thr = buf.threshold();
        }
    }
    for (int j = 0; j < K; ++j) { V[j] = buf.values[j]; I[j] = buf.indices[j]; }
}

extern "C" int ref_buffer_stream(const float* s, int64_t n, int64_t k, float* V, int32_t* I)
{
    switch (k) {
        case 1: run<1>(s, n, V, I); return 0;
        case 2: run<2>(s, n, V, I); return 0;
        case 4: run<4>(s, n, V, I); return 0;
        case 8: run<8>(s, n, V, I); return 0;
        case 16: run<16>(s, n, V, I); return 0;
        case 32: run<32>(s, n, V, I); return 0;
        case 64: run<64>(s, n, V, I); return 0;
        case 128: run<128>(s, n, V, I); return 0;
        default: return 1;
    }
}
