// stk_internal.h -- error plumbing shared by the C ABI translation units.
#pragma once
#include <stdint.h>

namespace stk {

// Records a printf-style message for stk_last_error() and returns `code`.
int set_error(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();

// Reference wording for an unsupported k (streamtopk_exact.cu:826-828,
// streamtopk_cpu.cpp:119-121).
bool k_supported(int64_t k);

}  // namespace stk
