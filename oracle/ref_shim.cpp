// ref_shim.cpp -- C-linkage wrappers around the reference's own CPU ops, so that the tests can call the
// reference build in oracle/_ref (src/qwen_ops.h declares them with C++ linkage). Test infrastructure only.
#include <cstdint>

#include "qwen_ops.h"

extern "C" {
void ref_rmsnorm(const float* x, const float* w, float* y, int n, float eps) { qwen_rmsnorm(x, w, y, n, eps); }
float ref_silu(float x) { return qwen_silu(x); }
// SwiGLU as the reference forms it from its CPU op: silu(g) * u per element (src/qwen_ops.h:47)
void ref_swiglu(const float* g, const float* u, float* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = qwen_silu(g[i]) * u[i];
}
}
