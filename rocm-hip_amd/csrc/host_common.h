// host_common.h -- launch helper and library state shared by the C-ABI launchers.
#ifndef HOST_COMMON_H
#define HOST_COMMON_H

#include <hip/hip_runtime.h>
#include <stdint.h>

// 1 once qmatvec_init / gpu_ops_init found a gfx950 device (either one initialises the whole library)
extern "C" int moe_lib_ready(void);

// Compute units of the initialised device (persistent grids size themselves by it)
int moe_device_cus(void);

struct qmatvec_q8;
// gpu_swiglu's SwiGLU and quantized bundle without its argument checks; out may be null (no fp32 values written);
// parts: the bundle's formats wanted (1: Q8_0 + Q8_1 sums, 2: Q8_K, 3: both; lengths not a multiple of 256 get both)
hipError_t moe_swiglu_q8(const float* g, const float* u, float* out, int n, const qmatvec_q8* q8, hipStream_t stream,
                         int parts);

// gpu_moe_router that also quantizes x [T][n] into q8 (formats as in moe_swiglu_q8's parts); gpu_add_rmsnorm that
// also quantizes y. Both return hipErrorInvalidValue where their conditions (n % 256 == 0, alignment; the norm:
// n <= 4096) do not hold, and the caller then launches the quantizer on its own.
hipError_t moe_router_quantize(const float* logits, const float* x, const float* w_shexp, int* ids, float* wts,
                               float* sg, int n_expert, int n_used, int n, int T, int ids_stride, const qmatvec_q8* q8,
                               int parts, hipStream_t stream);
hipError_t moe_add_rmsnorm_q8(const float* x_in, const float* add, float* x_out, const float* w, float* y, int n,
                              int T, float eps, const qmatvec_q8* q8, int parts, hipStream_t stream);

template <typename T>
struct same_type {
    typedef T type;
};

// Launch a kernel and return its launch status (no sticky error state is consulted)
template <typename... Args>
static inline hipError_t launch_kernel(void (*k)(Args...), dim3 grid, dim3 block, size_t shm, hipStream_t s,
                                       typename same_type<Args>::type... args) {
    void* ptrs[] = {(void*)&args..., nullptr};
    return hipLaunchKernel((const void*)k, grid, block, ptrs, shm, s);
}

static inline bool aligned(const void* p, uintptr_t a) { return ((uintptr_t)p & (a - 1)) == 0; }

#endif  // HOST_COMMON_H
