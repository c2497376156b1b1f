// noalloc.hip -- moe_layer_forward_noalloc: moe_layer_forward with its scratch in a library-owned device array, for
// callers that cannot allocate (code under HIP graph capture, serving loops, harnesses that forbid hipMalloc).
//
// The scratch is one file-scope __device__ array of MOE_NOALLOC_SCRATCH_BYTES. Each GPU the library runs on holds
// its own copy (allocated with the code object, held until the process ends). Host code never passes the array's
// name to a kernel (on the host it is a stand-in, not a device address): the first call on a device, with that
// device current, looks up the device address with hipGetSymbolAddress and keeps it per device. Every call on a
// device shares that device's array, so calls that overlap on one GPU (two streams, two threads) race; the layer
// writes every scratch byte it reads, so nothing needs clearing between calls. qmatvec_free drops the looked-up
// addresses (moe_noalloc_forget), so that a later call after a device reset or a reload of the code object looks
// them up again.

#include <hip/hip_runtime.h>

#include <mutex>

#include "moe_layer.h"

static __device__ __align__(256) unsigned char scratch[MOE_NOALLOC_SCRATCH_BYTES];

#define NOALLOC_MAX_DEVICES 64

static std::mutex g_mu;
static void* g_ptr[NOALLOC_MAX_DEVICES];  // the array's device address per device ordinal (null: not looked up)

// The current device's copy of the array, looked up once per device
static hipError_t scratch_ptr(void** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= NOALLOC_MAX_DEVICES) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lk(g_mu);
    if (!g_ptr[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        if (!p) return hipErrorInvalidSymbol;
        g_ptr[dev] = p;
    }
    *out = g_ptr[dev];
    return hipSuccess;
}

// Forget every looked-up address (library teardown)
void moe_noalloc_forget(void) {
    std::lock_guard<std::mutex> lk(g_mu);
    for (void*& p : g_ptr) p = nullptr;
}

extern "C" hipError_t moe_layer_forward_noalloc(const moe_layer_desc* d, const float* x, const float* logits, int T,
                                                float* out, int* ids_out, float* wts_out, hipStream_t stream) {
    if (!d || !x || !out || T <= 0) return hipErrorInvalidValue;
    const size_t need = moe_layer_scratch_bytes(d, T);
    if (need == 0 || need > (size_t)MOE_NOALLOC_SCRATCH_BYTES) return hipErrorInvalidValue;
    void* s = nullptr;
    const hipError_t e = scratch_ptr(&s);
    if (e != hipSuccess) return e;
    return moe_layer_forward(d, x, logits, T, out, ids_out, wts_out, s, (size_t)MOE_NOALLOC_SCRATCH_BYTES, stream);
}
