// boundary_caller.cpp -- a caller of the MoE boundary written against whichever qmatvec.h / gpu_ops.h the include
// path names: the reference's own (src/qmatvec.h, src/gpu_ops.h) or this repository's (include/). Linked against
// librocm_hip_moe.so and run without a GPU, it calls every boundary function with the header's own types and
// prints the results; built against both header sets it must compile, link and print the same lines. Test
// infrastructure (tests/test_abi.py builds and runs it).
#include <stddef.h>
#include <stdint.h>
#include <stdio.h>

#include "gpu_ops.h"
#include "qmatvec.h"

#define SHOW(expr) printf("%s = %lld\n", #expr, (long long)(expr))

int main() {
    // the activation bundle's layout
    printf("sizeof(qmatvec_q8) = %zu\n", sizeof(qmatvec_q8));
    printf("offsets q0 %zu d0 %zu qK %zu dK %zu bsK %zu s0 %zu max_k %zu xh %zu xh_bf16 %zu\n",
           offsetof(qmatvec_q8, q0), offsetof(qmatvec_q8, d0), offsetof(qmatvec_q8, qK), offsetof(qmatvec_q8, dK),
           offsetof(qmatvec_q8, bsK), offsetof(qmatvec_q8, s0), offsetof(qmatvec_q8, max_k),
           offsetof(qmatvec_q8, xh), offsetof(qmatvec_q8, xh_bf16));
    // host-side queries (no device needed)
    SHOW(qmatvec_q8_bytes(4096) >= 4096 * 2);
    static unsigned char mem[1 << 16];
    qmatvec_q8 q;
    qmatvec_q8_bind(&q, mem, 4096);
    SHOW(q.max_k);
    SHOW((unsigned char*)q.q0 >= mem && (unsigned char*)q.q0 < mem + sizeof(mem));
    SHOW(qmatvec_q8_supported(8, 2048));
    SHOW(qmatvec_q8_supported(12, 3072));
    SHOW(qmatvec_supported(0));
    SHOW(qmatvec_id_batch_tile(8, 768, 2048) > 0);
    SHOW(qmatvec_q8_id_batch_supported(8, 2048));
    SHOW(gpu_moe_max_tiles(2427, 8, 128, 64));
    SHOW(qmatvec_set_out_scale(nullptr, nullptr, 0, nullptr, 0));
    qmatvec_drop_out_scales(nullptr);
    // without a GPU: init fails, every launcher refuses (no fallback), nothing is touched
    SHOW(qmatvec_init(nullptr) != 0);
    SHOW(gpu_ops_init(nullptr) != 0);
    float f[64] = {};
    int32_t ids[8] = {};
    int it[8] = {};
    const hipStream_t s = nullptr;
    SHOW(qmatvec_quantize(f, 32, &q, s) != hipSuccess);
    SHOW(qmatvec_launch(0, f, 8, f, f, 1, 2, s) != hipSuccess);
    SHOW(qmatvec_launch_batch(0, f, 8, f, f, 1, 2, 1, s) != hipSuccess);
    SHOW(qmatvec_launch_q8(8, f, 34, &q, f, 1, 32, s) != hipSuccess);
    SHOW(qmatvec_launch_q8_pair(8, f, 1, f, f, 1, f, 34, &q, 32, s) != hipSuccess);
    SHOW(qmatvec_launch_q8_batch(8, f, 34, &q, f, 1, 1, 32, 1, s) != hipSuccess);
    SHOW(qmatvec_launch_q8_id(8, f, 34, ids, 1, 0, &q, f, 1, 32, 1, s) != hipSuccess);
    SHOW(qmatvec_launch_q8_id_pair(8, f, f, 34, ids, 1, 0, &q, f, f, 1, 32, 1, s) != hipSuccess);
    SHOW(qmatvec_launch_q8_id_x(8, f, f, f, f, 34, ids, 1, 0, &q, f, f, 1, 32, 1, s) != hipSuccess);
    SHOW(qmatvec_launch_q8_id_batch(8, f, 34, &q, f, 128, 256, 1, 64, ids, ids, ids, ids, ids, ids, s) != hipSuccess);
    SHOW(gpu_add_rmsnorm(f, nullptr, nullptr, nullptr, f, 32, 1, 1e-6f, nullptr, s) != hipSuccess);
    SHOW(gpu_swiglu(f, f, f, 32, nullptr, s) != hipSuccess);
    SHOW(gpu_moe_router(f, f, nullptr, it, f, f, 8, 2, 8, 1, s, 0) != hipSuccess);
    SHOW(gpu_moe_combine(f, f, nullptr, nullptr, f, 2, 8, 1, s) != hipSuccess);
    SHOW(gpu_moe_combine_scaled(f, f, nullptr, nullptr, it, f, f, 2, 8, 1, s) != hipSuccess);
    SHOW(gpu_moe_group(it, 1, 2, 8, 1, it, it, it, it, it, it, s) != hipSuccess);
    qmatvec_free();
    gpu_ops_free();
    return 0;
}
