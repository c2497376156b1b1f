// grouped.h -- internal entry points of the grouped MFMA kernels (grouped_gemm.hip) for the C-ABI launchers.
#ifndef GROUPED_H
#define GROUPED_H

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "qmatvec.h"

// A shared expert run as more tiles of a grouped launch: its T tokens (activation rows 0..T-1, in entry-tile order
// after the routed tiles when the launch hands activations over so), output rows out0 + token, weights from the
// operand tiles v / s (v2 / s2: the up matrix of a gate / up launch) of its one matrix
struct GShared {
    const uint8_t* v;
    const uint8_t* s;
    const uint8_t* v2;
    const uint8_t* s2;
    int T;
    long long out0;
};

bool moe_grouped_mfma_ok(int type, int N, int K);
int moe_grouped_mfma_tile(void);
hipError_t moe_launch_grouped_mfma(int type, const uint8_t* v, const uint8_t* s, long long vrb, long long srb,
                                   const qmatvec_q8* q, float* y, int N, int K, int max_tiles, const int32_t* n_tiles,
                                   const int32_t* tile_e, const int32_t* tile_start, const int32_t* tile_n,
                                   const int32_t* in_rows, const int32_t* out_rows, int xt, const GShared* sh,
                                   hipStream_t stream);
hipError_t moe_launch_grouped_swiglu(int type, const uint8_t* vg, const uint8_t* sg, const uint8_t* vu,
                                     const uint8_t* su, long long vrb, long long srb, const qmatvec_q8* q, int8_t* aq,
                                     float* ad, int N, int K, int max_tiles, const int32_t* n_tiles,
                                     const int32_t* tile_e, const int32_t* tile_start, const int32_t* tile_n,
                                     const int32_t* in_rows, const int32_t* out_rows, int xt, const GShared* sh,
                                     hipStream_t stream);
hipError_t moe_launch_grouped_gate_up(int type, const uint8_t* vg, const uint8_t* sg, const uint8_t* vu,
                                      const uint8_t* su, long long vrb, long long srb, const qmatvec_q8* q, float* y,
                                      int N, int K, int max_tiles, const int32_t* n_tiles, const int32_t* tile_e,
                                      const int32_t* tile_start, const int32_t* tile_n, const int32_t* in_rows,
                                      const int32_t* out_rows, hipStream_t stream);
hipError_t moe_launch_dense_mfma(int type, const uint8_t* v, const uint8_t* s, long long vrb, long long srb,
                                 const qmatvec_q8* q, float* y, long long ldy, int N, int K, int T,
                                 hipStream_t stream);
bool moe_packed_tiles(const void* W, int type, int K, size_t row_bytes, const uint8_t** vt, const uint8_t** st,
                      long long* vgs, long long* sgs);

#endif  // GROUPED_H
