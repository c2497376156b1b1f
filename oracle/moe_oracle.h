/* moe_oracle.h -- CPU restatement of the reference's MoE FFN semantics.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker that the HIP path is compared against. Only the
 * tests, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it; the product library never
 * links or calls it.
 *
 * Every function names the reference file:line whose behaviour it restates (paths relative to the
 * CowboyTim/rocm-hip tree). Type ids are ggml's (Q8_0 = 8, Q4_K = 12, ROCmFP4 = 100, ROCmFP4_FAST = 101).
 */
#ifndef MOE_ORACLE_H
#define MOE_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { ORC_F32 = 0, ORC_Q8_0 = 8, ORC_Q4_K = 12, ORC_ROCMFP4 = 100, ORC_ROCMFP4_FAST = 101 };

/* ---- scalars ---- */
float orc_fp16_to_f32(uint16_t h);
uint16_t orc_f32_to_fp16(float f); /* round to nearest even, as __float2half */
float orc_ue4m3_half(uint8_t e);

/* ---- block formats ---- */
int orc_block_values(int type);   /* values per block, 0 if unsupported */
int orc_block_bytes(int type);    /* bytes per block */
size_t orc_row_size(int type, int64_t k);
int orc_dequant(int type, const void *src, float *dst, int64_t n);
/* Whether the type is dotted with Q8_K activations (K-quants) rather than Q8_0. */
int orc_reads_q8k(int type);

/* ---- activation quantizers ---- */
/* Q8_0 per 32 values: q int8[n], d float[n/32] (FP16-rounded), s int32[n/32] (Q8_1 sum bits). */
void orc_quantize_q8_0(const float *x, int64_t n, int8_t *q, float *d, int32_t *s);
/* Q8_K per 256 values: q int8[n], d float[n/256], bs int32[n/16]. */
void orc_quantize_q8_K(const float *x, int64_t n, int8_t *q, float *d, int32_t *bs);
/* x quantized for wtype's activation format and decoded back to float. */
void orc_q8_roundtrip(int wtype, const float *x, float *out, int64_t k);

/* ---- integer block dots ---- */
/* Integer dot terms of one weight row against quantized activations, one int32 per unit:
 *  Q8_0:          K/32 units, sum of 32 products per block
 *  ROCmFP4:       K/16 units, the two 16-value halves of each block (scale e[0] / e[1])
 *  ROCmFP4_FAST:  K/32 units, sum of 32 products per block
 *  Q4_K:          K/32 units, sum of 32 (unscaled 4-bit) products per sub-block
 * xq is the int8 activation of the matching format (Q8_0 q or Q8_K q). Returns the unit count. */
int orc_block_dots(int type, const void *wrow, const int8_t *xq, int k, int32_t *out);

/* y[n] from the integer block dots and the scales, accumulated in double. */
double orc_row_dot_int(int type, const void *wrow, const int8_t *xq, const float *xd, const int32_t *xbs, int k);
/* y[n] as the reference's CPU harness computes it: decoded weights times the round-tripped
 * activation, double accumulation. */
double orc_row_dot_deq(int type, const void *wrow, const float *x_rt, int k);

/* y[N] = W x with x float [K]: quantize + round trip, then orc_row_dot_deq per row. */
void orc_matvec(int type, const void *W, size_t row_bytes, const float *x, float *y, int n, int k);
/* Router logits: y[N] = W x with W float [N][K], double accumulation. */
void orc_matvec_f32(const float *W, const float *x, float *y, int n, int k);

/* ---- router ---- */
/* logits [T][NE] -> ids [T][stride] (descending, ties to the lower index), wts [T][NU] renormalised by
 * max(sum, 6.103515625e-5); sg [T] = sigmoid(x . w_shexp) if w_shexp. stride > NU: id NU = -1. */
int orc_router(const float *logits, const float *x, const float *w_shexp, int32_t *ids, float *wts, float *sg,
               int ne, int nu, int n, int t, int ids_stride);

/* ---- dispatch ---- */
/* Group ids [T][NU] by expert: counts [NE], offsets [NE] (exclusive scan), entries sorted by (expert, entry
 * index): tok_rows / pair_rows [T*NU]; tiles: tile_e / tile_start / tile_n (<= max_tiles), n_tiles. */
int orc_group(const int32_t *ids, int t, int nu, int ne, int tile, int32_t *counts, int32_t *offsets,
              int32_t *tok_rows, int32_t *pair_rows, int32_t *n_tiles, int32_t *tile_e, int32_t *tile_start,
              int32_t *tile_n, int max_tiles);
int orc_max_tiles(int t, int nu, int ne, int tile);

/* ---- elementwise ---- */
void orc_swiglu(const float *g, const float *u, float *out, int64_t n);
void orc_combine(const float *down, const float *wts, const float *shared, const float *sg, float *out, int nu,
                 int n, int t);
void orc_rmsnorm(const float *x, const float *w, float *y, int n, float eps);

/* ---- one MoE FFN layer ---- */
typedef struct orc_moe_layer {
    int type;          /* expert weight type (gate, up, down share it) */
    int n_embd;        /* E */
    int n_expert;      /* NE */
    int n_used;        /* NU */
    int n_ff;          /* FE */
    const float *w_router;   /* [NE][E], or NULL with logits given */
    const void *w_gate;      /* [NE*FE] rows of row_size(type, E) */
    const void *w_up;
    const void *w_down;      /* [NE*E] rows of row_size(type, FE) */
    const void *s_gate;      /* shared expert (FE rows) or NULL */
    const void *s_up;
    const void *s_down;
    const float *w_shexp;    /* [E] shared-expert gate vector or NULL (gate 1) */
} orc_moe_layer;

/* out [T][E] = MoE(x [T][E]). logits_in [T][NE] (NULL: W_router x). ids_out [T][NU] / wts_out [T][NU]
 * receive the routing. Follows QwenModel::moe_core (src/qwen_model.cpp:904-937). */
int orc_moe_forward(const orc_moe_layer *L, const float *x, const float *logits_in, int t, float *out,
                    int32_t *ids_out, float *wts_out);

/* OpenMP threads of the row loops (the results do not depend on the count); returns the count in effect */
int orc_set_threads(int n);

#ifdef __cplusplus
}
#endif
#endif
