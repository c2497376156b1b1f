/* moe_oracle.c -- CPU restatement of the reference's MoE FFN semantics (see moe_oracle.h).
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP path, never part of it.
 *
 * Parity pins (tests/test_oracle.py): the decoders are compared bit for bit with the reference's own
 * qt_to_float (oracle/_ref, compiled from src/quant_types.cpp) and with hand-built known-answer blocks; the
 * quantizers against closed forms and their special cases; the integer block dots against a brute-force
 * int64 sum over the decoded codes; orc_row_dot_int against orc_row_dot_deq (two independent routes to the
 * same number); the router against brute force on small expert counts; the dispatch against its invariants.
 */
#include "moe_oracle.h"

#include <omp.h>

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ scalars */

/* IEEE binary16 -> binary32, exact (src/quant_types.cpp:16-41 restates the same conversion). */
float orc_fp16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h >> 15) << 31;
    const int exp = (h >> 10) & 0x1f;
    const uint32_t man = h & 0x3ffu;
    uint32_t bits;
    if (exp == 0x1f) {
        bits = sign | 0x7f800000u | (man << 13);
    } else if (exp != 0) {
        bits = sign | ((uint32_t)(exp - 15 + 127) << 23) | (man << 13);
    } else if (man == 0) {
        bits = sign;
    } else { /* subnormal: man * 2^-24, exact in float */
        float f = (float)man * 0x1p-24f;
        memcpy(&bits, &f, 4);
        bits |= sign;
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* binary32 -> binary16, round to nearest even (the conversion __float2half performs). */
uint16_t orc_f32_to_fp16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    const uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) /* inf / nan */
        return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u | ((ax >> 13) & 0x3ffu) : 0u));
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* rounds to >= 65520: overflow */
    const int e = (int)(ax >> 23) - 127;
    if (e >= -14) { /* normal half */
        uint32_t m = ax & 0x7fffffu;
        uint32_t h = ((uint32_t)(e + 15) << 10) | (m >> 13);
        const uint32_t rem = m & 0x1fffu;
        if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h; /* carry may bump the exponent: still right */
        return (uint16_t)(sign | h);
    }
    /* subnormal half: value = q * 2^-24 with q = round(|f| * 2^24) */
    if (e < -25) return sign; /* below half the smallest subnormal */
    const uint32_t m = (ax & 0x7fffffu) | 0x800000u; /* |f| = m * 2^(e-23) */
    const int shift = -e - 1;                          /* q = m >> (shift) with e-23+24 = e+1 */
    uint32_t q = m >> shift;
    const uint32_t rem = m & ((1u << shift) - 1u), half = 1u << (shift - 1);
    if (rem > half || (rem == half && (q & 1u))) ++q;
    return (uint16_t)(sign | q);
}

/* Unsigned E4M3 scale byte at half scale; 0x7f and above decode to 0 (src/quant_types.cpp:352-357). */
float orc_ue4m3_half(uint8_t e) {
    if (e >= 0x7f) return 0.0f;
    const int ex = e >> 3, m = e & 7;
    if (ex == 0) return ldexpf((float)m, -10);
    return ldexpf((float)(8 + m), ex - 11);
}

/* FP4 codebook of the engine's ROCmFP4 at half scale (src/quant_types.cpp:349). */
static const int8_t k_fp4[16] = {0, 1, 2, 3, 4, 6, 8, 10, 0, -1, -2, -3, -4, -6, -8, -10};

static float rd16(const uint8_t *p) { return orc_fp16_to_f32((uint16_t)(p[0] | (p[1] << 8))); }

/* ------------------------------------------------------------------ formats */

int orc_block_values(int type) {
    switch (type) {
    case ORC_F32: return 1;
    case ORC_Q8_0: case ORC_ROCMFP4: case ORC_ROCMFP4_FAST: return 32;
    case ORC_Q4_K: return 256;
    default: return 0;
    }
}

/* Block sizes from the reference's traits table (src/quant_types.cpp:591-615). */
int orc_block_bytes(int type) {
    switch (type) {
    case ORC_F32: return 4;
    case ORC_Q8_0: return 34;
    case ORC_ROCMFP4: return 18;
    case ORC_ROCMFP4_FAST: return 17;
    case ORC_Q4_K: return 144;
    default: return 0;
    }
}

size_t orc_row_size(int type, int64_t k) {
    const int bv = orc_block_values(type);
    if (!bv || k % bv) return 0;
    return (size_t)(k / bv) * (size_t)orc_block_bytes(type);
}

int orc_reads_q8k(int type) { return type == ORC_Q4_K; }

/* The 6-bit scale and min of sub-block j of a Q4_K super-block (src/quant_types.cpp:193-202). */
static void q4k_scale_min(int j, const uint8_t *s, int *sc, int *mn) {
    if (j < 4) {
        *sc = s[j] & 63;
        *mn = s[j + 4] & 63;
    } else {
        *sc = (s[j + 4] & 15) | ((s[j - 4] >> 6) << 4);
        *mn = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
    }
}

/* Decoders: src/quant_types.cpp:182-189 (Q8_0), 265-287 (Q4_K), 360-370 (ROCmFP4), 373-381 (FAST). The
 * float expression order is the reference's (q * d; d1 * q - m1; codebook * e). */
int orc_dequant(int type, const void *src, float *y, int64_t n) {
    const uint8_t *b = (const uint8_t *)src;
    const int bv = orc_block_values(type);
    if (!bv || n % bv) return -1;
    switch (type) {
    case ORC_F32:
        memcpy(y, src, (size_t)n * 4);
        return 0;
    case ORC_Q8_0:
        for (int64_t i = 0; i < n / 32; ++i, b += 34, y += 32) {
            const float d = rd16(b);
            for (int j = 0; j < 32; ++j) y[j] = (float)(int8_t)b[2 + j] * d;
        }
        return 0;
    case ORC_ROCMFP4:
        for (int64_t i = 0; i < n / 32; ++i, b += 18, y += 32) {
            const float e0 = orc_ue4m3_half(b[16]), e1 = orc_ue4m3_half(b[17]);
            for (int j = 0; j < 16; ++j) {
                y[j] = (float)k_fp4[b[j] & 15] * e0;
                y[j + 16] = (float)k_fp4[b[j] >> 4] * e1;
            }
        }
        return 0;
    case ORC_ROCMFP4_FAST:
        for (int64_t i = 0; i < n / 32; ++i, b += 17, y += 32) {
            const float e = orc_ue4m3_half(b[16]);
            for (int j = 0; j < 16; ++j) {
                y[j] = (float)k_fp4[b[j] & 15] * e;
                y[j + 16] = (float)k_fp4[b[j] >> 4] * e;
            }
        }
        return 0;
    case ORC_Q4_K:
        for (int64_t i = 0; i < n / 256; ++i, b += 144) {
            const float d = rd16(b), dmin = rd16(b + 2);
            const uint8_t *q = b + 16;
            for (int c = 0; c < 4; ++c) {
                int sc, mn;
                q4k_scale_min(2 * c, b + 4, &sc, &mn);
                const float d1 = d * (float)sc, m1 = dmin * (float)mn;
                q4k_scale_min(2 * c + 1, b + 4, &sc, &mn);
                const float d2 = d * (float)sc, m2 = dmin * (float)mn;
                for (int l = 0; l < 32; ++l) *y++ = d1 * (float)(q[32 * c + l] & 15) - m1;
                for (int l = 0; l < 32; ++l) *y++ = d2 * (float)(q[32 * c + l] >> 4) - m2;
            }
        }
        return 0;
    }
    return -1;
}

/* ------------------------------------------------------------------ activation quantizers */

/* Q8_0 + Q8_1 sum per 32 values, as src/q8_device.h:60-73 and tests/matvec_verify.cpp:67-74:
 * amax, id = 127 / amax (unrounded), q = round-half-even(x * id), d = F16(amax / 127),
 * s = F16(amax / 127 * sum q) stored as float bits. */
void orc_quantize_q8_0(const float *x, int64_t n, int8_t *q, float *d, int32_t *s) {
    for (int64_t b = 0; b < n / 32; ++b) {
        const float *xb = x + 32 * b;
        float amax = 0.0f;
        for (int j = 0; j < 32; ++j) amax = fmaxf(amax, fabsf(xb[j]));
        const float id = amax != 0.0f ? 127.0f / amax : 0.0f;
        int sum = 0;
        for (int j = 0; j < 32; ++j) {
            const int v = (int)nearbyintf(xb[j] * id);
            q[32 * b + j] = (int8_t)v;
            sum += v;
        }
        const float dd = amax / 127.0f;
        d[b] = orc_fp16_to_f32(orc_f32_to_fp16(dd));
        if (s) {
            const float sv = orc_fp16_to_f32(orc_f32_to_fp16(dd * (float)sum));
            memcpy(&s[b], &sv, 4);
        }
    }
}

/* Q8_K per 256 values, as src/q8_device.h:75-103 and tests/matvec_verify.cpp:58-66: the signed value of
 * largest |x| (first index on ties), iscale = -127 / max, q = min(127, round-half-even(iscale * x)),
 * d = 1 / iscale, bs = sums of 16 q. */
void orc_quantize_q8_K(const float *x, int64_t n, int8_t *q, float *d, int32_t *bs) {
    for (int64_t b = 0; b < n / 256; ++b) {
        const float *xb = x + 256 * b;
        float amax = 0.0f, mx = 0.0f;
        for (int j = 0; j < 256; ++j)
            if (fabsf(xb[j]) > amax) {
                amax = fabsf(xb[j]);
                mx = xb[j];
            }
        float iscale = 0.0f;
        if (amax != 0.0f) iscale = -127.0f / mx;
        for (int j = 0; j < 256; ++j) {
            int v = 0;
            if (amax != 0.0f) {
                v = (int)nearbyintf(iscale * xb[j]);
                if (v > 127) v = 127;
            }
            q[256 * b + j] = (int8_t)v;
        }
        d[b] = amax != 0.0f ? 1.0f / iscale : 0.0f;
        if (bs)
            for (int g = 0; g < 16; ++g) {
                int sum = 0;
                for (int j = 0; j < 16; ++j) sum += q[256 * b + 16 * g + j];
                bs[16 * b + g] = sum;
            }
    }
}

/* tests/matvec_verify.cpp:56-75: x quantized in the weight type's activation format and decoded back. */
void orc_q8_roundtrip(int wtype, const float *x, float *out, int64_t k) {
    int8_t *q = (int8_t *)malloc((size_t)k);
    if (orc_reads_q8k(wtype)) {
        float *d = (float *)malloc((size_t)(k / 256) * 4);
        orc_quantize_q8_K(x, k, q, d, NULL);
        for (int64_t i = 0; i < k; ++i) out[i] = d[i / 256] * (float)q[i];
        free(d);
    } else {
        float *d = (float *)malloc((size_t)(k / 32) * 4);
        orc_quantize_q8_0(x, k, q, d, NULL);
        for (int64_t i = 0; i < k; ++i) out[i] = d[i / 32] * (float)q[i];
        free(d);
    }
    free(q);
}

/* ------------------------------------------------------------------ integer block dots */

/* The integer terms of the reference's int8 kernels: q8_0_q8_block (src/matvec_q.hip:1530-1536),
 * p4_q8_block halves (:1351-1361), rocmfp4_fast_q8_block (:1456-1466) and the Q4_K sub-block sums of
 * mv_kquant (:1716-1747), here per whole unit from the decoded codes. */
int orc_block_dots(int type, const void *wrow, const int8_t *xq, int k, int32_t *out) {
    const uint8_t *b = (const uint8_t *)wrow;
    switch (type) {
    case ORC_Q8_0:
        for (int i = 0; i < k / 32; ++i, b += 34) {
            int64_t s = 0;
            for (int j = 0; j < 32; ++j) s += (int64_t)(int8_t)b[2 + j] * xq[32 * i + j];
            out[i] = (int32_t)s;
        }
        return k / 32;
    case ORC_ROCMFP4:
        for (int i = 0; i < k / 32; ++i, b += 18) {
            int64_t s0 = 0, s1 = 0;
            for (int j = 0; j < 16; ++j) {
                s0 += (int64_t)k_fp4[b[j] & 15] * xq[32 * i + j];
                s1 += (int64_t)k_fp4[b[j] >> 4] * xq[32 * i + 16 + j];
            }
            out[2 * i] = (int32_t)s0;
            out[2 * i + 1] = (int32_t)s1;
        }
        return k / 16;
    case ORC_ROCMFP4_FAST:
        for (int i = 0; i < k / 32; ++i, b += 17) {
            int64_t s = 0;
            for (int j = 0; j < 16; ++j)
                s += (int64_t)k_fp4[b[j] & 15] * xq[32 * i + j] + (int64_t)k_fp4[b[j] >> 4] * xq[32 * i + 16 + j];
            out[i] = (int32_t)s;
        }
        return k / 32;
    case ORC_Q4_K:
        for (int i = 0; i < k / 256; ++i, b += 144) {
            const uint8_t *q = b + 16;
            for (int c = 0; c < 4; ++c) {
                int64_t lo = 0, hi = 0;
                for (int l = 0; l < 32; ++l) {
                    lo += (int64_t)(q[32 * c + l] & 15) * xq[256 * i + 64 * c + l];
                    hi += (int64_t)(q[32 * c + l] >> 4) * xq[256 * i + 64 * c + 32 + l];
                }
                out[8 * i + 2 * c] = (int32_t)lo;
                out[8 * i + 2 * c + 1] = (int32_t)hi;
            }
        }
        return k / 32;
    }
    return -1;
}

/* The float combination of the integer terms, in double: Q8_0 e dx s (src/matvec_q.hip:1536), ROCmFP4
 * e0 dx s0 + e1 dx s1 (:1287-1289), FAST e dx (s0 + s1) (:1466), Q4_K d dx sum(sc s) - dmin dx sum(m bs)
 * (:1740-1746). xd: the activation scales (per 32, or per 256 for Q4_K); xbs: Q8_K sums of 16 (Q4_K). */
double orc_row_dot_int(int type, const void *wrow, const int8_t *xq, const float *xd, const int32_t *xbs, int k) {
    const uint8_t *b = (const uint8_t *)wrow;
    int32_t *u = (int32_t *)malloc((size_t)(k / 16 + 8) * 4);
    const int nu = orc_block_dots(type, wrow, xq, k, u);
    double acc = 0.0;
    if (nu < 0) {
        free(u);
        return NAN;
    }
    switch (type) {
    case ORC_Q8_0:
        for (int i = 0; i < k / 32; ++i) acc += (double)rd16(b + 34 * i) * (double)xd[i] * (double)u[i];
        break;
    case ORC_ROCMFP4:
        for (int i = 0; i < k / 32; ++i) {
            const uint8_t *bb = b + 18 * i;
            acc += (double)orc_ue4m3_half(bb[16]) * xd[i] * u[2 * i] +
                   (double)orc_ue4m3_half(bb[17]) * xd[i] * u[2 * i + 1];
        }
        break;
    case ORC_ROCMFP4_FAST:
        for (int i = 0; i < k / 32; ++i) acc += (double)orc_ue4m3_half(b[17 * i + 16]) * xd[i] * u[i];
        break;
    case ORC_Q4_K:
        for (int i = 0; i < k / 256; ++i) {
            const uint8_t *bb = b + 144 * i;
            int64_t isum = 0, msum = 0;
            for (int j = 0; j < 8; ++j) {
                int sc, mn;
                q4k_scale_min(j, bb + 4, &sc, &mn);
                isum += (int64_t)sc * u[8 * i + j];
                msum += (int64_t)mn * (xbs[16 * i + 2 * j] + xbs[16 * i + 2 * j + 1]);
            }
            acc += (double)rd16(bb) * xd[i] * (double)isum - (double)rd16(bb + 2) * xd[i] * (double)msum;
        }
        break;
    }
    free(u);
    return acc;
}

/* tests/matvec_verify.cpp:130-136: decoded row times the round-tripped x, double accumulation. */
double orc_row_dot_deq(int type, const void *wrow, const float *x_rt, int k) {
    float *w = (float *)malloc((size_t)k * 4);
    orc_dequant(type, wrow, w, k);
    double acc = 0.0;
    for (int i = 0; i < k; ++i) acc += (double)w[i] * (double)x_rt[i];
    free(w);
    return acc;
}

void orc_matvec(int type, const void *W, size_t row_bytes, const float *x, float *y, int n, int k) {
    float *xr = (float *)malloc((size_t)k * 4);
    orc_q8_roundtrip(type, x, xr, k);
    for (int r = 0; r < n; ++r) y[r] = (float)orc_row_dot_deq(type, (const uint8_t *)W + (size_t)r * row_bytes, xr, k);
    free(xr);
}

void orc_matvec_f32(const float *W, const float *x, float *y, int n, int k) {
#pragma omp parallel for schedule(static)
    for (int r = 0; r < n; ++r) {
        double acc = 0.0;
        for (int i = 0; i < k; ++i) acc += (double)W[(size_t)r * k + i] * (double)x[i];
        y[r] = (float)acc;
    }
}

/* ------------------------------------------------------------------ router */

/* src/gpu_ops.hip:185-241 (moe_router) with the selection rule of tests/forward_verify.cpp:395-403: the
 * NU largest probabilities in descending order, ties to the lower expert index (stable sort). Softmax is
 * strictly monotonic, so ranking the probabilities is ranking the logits; it is done on the logits here,
 * which keeps the rank exact where expf would round two probabilities together. */
int orc_router(const float *logits, const float *x, const float *w_shexp, int32_t *ids, float *wts, float *sg,
               int ne, int nu, int n, int t, int ids_stride) {
    if (ne <= 0 || nu <= 0 || nu > ne || t <= 0) return -1;
    if (ids_stride == 0) ids_stride = nu;
    if (ids_stride < nu) return -1;
    int *order = (int *)malloc((size_t)ne * sizeof(int));
    double *p = (double *)malloc((size_t)ne * sizeof(double));
    for (int tt = 0; tt < t; ++tt) {
        const float *l = logits + (size_t)tt * ne;
        double mx = -INFINITY, sum = 0.0;
        for (int e = 0; e < ne; ++e) mx = l[e] > mx ? l[e] : mx;
        for (int e = 0; e < ne; ++e) sum += (p[e] = exp((double)l[e] - mx));
        for (int e = 0; e < ne; ++e) p[e] /= sum;
        /* selection: NU rounds of "largest remaining, lowest index on ties" (a stable descending sort) */
        for (int e = 0; e < ne; ++e) order[e] = 0;
        double ws = 0.0;
        for (int r = 0; r < nu; ++r) {
            int best = -1;
            for (int e = 0; e < ne; ++e)
                if (!order[e] && (best < 0 || l[e] > l[best])) best = e;
            order[best] = 1;
            ids[(size_t)tt * ids_stride + r] = best;
            ws += p[best];
        }
        if (ids_stride > nu) ids[(size_t)tt * ids_stride + nu] = -1;
        const double wsum = ws > 6.103515625e-5 ? ws : 6.103515625e-5;
        for (int r = 0; r < nu; ++r) wts[(size_t)tt * nu + r] = (float)(p[ids[(size_t)tt * ids_stride + r]] / wsum);
        if (w_shexp && sg) {
            double dd = 0.0;
            for (int i = 0; i < n; ++i) dd += (double)x[(size_t)tt * n + i] * w_shexp[i];
            sg[tt] = (float)(1.0 / (1.0 + exp(-dd)));
        }
    }
    free(order);
    free(p);
    return 0;
}

/* ------------------------------------------------------------------ dispatch */

/* src/gpu_ops.h:72-75 */
int orc_max_tiles(int t, int nu, int ne, int tile) {
    const int n = t * nu, bound = ne + n / tile;
    return n < bound ? n : bound;
}

/* src/gpu_ops.hip:273-320 (moe_group): histogram, exclusive scans of entry and tile counts, the tile table in
 * expert order, and the entries grouped by expert. Every (token, slot) entry is counted and placed, a repeated
 * id within a token's row included (the reference's histogram at :281 and placement at :316-320 count each
 * entry). The reference leaves the order inside an expert's run to its atomics; this oracle fixes it to
 * ascending entry index, which the HIP path also produces. Ids outside [0, ne) are skipped: the reference
 * indexes its LDS histogram with them unchecked (undefined there), the HIP path skips them too. */
static int group_valid(const int32_t *row, int j, int ne) { return row[j] >= 0 && row[j] < ne; }

int orc_group(const int32_t *ids, int t, int nu, int ne, int tile, int32_t *counts, int32_t *offsets,
              int32_t *tok_rows, int32_t *pair_rows, int32_t *n_tiles, int32_t *tile_e, int32_t *tile_start,
              int32_t *tile_n, int max_tiles) {
    const int n = t * nu;
    if (t <= 0 || nu <= 0 || ne <= 0 || tile <= 0) return -1;
    for (int e = 0; e < ne; ++e) counts[e] = 0;
    for (int i = 0; i < n; ++i)
        if (group_valid(ids + (size_t)(i / nu) * nu, i % nu, ne)) ++counts[ids[i]];
    int off = 0, nt = 0;
    for (int e = 0; e < ne; ++e) {
        offsets[e] = off;
        for (int k = 0; k * tile < counts[e]; ++k) {
            if (nt >= max_tiles) return -2;
            tile_e[nt] = e;
            tile_start[nt] = off + k * tile;
            tile_n[nt] = counts[e] - k * tile < tile ? counts[e] - k * tile : tile;
            ++nt;
        }
        off += counts[e];
    }
    *n_tiles = nt;
    int32_t *next = (int32_t *)malloc((size_t)ne * 4);
    memcpy(next, offsets, (size_t)ne * 4);
    for (int i = 0; i < n; ++i) {
        const int e = ids[i];
        if (!group_valid(ids + (size_t)(i / nu) * nu, i % nu, ne)) continue;
        const int p = next[e]++;
        tok_rows[p] = i / nu;
        pair_rows[p] = i;
    }
    free(next);
    return 0;
}

/* ------------------------------------------------------------------ elementwise */

/* src/gpu_ops.hip:103-114 with src/qwen_ops.h:47's SiLU: g / (1 + e^-g) * u in float. */
void orc_swiglu(const float *g, const float *u, float *out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = g[i] / (1.0f + expf(-g[i])) * u[i];
}

/* src/gpu_ops.hip:245-264: w0 d0, then += wj dj in slot order, then + sg shared (+ shared without sg). */
void orc_combine(const float *down, const float *wts, const float *shared, const float *sg, float *out, int nu,
                 int n, int t) {
    for (int tt = 0; tt < t; ++tt)
        for (int i = 0; i < n; ++i) {
            const float *d = down + (size_t)tt * nu * n + i;
            const float *w = wts + (size_t)tt * nu;
            float acc = w[0] * d[0];
            for (int j = 1; j < nu; ++j) acc += w[j] * d[(size_t)j * n];
            if (shared) acc += sg ? shared[(size_t)tt * n + i] * sg[tt] : shared[(size_t)tt * n + i];
            out[(size_t)tt * n + i] = acc;
        }
}

/* src/qwen_ops.cpp:8-13 */
void orc_rmsnorm(const float *x, const float *w, float *y, int n, float eps) {
    double ss = 0.0;
    for (int i = 0; i < n; ++i) ss += (double)x[i] * x[i];
    const float inv = (float)(1.0 / sqrt(ss / n + eps));
    for (int i = 0; i < n; ++i) y[i] = x[i] * inv * (w ? w[i] : 1.0f);
}

/* ------------------------------------------------------------------ one layer */

/* One expert FFN for one token: gate/up on the round-tripped x, SwiGLU, round trip, down. */
static void expert_ffn(int type, const uint8_t *wg, const uint8_t *wu, const uint8_t *wd, const float *x_rt, int E,
                       int FE, float *out) {
    const size_t rb_in = orc_row_size(type, E), rb_out = orc_row_size(type, FE);
    float *g = (float *)malloc((size_t)FE * 4), *u = (float *)malloc((size_t)FE * 4);
    float *a = (float *)malloc((size_t)FE * 4), *ar = (float *)malloc((size_t)FE * 4);
#pragma omp parallel for schedule(static)
    for (int r = 0; r < FE; ++r) {
        g[r] = (float)orc_row_dot_deq(type, wg + (size_t)r * rb_in, x_rt, E);
        u[r] = (float)orc_row_dot_deq(type, wu + (size_t)r * rb_in, x_rt, E);
    }
    orc_swiglu(g, u, a, FE);
    orc_q8_roundtrip(type, a, ar, FE);
#pragma omp parallel for schedule(static)
    for (int i = 0; i < E; ++i) out[i] = (float)orc_row_dot_deq(type, wd + (size_t)i * rb_out, ar, FE);
    free(g);
    free(u);
    free(a);
    free(ar);
}

/* QwenModel::moe_core (src/qwen_model.cpp:904-937): router logits, moe_router, the selected experts' gate/up
 * on the quantized input, SwiGLU quantized for down, down, and moe_combine with the gated shared expert. */
int orc_moe_forward(const orc_moe_layer *L, const float *x, const float *logits_in, int t, float *out,
                    int32_t *ids_out, float *wts_out) {
    const int E = L->n_embd, NE = L->n_expert, NU = L->n_used, FE = L->n_ff, type = L->type;
    const size_t rb_in = orc_row_size(type, E), rb_out = orc_row_size(type, FE);
    if (!rb_in || !rb_out) return -1;
    float *logits = (float *)malloc((size_t)t * NE * 4);
    int32_t *ids = (int32_t *)malloc((size_t)t * NU * 4);
    float *wts = (float *)malloc((size_t)t * NU * 4), *sg = (float *)malloc((size_t)t * 4);
    float *xr = (float *)malloc((size_t)E * 4);
    float *down = (float *)malloc((size_t)NU * E * 4), *shared = (float *)malloc((size_t)E * 4);
    for (int tt = 0; tt < t; ++tt) {
        if (logits_in)
            memcpy(logits + (size_t)tt * NE, logits_in + (size_t)tt * NE, (size_t)NE * 4);
        else
            orc_matvec_f32(L->w_router, x + (size_t)tt * E, logits + (size_t)tt * NE, NE, E);
    }
    orc_router(logits, x, L->w_shexp, ids, wts, sg, NE, NU, E, t, NU);
    for (int tt = 0; tt < t; ++tt) {
        orc_q8_roundtrip(type, x + (size_t)tt * E, xr, E);
        for (int j = 0; j < NU; ++j) {
            const size_t e = (size_t)ids[(size_t)tt * NU + j];
            expert_ffn(type, (const uint8_t *)L->w_gate + e * FE * rb_in, (const uint8_t *)L->w_up + e * FE * rb_in,
                       (const uint8_t *)L->w_down + e * E * rb_out, xr, E, FE, down + (size_t)j * E);
        }
        if (L->s_gate) expert_ffn(type, L->s_gate, L->s_up, L->s_down, xr, E, FE, shared);
        orc_combine(down, wts + (size_t)tt * NU, L->s_gate ? shared : NULL, L->w_shexp ? sg + tt : NULL,
                    out + (size_t)tt * E, NU, E, 1);
    }
    if (ids_out) memcpy(ids_out, ids, (size_t)t * NU * 4);
    if (wts_out) memcpy(wts_out, wts, (size_t)t * NU * 4);
    free(logits);
    free(ids);
    free(wts);
    free(sg);
    free(xr);
    free(down);
    free(shared);
    return 0;
}

/* Threads of the row loops (OpenMP over output rows; every row is computed alone, so the results do not depend on
 * the count). Returns the count in effect. */
int orc_set_threads(int n) {
    if (n > 0) omp_set_num_threads(n);
    return omp_get_max_threads();
}
