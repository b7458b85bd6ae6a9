/*
 * fmoracle.c — CPU restatement of FreeMoe's MoE expert-layer arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP path, never part of it.
 * Build flags (oracle/Makefile): -O2 -mfma -ffp-contract=off, so that every
 * fused multiply-add below is an explicit fmaf() and nothing else is fused.
 *
 * Reference paths cited as file:line are relative to the FreeMoe tree.
 */
#include "fmoracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------ */
/* Scalars                                                                   */
/* ------------------------------------------------------------------------ */

/* IEEE binary16 -> binary32, exact (quant.cpp:23-48): subnormal halves are
 * renormalised, infinities and NaN payloads carried into the wider format. */
float fmo_fp16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1Fu;
    uint32_t man = h & 0x3FFu;
    uint32_t bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else {
            /* value = man * 2^-24; shift until the implicit bit appears */
            int e = -14;
            while (!(man & 0x400u)) {
                man <<= 1;
                --e;
            }
            man &= 0x3FFu;
            bits = sign | ((uint32_t)(e + 127) << 23) | (man << 13);
        }
    } else if (exp == 0x1F) {
        bits = sign | 0x7F800000u | (man << 13);
    } else {
        bits = sign | ((exp - 15 + 127) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

static uint16_t rd16(const uint8_t *p) {
    uint16_t v;
    memcpy(&v, p, 2);
    return v;
}

/* Block geometry for the types on this path (gguf.cpp:58-106). */
int fmo_quant_geometry(uint32_t type_id, uint32_t *block_size, uint32_t *block_bytes) {
    uint32_t bs, bb;
    switch (type_id) {
    case FMO_TYPE_F32: bs = 1; bb = 4; break;
    case FMO_TYPE_Q4_0: bs = 32; bb = 18; break;
    case FMO_TYPE_Q8_0: bs = 32; bb = 34; break;
    case FMO_TYPE_Q4_K: bs = 256; bb = 144; break;
    case FMO_TYPE_Q6_K: bs = 256; bb = 210; break;
    default: return FMO_ERR_UNSUPPORTED_QUANTISATION;
    }
    if (block_size) *block_size = bs;
    if (block_bytes) *block_bytes = bb;
    return FMO_OK;
}

/* 6-bit scale/min pair j of a Q4_K super-block (quant.cpp:63-71). */
static void k4_scale_min(int j, const uint8_t *q, uint8_t *sc, uint8_t *m) {
    if (j < 4) {
        *sc = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *sc = (uint8_t)((q[j + 4] & 0x0F) | ((q[j - 4] >> 6) << 4));
        *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

/* One block -> floats (quant.cpp:163-318, the F32/Q4_0/Q8_0/Q4_K cases). */
int fmo_dequantize_block(uint32_t type_id, const uint8_t *src, float *dst) {
    switch (type_id) {
    case FMO_TYPE_F32:
        memcpy(dst, src, 4);
        return FMO_OK;
    case FMO_TYPE_Q4_0: {
        /* f16 d; byte j: low nibble -> element j, high nibble -> j+16; d*(q-8) */
        const float d = fmo_fp16_to_f32(rd16(src));
        const uint8_t *qs = src + 2;
        for (int j = 0; j < 16; ++j) {
            dst[j] = d * (float)((int)(qs[j] & 0x0F) - 8);
            dst[j + 16] = d * (float)((int)(qs[j] >> 4) - 8);
        }
        return FMO_OK;
    }
    case FMO_TYPE_Q8_0: {
        const float d = fmo_fp16_to_f32(rd16(src));
        const int8_t *qs = (const int8_t *)(src + 2);
        for (int j = 0; j < 32; ++j) dst[j] = d * (float)qs[j];
        return FMO_OK;
    }
    case FMO_TYPE_Q4_K: {
        /* f16 d, f16 dmin, 12 B packed (sc,m)x8, 128 B nibbles. Group g uses
         * 32 bytes: low nibbles -> 64g+l with pair 2g, high -> 64g+32+l with
         * pair 2g+1; value (d*sc)*q - dmin*m. */
        const float d = fmo_fp16_to_f32(rd16(src));
        const float dmin = fmo_fp16_to_f32(rd16(src + 2));
        const uint8_t *scales = src + 4;
        const uint8_t *qs = src + 16;
        for (int g = 0; g < 4; ++g) {
            uint8_t sc, m;
            k4_scale_min(2 * g, scales, &sc, &m);
            const float d1 = d * (float)sc, m1 = dmin * (float)m;
            k4_scale_min(2 * g + 1, scales, &sc, &m);
            const float d2 = d * (float)sc, m2 = dmin * (float)m;
            for (int l = 0; l < 32; ++l) dst[64 * g + l] = d1 * (float)(qs[l] & 0x0F) - m1;
            for (int l = 0; l < 32; ++l) dst[64 * g + 32 + l] = d2 * (float)(qs[l] >> 4) - m2;
            qs += 32;
        }
        return FMO_OK;
    }
    case FMO_TYPE_Q6_K: {
        /* quant.cpp:347-371: 128 B low nibbles ql, 64 B high 2-bit pairs qh,
         * 16 int8 sub-block scales, f16 d. Two halves of 128 elements; in a
         * half, l < 32 gives elements l, l+32, l+64, l+96 from ql[l] / ql[l+32]
         * (low and high nibbles) and the four bit pairs of qh[l]; sub-block
         * scale is = l / 16 (+0, +2, +4, +6); value d * sc * (q - 32),
         * evaluated (d * sc) * q as the reference's left-to-right product. */
        const uint8_t *ql = src, *qh = src + 128;
        const int8_t *sc = (const int8_t *)(src + 192);
        const float d = fmo_fp16_to_f32(rd16(src + 208));
        float *y = dst;
        for (int n = 0; n < 256; n += 128) {
            for (int l = 0; l < 32; ++l) {
                const int is = l / 16;
                const int q1 = (int)((ql[l] & 0x0F) | (((qh[l] >> 0) & 3) << 4)) - 32;
                const int q2 = (int)((ql[l + 32] & 0x0F) | (((qh[l] >> 2) & 3) << 4)) - 32;
                const int q3 = (int)((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
                const int q4 = (int)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
                y[l] = d * (float)sc[is] * (float)q1;
                y[l + 32] = d * (float)sc[is + 2] * (float)q2;
                y[l + 64] = d * (float)sc[is + 4] * (float)q3;
                y[l + 96] = d * (float)sc[is + 6] * (float)q4;
            }
            y += 128;
            ql += 64;
            qh += 32;
            sc += 8;
        }
        return FMO_OK;
    }
    default:
        return FMO_ERR_UNSUPPORTED_QUANTISATION;
    }
}

/* quant.cpp:723-732 */
int fmo_dequantize_region(uint32_t type_id, const uint8_t *src, float *dst, uint64_t count) {
    uint32_t bs, bb;
    int rc = fmo_quant_geometry(type_id, &bs, &bb);
    if (rc) return rc;
    if (count % bs) return FMO_ERR_SHAPE_MISMATCH;
    for (uint64_t b = 0; b < count / bs; ++b) {
        rc = fmo_dequantize_block(type_id, src + b * bb, dst + b * bs);
        if (rc) return rc;
    }
    return FMO_OK;
}

/* ------------------------------------------------------------------------ */
/* Row dots                                                                  */
/* ------------------------------------------------------------------------ */

/* _mm256 horizontal sum as kernels.cpp hsum256 (kernels.cpp:600-605) and the
 * tails of gemv_avx2_row / row_dot_*_avx2: s_i = t_i + t_{i+4}, then
 * (s0 + s1) + (s2 + s3). IEEE addition is commutative, so only the tree
 * shape matters. */
static float hsum8(const float t[8]) {
    const float s0 = t[0] + t[4], s1 = t[1] + t[5], s2 = t[2] + t[6], s3 = t[3] + t[7];
    return (s0 + s1) + (s2 + s3);
}

/* gemv_scalar / dot_isa(Scalar) (kernels.cpp:132-140, 251-260): ascending k,
 * separate multiply and add (kernels.cpp is built without FMA outside its
 * target("avx2,fma") functions). */
static float dot_scalar(const float *a, const float *b, uint32_t n) {
    float acc = 0.0f;
    for (uint32_t k = 0; k < n; ++k) acc += a[k] * b[k];
    return acc;
}

/* gemv_avx2_row (kernels.cpp:147-167): two 8-lane FMA chains over 16-element
 * strides (acc0 takes k mod 16 < 8), an 8-element tail into acc0, lane-wise
 * acc0 + acc1, hsum, then a scalar tail contracted to FMA. */
static float dot_f32_avx2(const float *row, const float *x, uint32_t n) {
    float a0[8] = {0}, a1[8] = {0}, t[8];
    uint32_t k = 0;
    for (; k + 16 <= n; k += 16)
        for (int l = 0; l < 8; ++l) {
            a0[l] = fmaf(row[k + l], x[k + l], a0[l]);
            a1[l] = fmaf(row[k + 8 + l], x[k + 8 + l], a1[l]);
        }
    for (; k + 8 <= n; k += 8)
        for (int l = 0; l < 8; ++l) a0[l] = fmaf(row[k + l], x[k + l], a0[l]);
    for (int l = 0; l < 8; ++l) t[l] = a0[l] + a1[l];
    float total = hsum8(t);
    for (; k < n; ++k) total = fmaf(row[k], x[k], total);
    return total;
}

/* row_dot_q4_0_avx2 (kernels.cpp:673-694). Lane l of block b holds elements
 * l, 8+l (low nibbles of bytes l, 8+l) and 16+l, 24+l (their high nibbles):
 *   lo = fma(q[l], x[l], q[8+l]*x[8+l])        (g++ fuses the bytes 0..7 half)
 *   hi = fma(q'[l], x[16+l], q'[8+l]*x[24+l])
 *   c  = (lo + hi) - 8*((x[l]+x[8+l]) + (x[16+l]+x[24+l]))
 *   t[l] = fma(c, d, t[l]) */
static float dot_q4_0_avx2(const uint8_t *row, const float *x, uint32_t n) {
    float t[8] = {0};
    for (uint32_t b = 0; b < n / 32; ++b) {
        const uint8_t *blk = row + b * 18;
        const float d = fmo_fp16_to_f32(rd16(blk));
        const uint8_t *qs = blk + 2;
        const float *xb = x + b * 32;
        for (int l = 0; l < 8; ++l) {
            const float qa = (float)(qs[l] & 0x0F), qb = (float)(qs[8 + l] & 0x0F);
            const float qc = (float)(qs[l] >> 4), qd = (float)(qs[8 + l] >> 4);
            const float lo = fmaf(qa, xb[l], qb * xb[8 + l]);
            const float hi = fmaf(qc, xb[16 + l], qd * xb[24 + l]);
            const float sx = (xb[l] + xb[8 + l]) + (xb[16 + l] + xb[24 + l]);
            const float c = (lo + hi) - 8.0f * sx;
            t[l] = fmaf(c, d, t[l]);
        }
    }
    return hsum8(t);
}

/* row_dot_q8_0_avx2 (kernels.cpp:639-653): per block a 4-step FMA chain per
 * lane over elements l, 8+l, 16+l, 24+l from zero, then t = fma(acc, d, t). */
static float dot_q8_0_avx2(const uint8_t *row, const float *x, uint32_t n) {
    float t[8] = {0};
    for (uint32_t b = 0; b < n / 32; ++b) {
        const uint8_t *blk = row + b * 34;
        const float d = fmo_fp16_to_f32(rd16(blk));
        const int8_t *qs = (const int8_t *)(blk + 2);
        const float *xb = x + b * 32;
        for (int l = 0; l < 8; ++l) {
            float acc = 0.0f;
            for (int k = 0; k < 32; k += 8) acc = fmaf((float)qs[k + l], xb[k + l], acc);
            t[l] = fmaf(acc, d, t[l]);
        }
    }
    return hsum8(t);
}

/* row_dot_q4_k_avx2 (kernels.cpp:720-771). Per 64-element group: lane chains
 * over bytes l, 8+l, 16+l, 24+l of the group's 32 bytes (low nibbles against
 * x[k+l], high against x[32+k+l]); per-group sums of x; then in scalar
 *   part = fma(d*sc, hsum(acc), -((dmin*m) * hsum(sx)))   (g++ fuses this)
 *   total += part_lo + part_hi. */
static float dot_q4_k_avx2(const uint8_t *row, const float *x, uint32_t n) {
    float total = 0.0f;
    for (uint32_t b = 0; b < n / 256; ++b) {
        const uint8_t *blk = row + b * 144;
        const float d = fmo_fp16_to_f32(rd16(blk));
        const float dmin = fmo_fp16_to_f32(rd16(blk + 2));
        const uint8_t *scales = blk + 4;
        const uint8_t *qs = blk + 16;
        const float *xb = x + b * 256;
        for (int g = 0; g < 4; ++g) {
            uint8_t sc1, m1, sc2, m2;
            k4_scale_min(2 * g, scales, &sc1, &m1);
            k4_scale_min(2 * g + 1, scales, &sc2, &m2);
            const uint8_t *q = qs + 32 * g;
            const float *grp = xb + 64 * g;
            float alo[8] = {0}, ahi[8] = {0}, sxl[8], sxh[8];
            for (int k = 0; k < 32; k += 8)
                for (int l = 0; l < 8; ++l) {
                    alo[l] = fmaf((float)(q[k + l] & 0x0F), grp[k + l], alo[l]);
                    ahi[l] = fmaf((float)(q[k + l] >> 4), grp[32 + k + l], ahi[l]);
                }
            for (int l = 0; l < 8; ++l) {
                sxl[l] = (grp[l] + grp[8 + l]) + (grp[16 + l] + grp[24 + l]);
                sxh[l] = (grp[32 + l] + grp[40 + l]) + (grp[48 + l] + grp[56 + l]);
            }
            const float dsc1 = d * (float)sc1, dm1 = dmin * (float)m1;
            const float dsc2 = d * (float)sc2, dm2 = dmin * (float)m2;
            const float part_lo = fmaf(dsc1, hsum8(alo), -(dm1 * hsum8(sxl)));
            const float part_hi = fmaf(dsc2, hsum8(ahi), -(dm2 * hsum8(sxh)));
            total += part_lo + part_hi;
        }
    }
    return total;
}

/* row_dot_fused_scalar (kernels.cpp:574-590): decode one block, dot it in
 * ascending order from zero, add the block's dot to the running total. */
static float dot_fused_scalar(uint32_t type_id, const uint8_t *row, const float *x, uint32_t n) {
    uint32_t bs, bb;
    fmo_quant_geometry(type_id, &bs, &bb);
    float total = 0.0f, dec[256];
    for (uint32_t b = 0; b < n / bs; ++b) {
        fmo_dequantize_block(type_id, row + (uint64_t)b * bb, dec);
        total += dot_scalar(dec, x + (uint64_t)b * bs, bs);
    }
    return total;
}

/* row_dot_fused_scalar with the AVX2 ISA (kernels.cpp:574-590, selected by
 * select_row_dot for the block types without a dedicated kernel, e.g. Q6_K):
 * each block decoded, dotted by dot_avx2 (kernels.cpp:206-223), and the
 * block's dot added to the running total (a plain add: that function is
 * compiled without FMA). */
static float dot_fused_avx2(uint32_t type_id, const uint8_t *row, const float *x, uint32_t n) {
    uint32_t bs, bb;
    fmo_quant_geometry(type_id, &bs, &bb);
    float total = 0.0f, dec[256];
    for (uint32_t b = 0; b < n / bs; ++b) {
        fmo_dequantize_block(type_id, row + (uint64_t)b * bb, dec);
        total += dot_f32_avx2(dec, x + (uint64_t)b * bs, bs);
    }
    return total;
}

/* gemv (kernels.cpp:470-508) for F32 and gemv_quant (kernels.cpp:846-878)
 * for the block types. Threading splits rows only, so it never changes bits. */
int fmo_gemv(int isa, uint32_t type_id, const uint8_t *weights, const float *x, float *y,
             uint32_t out_dim, uint32_t in_dim) {
    if (out_dim == 0 || in_dim == 0) return FMO_OK;
    if (!weights || !x || !y) return FMO_ERR_INVALID_ARGUMENT;
    uint32_t bs, bb;
    int rc = fmo_quant_geometry(type_id, &bs, &bb);
    if (rc) return rc;
    if (in_dim % bs) return FMO_ERR_SHAPE_MISMATCH;
    const uint64_t row_bytes = (uint64_t)(in_dim / bs) * bb;
    for (uint32_t o = 0; o < out_dim; ++o) {
        const uint8_t *row = weights + (uint64_t)o * row_bytes;
        float v;
        if (isa == FMO_ISA_SCALAR) {
            v = type_id == FMO_TYPE_F32 ? dot_scalar((const float *)row, x, in_dim)
                                        : dot_fused_scalar(type_id, row, x, in_dim);
        } else {
            switch (type_id) {
            case FMO_TYPE_F32: v = dot_f32_avx2((const float *)row, x, in_dim); break;
            case FMO_TYPE_Q4_0: v = dot_q4_0_avx2(row, x, in_dim); break;
            case FMO_TYPE_Q8_0: v = dot_q8_0_avx2(row, x, in_dim); break;
            case FMO_TYPE_Q4_K: v = dot_q4_k_avx2(row, x, in_dim); break;
            default: v = dot_fused_avx2(type_id, row, x, in_dim); break;
            }
        }
        y[o] = v;
    }
    return FMO_OK;
}

/* gemm_quant / gemm_rows (kernels.cpp:289-345): every row dequantised
 * (dequantize_row) and dotted with each token's input by dot_isa
 * (kernels.cpp:251-260): dot_avx2 (kernels.cpp:206-223, the order of
 * gemv_avx2_row) for the AVX2 ISA, the plain multiply-add loop for the scalar
 * one. y is [tokens x out_dim], x [tokens x in_dim]. */
int fmo_gemm(int isa, uint32_t type_id, const uint8_t *weights, const float *x, float *y, uint32_t tokens,
             uint32_t out_dim, uint32_t in_dim) {
    if (tokens == 0 || out_dim == 0 || in_dim == 0) return FMO_OK;
    if (!weights || !x || !y) return FMO_ERR_INVALID_ARGUMENT;
    uint32_t bs, bb;
    int rc = fmo_quant_geometry(type_id, &bs, &bb);
    if (rc) return rc;
    if (in_dim % bs) return FMO_ERR_SHAPE_MISMATCH;
    const uint64_t row_bytes = (uint64_t)(in_dim / bs) * bb;
    float *rowf = (float *)malloc((size_t)in_dim * sizeof(float));
    if (!rowf) return FMO_ERR_INVALID_ARGUMENT;
    for (uint32_t o = 0; o < out_dim; ++o) {
        rc = fmo_dequantize_region(type_id, weights + (uint64_t)o * row_bytes, rowf, in_dim);
        if (rc) break;
        for (uint32_t t = 0; t < tokens; ++t) {
            const float *xt = x + (uint64_t)t * in_dim;
            y[(uint64_t)t * out_dim + o] =
                isa == FMO_ISA_SCALAR ? dot_scalar(rowf, xt, in_dim) : dot_f32_avx2(rowf, xt, in_dim);
        }
    }
    free(rowf);
    return rc;
}

/* FNV-1a 64 (the expert-slot checksum of residency.cpp:700-720 and the
 * native adapter's expert checksums): h = (h xor byte) * prime mod 2^64,
 * continued from h0 (the offset basis 14695981039346656037 for a new
 * payload). */
uint64_t fmo_fnv1a64(uint64_t h0, const uint8_t *data, uint64_t n) {
    uint64_t h = h0;
    for (uint64_t i = 0; i < n; ++i) h = (h ^ data[i]) * 1099511628211ull;
    return h;
}

/* ------------------------------------------------------------------------ */
/* Layer pieces                                                              */
/* ------------------------------------------------------------------------ */

/* rmsnorm lambda (engine.cpp:723-740): double sum of squares in index order,
 * s = 1/sqrt(ss/n + eps), gain = float(norm_bias + w), y = float(x*s*gain). */
int fmo_rmsnorm(const float *x, const float *w, uint32_t n, double eps, double norm_bias,
                float *y) {
    if (!x || !y || n == 0) return FMO_ERR_INVALID_ARGUMENT;
    double ss = 0.0;
    for (uint32_t i = 0; i < n; ++i) ss += (double)x[i] * x[i];
    const double scale = 1.0 / sqrt(ss / (double)n + eps);
    for (uint32_t i = 0; i < n; ++i) {
        const float gain = w ? (float)(norm_bias + (double)w[i]) : 1.0f;
        y[i] = (float)((double)x[i] * scale * (double)gain);
    }
    return FMO_OK;
}

/* Engine::softmax (engine.cpp:378-393): float max, double exponentials and
 * sum, float quotients; a non-finite input is an internal error. */
int fmo_softmax(const float *v, uint32_t n, float *out) {
    if (n == 0) return FMO_OK;
    float m = v[0];
    for (uint32_t i = 1; i < n; ++i)
        if (v[i] > m) m = v[i];
    double *e = (double *)malloc(sizeof(double) * n);
    if (!e) return FMO_ERR_INTERNAL;
    double sum = 0.0;
    for (uint32_t i = 0; i < n; ++i) {
        if (!isfinite(v[i])) {
            free(e);
            return FMO_ERR_INTERNAL;
        }
        e[i] = exp((double)v[i] - (double)m);
        sum += e[i];
    }
    for (uint32_t i = 0; i < n; ++i) out[i] = (float)(e[i] / sum);
    free(e);
    return FMO_OK;
}

/* Engine::topk (engine.cpp:395-411): stable descending order, ties to the
 * lower index. NaN or +inf among the scores is an internal error (only seen
 * when n >= 2, since a one-element sort compares nothing); k > n is an
 * invalid argument, checked after the sort. Selection by insertion: for each
 * rank take the best remaining index, the first one on ties. */
int fmo_topk(const float *s, uint32_t n, uint32_t k, uint32_t *ids) {
    if (n >= 2)
        for (uint32_t i = 0; i < n; ++i)
            if (isnan(s[i]) || s[i] == INFINITY) return FMO_ERR_INTERNAL;
    if (k > n) return FMO_ERR_INVALID_ARGUMENT;
    unsigned char *taken = (unsigned char *)calloc(n ? n : 1, 1);
    if (!taken) return FMO_ERR_INTERNAL;
    for (uint32_t r = 0; r < k; ++r) {
        uint32_t best = n;
        for (uint32_t i = 0; i < n; ++i) {
            if (taken[i]) continue;
            if (best == n || s[i] > s[best]) best = i;
        }
        taken[best] = 1;
        ids[r] = best;
    }
    free(taken);
    return FMO_OK;
}

/* Router -> gating -> top-k -> weights (engine.cpp:1603-1616, 1634-1639,
 * 1679-1702). */
int fmo_route(int isa, const fmo_layer *L, const float *x, float *h_out, float *logits_out,
              float *probs_out, uint32_t *ids, float *weights) {
    const uint32_t H = L->hidden, E = L->experts, K = L->top_k;
    float *h = (float *)malloc(sizeof(float) * H);
    float *logits = (float *)malloc(sizeof(float) * E);
    float *probs = (float *)malloc(sizeof(float) * E);
    int rc = FMO_ERR_INTERNAL;
    if (!h || !logits || !probs) goto done;
    rc = fmo_rmsnorm(x, L->norm_weight, H, L->rms_eps, L->norm_bias, h);
    if (rc) goto done;
    rc = fmo_gemv(isa, L->router_type, L->router, h, logits, E, H);
    if (rc) goto done;
    if (L->router_bias)
        for (uint32_t e = 0; e < E; ++e) logits[e] += L->router_bias[e];
    rc = fmo_softmax(logits, E, probs);
    if (rc) goto done;
    rc = fmo_topk(probs, E, K, ids);
    if (rc) goto done;
    {
        float total = 0.0f;
        for (uint32_t i = 0; i < K; ++i) {
            weights[i] = probs[ids[i]];
            total += weights[i];
        }
        if (L->weights_norm) {
            const double den = L->epsilon_additive ? (double)total + L->weights_epsilon
                                                   : fmax((double)total, L->weights_epsilon);
            for (uint32_t i = 0; i < K; ++i) weights[i] = (float)((double)weights[i] / den);
        }
        for (uint32_t i = 0; i < K; ++i)
            weights[i] = (float)((double)weights[i] * L->weights_scale);
    }
    if (h_out) memcpy(h_out, h, sizeof(float) * H);
    if (logits_out) memcpy(logits_out, logits, sizeof(float) * E);
    if (probs_out) memcpy(probs_out, probs, sizeof(float) * E);
done:
    free(h);
    free(logits);
    free(probs);
    return rc;
}

/* silu in double, rounded to float, times up in float (activation.hpp:33,
 * 38-54, 84). */
static float swiglu(float gate, float up) {
    const double g = (double)gate;
    return (float)(g / (1.0 + exp(-g))) * up;
}

/* The expert half of the MoE block for a given routing (engine.cpp:1710-1776)
 * and the residual add (engine.cpp:813-816, 1822): for each rank i in order,
 * gate/up of expert ids[i] on h, SwiGLU, down, ffn += weights[i] * down (a
 * multiply, then an add); out = x + ffn. */
int fmo_moe_experts(int isa, const fmo_layer *L, const float *x, const float *h, const uint32_t *ids,
                    const float *weights, float *out, float *act_out) {
    const uint32_t H = L->hidden, F = L->ffn, K = L->top_k;
    float *ffn = (float *)calloc(H, sizeof(float));
    float *gate = (float *)malloc(sizeof(float) * F);
    float *up = (float *)malloc(sizeof(float) * F);
    float *act = (float *)malloc(sizeof(float) * F);
    float *down = (float *)malloc(sizeof(float) * H);
    int rc = FMO_ERR_INTERNAL;
    if (!ffn || !gate || !up || !act || !down) goto done;
    for (uint32_t i = 0; i < K; ++i) {
        const uint32_t e = ids[i];
        if (e >= L->experts) {
            rc = FMO_ERR_INTERNAL;
            goto done;
        }
        rc = fmo_gemv(isa, L->gate_type, L->gate[e], h, gate, F, H);
        if (!rc) rc = fmo_gemv(isa, L->up_type, L->up[e], h, up, F, H);
        if (rc) goto done;
        for (uint32_t j = 0; j < F; ++j) act[j] = swiglu(gate[j], up[j]);
        if (act_out) memcpy(act_out + (uint64_t)i * F, act, sizeof(float) * F);
        rc = fmo_gemv(isa, L->down_type, L->down[e], act, down, H, F);
        if (rc) goto done;
        for (uint32_t j = 0; j < H; ++j) ffn[j] += weights[i] * down[j];
    }
    for (uint32_t j = 0; j < H; ++j) out[j] = x[j] + ffn[j];
    rc = FMO_OK;
done:
    free(ffn);
    free(gate);
    free(up);
    free(act);
    free(down);
    return rc;
}

/* The MoE block of Engine::forward_token (engine.cpp:1602-1776) and the
 * residual add: fmo_route, then fmo_moe_experts. */
int fmo_moe_layer(int isa, const fmo_layer *L, const float *x, float *out, uint32_t *ids,
                  float *weights, float *h_out, float *act_out) {
    float *h = (float *)malloc(sizeof(float) * L->hidden);
    if (!h) return FMO_ERR_INTERNAL;
    int rc = fmo_route(isa, L, x, h, NULL, NULL, ids, weights);
    if (!rc) rc = fmo_moe_experts(isa, L, x, h, ids, weights, out, act_out);
    if (!rc && h_out) memcpy(h_out, h, sizeof(float) * L->hidden);
    free(h);
    return rc;
}

int fmo_moe_layer_batch(int isa, const fmo_layer *L, const float *x, float *out,
                        uint32_t *ids, float *weights, uint32_t tokens) {
    for (uint32_t t = 0; t < tokens; ++t) {
        int rc = fmo_moe_layer(isa, L, x + (uint64_t)t * L->hidden, out + (uint64_t)t * L->hidden,
                               ids + (uint64_t)t * L->top_k, weights + (uint64_t)t * L->top_k,
                               NULL, NULL);
        if (rc) return rc;
    }
    return FMO_OK;
}

/* The reference has no bucketing; its routing record (engine.cpp:1707) is
 * inverted here: counts per expert, exclusive prefix sum, then tokens in
 * ascending order within each expert. */
int fmo_moe_bucket(const uint32_t *ids, uint32_t tokens, uint32_t top_k, uint32_t experts,
                   uint32_t *offsets, uint32_t *token_list, uint32_t *rank_list) {
    for (uint32_t e = 0; e <= experts; ++e) offsets[e] = 0;
    for (uint64_t i = 0; i < (uint64_t)tokens * top_k; ++i) {
        if (ids[i] >= experts) return FMO_ERR_INVALID_ARGUMENT;
        offsets[ids[i] + 1]++;
    }
    for (uint32_t e = 0; e < experts; ++e) offsets[e + 1] += offsets[e];
    uint32_t *fill = (uint32_t *)calloc(experts ? experts : 1, sizeof(uint32_t));
    if (!fill) return FMO_ERR_INTERNAL;
    for (uint32_t t = 0; t < tokens; ++t)
        for (uint32_t r = 0; r < top_k; ++r) {
            const uint32_t e = ids[(uint64_t)t * top_k + r];
            const uint32_t pos = offsets[e] + fill[e]++;
            token_list[pos] = t;
            rank_list[pos] = r;
        }
    free(fill);
    return FMO_OK;
}
