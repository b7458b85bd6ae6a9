/*
 * fmoracle — CPU restatement of FreeMoe's MoE expert-layer arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker that the HIP path is
 * compared against; it is never linked into, called by or shipped with the
 * product library (libfmx). Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py load it.
 *
 * Every function follows a cited reference function (paths relative to the
 * FreeMoe tree). Two kernel orders are restated:
 *   FMO_ISA_SCALAR  KernelIsa::Scalar  (gemv_scalar, row_dot_fused_scalar)
 *   FMO_ISA_AVX2    KernelIsa::Avx2Fma (what KernelIsa::Auto resolves to on any
 *                   AVX2+FMA host): the 8-lane FMA chains of kernels.cpp, with
 *                   the contractions g++ 11.4 -O2 -ffp-contract=fast applies to
 *                   them written out as explicit fmaf() calls.
 *
 * Pinning (what checks each function; see tests/test_oracle_*.py):
 *   fmo_fp16_to_f32        all 65536 inputs vs hardware F16C conversion; the
 *                          reference's quant_reference.bin fixture
 *   fmo_dequantize_block   quant_reference.bin (records for F32, Q4_0, Q8_0,
 *                          Q4_K); closed forms over every nibble / int8 value /
 *                          6-bit scale code; the compiled reference (oracle/_ref)
 *   fmo_gemv               dequantise-then-gemv_scalar identity (1e-5, the
 *                          reference's own quant_gemv test); bitwise against the
 *                          compiled reference's gemv / gemv_quant for both ISAs
 *   fmo_rmsnorm, fmo_softmax, fmo_topk, fmo_route, fmo_moe_layer
 *                          closed forms and brute force on tiny inputs; bitwise
 *                          against goldens produced by the compiled reference
 *                          engine (tests/golden)
 *   fmo_moe_bucket         brute-force inversion of the routing table
 */
#ifndef FMORACLE_H
#define FMORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes: the same integers as fmx_status in include/fmx.h. */
enum {
    FMO_OK = 0,
    FMO_ERR_INVALID_ARGUMENT = 1,
    FMO_ERR_UNSUPPORTED_QUANTISATION = 2,
    FMO_ERR_SHAPE_MISMATCH = 3,
    FMO_ERR_INTERNAL = 4,
};

enum { FMO_ISA_SCALAR = 0, FMO_ISA_AVX2 = 1 };

/* GGUF tensor type ids handled on this path (gguf.cpp:58-106). */
enum { FMO_TYPE_F32 = 0, FMO_TYPE_Q4_0 = 2, FMO_TYPE_Q8_0 = 8, FMO_TYPE_Q4_K = 12, FMO_TYPE_Q6_K = 14 };

float fmo_fp16_to_f32(uint16_t h);
int fmo_quant_geometry(uint32_t type_id, uint32_t *block_size, uint32_t *block_bytes);
int fmo_dequantize_block(uint32_t type_id, const uint8_t *src, float *dst);
int fmo_dequantize_region(uint32_t type_id, const uint8_t *src, float *dst, uint64_t count);

/* y[out_dim] = W[out_dim x in_dim] * x, W stored row-major in type_id blocks. */
int fmo_gemv(int isa, uint32_t type_id, const uint8_t *weights, const float *x, float *y,
             uint32_t out_dim, uint32_t in_dim);

/* FNV-1a 64 of n bytes, continued from h0. */
uint64_t fmo_fnv1a64(uint64_t h0, const uint8_t *data, uint64_t n);

/* y[tokens x out_dim] = x[tokens x in_dim] * W^T (gemm_quant: each row
 * dequantised, then dot_isa per token). */
int fmo_gemm(int isa, uint32_t type_id, const uint8_t *weights, const float *x, float *y, uint32_t tokens,
             uint32_t out_dim, uint32_t in_dim);

int fmo_rmsnorm(const float *x, const float *w, uint32_t n, double eps, double norm_bias,
                float *y);
int fmo_softmax(const float *v, uint32_t n, float *out);
int fmo_topk(const float *scores, uint32_t n, uint32_t k, uint32_t *ids);

/* One routed MoE layer (freemoe-tiny / Mixtral semantics: softmax gating,
 * optional logit bias, optional top-k renormalisation). Expert e's weights are
 * gate[e] (F x H), up[e] (F x H) and down[e] (H x F), each in its own type. */
typedef struct {
    uint32_t hidden, ffn, experts, top_k;
    const float *norm_weight;      /* [hidden]; NULL = unit gain */
    double rms_eps;
    double norm_bias;              /* 1.0 for zero-centred norm weights, else 0 */
    uint32_t router_type;
    const uint8_t *router;         /* [experts x hidden] */
    const float *router_bias;      /* [experts] logit bias or NULL */
    int weights_norm;              /* expert_weights_norm */
    int epsilon_additive;          /* expert_weights_epsilon_additive */
    double weights_epsilon;        /* expert_weights_epsilon */
    double weights_scale;          /* expert_weights_scale */
    uint32_t gate_type, up_type, down_type;
    const uint8_t *const *gate;    /* [experts] */
    const uint8_t *const *up;
    const uint8_t *const *down;
} fmo_layer;

/* Routing only: h = rmsnorm(x), logits, probs, ids, weights. Any output
 * pointer except ids/weights may be NULL. */
int fmo_route(int isa, const fmo_layer *L, const float *x, float *h, float *logits,
              float *probs, uint32_t *ids, float *weights);

/* Whole layer for one token: out = x + sum_i w_i * down_i(swiglu(gate_i h, up_i h)).
 * act (optional, [top_k x ffn]) receives the SwiGLU activations in rank order. */
int fmo_moe_layer(int isa, const fmo_layer *L, const float *x, float *out, uint32_t *ids,
                  float *weights, float *h, float *act);

/* The expert half for a given routing (ids, weights in rank order) and the
 * residual: out = x + sum_i weights[i] * down_i(swiglu(gate_i h, up_i h)). */
int fmo_moe_experts(int isa, const fmo_layer *L, const float *x, const float *h, const uint32_t *ids,
                    const float *weights, float *out, float *act);

/* Per-token loop over a batch (the reference has no batched MoE path). */
int fmo_moe_layer_batch(int isa, const fmo_layer *L, const float *x, float *out,
                        uint32_t *ids, float *weights, uint32_t tokens);

/* Per-expert token lists from a routing table ids[tokens x top_k]:
 * offsets[experts+1] exclusive prefix sum of counts; for expert e the entries
 * offsets[e]..offsets[e+1]-1 of token_list/rank_list hold the tokens (ascending)
 * that selected e and the rank at which they did. */
int fmo_moe_bucket(const uint32_t *ids, uint32_t tokens, uint32_t top_k, uint32_t experts,
                   uint32_t *offsets, uint32_t *token_list, uint32_t *rank_list);

#ifdef __cplusplus
}
#endif

#endif
