/*
 * fmx.h — C ABI of the MI355X (gfx950) MoE expert-layer library, libfmx.so.
 *
 * The library replaces FreeMoe's physical-GPU placeholder
 * (src/backend.cpp:528-571) and the CPU kernels the MoE block of
 * Engine::forward_token calls (src/engine.cpp:1466-1469, 1602-1776, 1822).
 * Each entry point below names the reference interface it stands in for.
 *
 * Conventions
 *   - Every function returns an fmx_status (0 = FMX_OK); nothing throws across
 *     the ABI. The integers follow the subset of fm::ErrorCode
 *     (include/fm/common.hpp:27-57) this path can raise; fmx_status_name()
 *     returns the reference's spelling.
 *   - Pointers documented as "device" are HBM addresses (from fmx_alloc or any
 *     other HIP allocation). `stream` is a hipStream_t (NULL = default stream).
 *     Compute entry points enqueue work and return; results are ready when the
 *     stream is synchronised (fmx_stream_sync) or a later fence completes.
 *   - Argument checks run on the host before anything is launched.
 *   - The library never allocates behind the caller's back on a compute call:
 *     scratch memory comes in through a workspace argument sized by the
 *     matching *_workspace_bytes() query.
 *
 * Weight layouts
 *   Raw      GGUF blocks, row-major [rows x cols] (gguf.cpp:58-106 geometry).
 *   Packed   the device layout the matvec/MoE kernels stream (fmx_pack()):
 *            per-lane byte streams so that every 16-byte load of a wavefront
 *            is aligned and fully used. Values are unchanged; only the byte
 *            order differs. F32 is not repacked (packed == raw).
 */
#ifndef FMX_H
#define FMX_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FMX_ABI_VERSION 1

typedef enum fmx_status {
    FMX_OK = 0,
    FMX_ERR_INVALID_ARGUMENT = 1,         /* INVALID_ARGUMENT */
    FMX_ERR_UNSUPPORTED_QUANTISATION = 2, /* UNSUPPORTED_QUANTISATION */
    FMX_ERR_SHAPE_MISMATCH = 3,           /* SHAPE_MISMATCH */
    FMX_ERR_INTERNAL = 4,                 /* INTERNAL_ERROR (e.g. non-finite router score) */
    FMX_ERR_ALLOCATION_FAILED = 5,        /* ALLOCATION_FAILED */
    FMX_ERR_TRANSFER_FAILED = 6,          /* TRANSFER_FAILED */
    FMX_ERR_FENCE_TIMEOUT = 7,            /* FENCE_TIMEOUT */
    FMX_ERR_DEVICE_LOSS = 8,              /* DEVICE_LOSS */
    FMX_ERR_NO_DEVICE = 9,                /* GPU_BACKEND_UNIMPLEMENTED: no usable gfx950 device */
    FMX_ERR_LAUNCH_FAILED = 10,           /* a HIP launch or runtime call failed */
} fmx_status;

/* Tensor type ids (GGUF, gguf.cpp:58-106) this library executes. */
enum { FMX_TYPE_F32 = 0, FMX_TYPE_Q4_0 = 2, FMX_TYPE_Q8_0 = 8, FMX_TYPE_Q4_K = 12, FMX_TYPE_Q6_K = 14 };

/* Faults forced from the host, as fm::BackendFault (include/fm/backend.hpp:118). */
enum { FMX_FAULT_NONE = 0, FMX_FAULT_TRANSFER = 1, FMX_FAULT_FENCE_DEFERRED = 2,
       FMX_FAULT_FENCE_TIMEOUT = 3, FMX_FAULT_DEVICE_LOSS = 4 };

int fmx_abi_version(void);
const char *fmx_status_name(int status);

/* ---------------------------------------------------------------- device -- */

typedef struct fmx_device_info {
    char name[64];              /* marketing name */
    char arch[32];              /* gcnArchName, e.g. "gfx950:sramecc+:xnack-" */
    uint64_t total_memory_bytes;
    uint64_t free_memory_bytes;
    uint32_t compute_units;
    uint32_t wavefront_size;
    uint32_t lds_bytes_per_cu;
    uint32_t clock_khz;
    uint32_t memory_clock_khz;
    uint32_t memory_bus_bits;
} fmx_device_info;

/* Backend::info() (include/fm/backend.hpp:22-36, 152). FMX_ERR_NO_DEVICE when
 * no gfx950 device is visible. */
int fmx_device_info_get(int ordinal, fmx_device_info *info);

/* Backend::allocate() (backend.hpp:153): HBM allocation, zero-filled. */
int fmx_alloc(uint64_t bytes, void **device_ptr);
int fmx_free(void *device_ptr);
/* Pinned host memory for the host mirror of a device buffer (the engine reads
 * DeviceBuffer::data on the host, engine.cpp:203, 330, 1733-1737). */
int fmx_host_alloc(uint64_t bytes, void **host_ptr);
int fmx_host_free(void *host_ptr);

/* Backend::upload() (backend.hpp:154): asynchronous H2D copy; *fence receives
 * an event recorded after the copy. */
int fmx_upload(void *device_dst, const void *host_src, uint64_t bytes, void *stream,
               void **fence);
int fmx_download(void *host_dst, const void *device_src, uint64_t bytes, void *stream);
/* Backend::fence_complete / wait_fence (backend.hpp:155-156). wait polls until
 * the fence completes or timeout_ms elapses (FMX_ERR_FENCE_TIMEOUT). */
int fmx_fence_query(void *fence, int *complete);
int fmx_fence_wait(void *fence, uint32_t timeout_ms);
int fmx_fence_release(void *fence);
int fmx_stream_sync(void *stream);

/* Backend::inject_fault / clear_faults (backend.hpp:160-161). Host-side only:
 * the next transfer / wait / compute call fails with the matching status, the
 * GPU itself is never touched. */
int fmx_inject_fault(int fault);
int fmx_clear_faults(void);

/* ---------------------------------------------------------- block types -- */

/* quant_geometry (include/fm/quant.hpp:19): elements and bytes per block. */
int fmx_quant_geometry(uint32_t type_id, uint32_t *block_size, uint32_t *block_bytes);

/* dequantize_tensor_region (include/fm/quant.hpp:30; quant.cpp:723-732):
 * `count` elements of raw blocks (device) -> F32 (device). */
int fmx_dequantize(uint32_t type_id, const void *raw, float *dst, uint64_t count, void *stream);

/* Bytes of the packed device layout of a [rows x cols] matrix. 0 on error. */
uint64_t fmx_packed_bytes(uint32_t type_id, uint32_t rows, uint32_t cols);
/* Raw (device) -> packed (device). Used when an expert slot is filled
 * (the slot payload the reference uploads in residency.cpp:681-696). */
int fmx_pack(uint32_t type_id, const void *raw, void *packed, uint32_t rows, uint32_t cols,
             void *stream);

/* Backend::matvec (backend.hpp:158-159) for F32 and gemv_quant
 * (include/fm/kernels.hpp:79; kernels.cpp:846-878) for the block types:
 * y[out_dim] = W x with W packed (device), x and y device F32. The result is
 * bit-identical to the reference's KernelIsa::Auto path on an AVX2+FMA host
 * (the per-lane FMA chains of kernels.cpp:147-167, 639-653, 673-694, 720-771). */
int fmx_matvec(uint32_t type_id, const void *packed, const float *x, float *y,
               uint32_t out_dim, uint32_t in_dim, void *stream);

/* gemm_quant (include/fm/kernels.hpp:68; kernels.cpp:289-345), the batched
 * product of the engine's dense prefill (engine.cpp:2007-2024):
 * y[t][o] = dot(dequantize_row(W row o), x[t]) for tokens t < `tokens`, W in
 * its raw GGUF rows (device, not packed), x [tokens x in_dim] and
 * y [tokens x out_dim] device F32. Bit-identical to the reference's
 * KernelIsa::Auto path (dot_avx2, kernels.cpp:206-223). No-op for a zero
 * dimension, as the reference. */
int fmx_gemm_quant(uint32_t type_id, const void *weights, const float *x, float *y, uint32_t tokens,
                   uint32_t out_dim, uint32_t in_dim, void *stream);

/* ------------------------------------------------------------ MoE layer -- */

/* One routed MoE layer with softmax gating (engine.cpp:1602-1776). All pointers
 * are device pointers. Expert e's packed projections are gate[e] (ffn x hidden),
 * up[e] (ffn x hidden) and down[e] (hidden x ffn): the three arrays are device
 * arrays of device pointers (the hot expert slot table), so the kernels find the
 * routed experts without a host round trip. */
typedef struct fmx_moe_layer {
    /* gate/up and down may hold different block types (e.g. Q4_K gate/up with
     * Q8_0 down); gate and up share one. */
    uint32_t hidden, ffn, experts, top_k;
    const float *norm_weight;     /* [hidden] RMSNorm gain, NULL = unit gain (16-byte aligned) */
    double rms_eps;               /* ModelConfig::rms_eps */
    double norm_bias;             /* 1.0 when norm weights are zero-centred */
    uint32_t router_type;         /* FMX_TYPE_F32, _Q4_0, _Q8_0, _Q4_K or _Q6_K (raw rows, hidden % 256 == 0) */
    const void *router;           /* [experts x hidden], 16-byte aligned: F32 raw row-major;
                                     a block type packed (fmx_pack), its logits then the
                                     gemv_quant row dots (engine.cpp:358-366) */
    const float *router_bias;     /* [experts] logit bias (ffn_gate_inp.bias) or NULL */
    int32_t weights_norm;         /* expert_weights_norm */
    int32_t epsilon_additive;     /* expert_weights_epsilon_additive */
    double weights_epsilon;       /* expert_weights_epsilon */
    double weights_scale;         /* expert_weights_scale */
    uint32_t gate_type, up_type, down_type;
    const void *const *gate;      /* device array [experts] of packed matrices (16-byte aligned) */
    const void *const *up;
    const void *const *down;
} fmx_moe_layer;

/* Workspace for fmx_moe_route / fmx_moe_decode / fmx_moe_prefill over
 * `tokens` tokens. */
uint64_t fmx_moe_workspace_bytes(const fmx_moe_layer *layer, uint32_t tokens);

/* RMSNorm -> router -> softmax -> stable top-k -> weights for `tokens`
 * independent rows of x ([tokens x hidden]). h receives the normalised rows,
 * ids/weights the routing in rank order ([tokens x top_k]); logits (optional,
 * [tokens x experts]) the router logits. Bit-identical to the reference. */
int fmx_moe_route(const fmx_moe_layer *layer, const float *x, uint32_t tokens, float *h,
                  float *logits, uint32_t *ids, float *weights, void *workspace,
                  uint64_t workspace_bytes, void *stream);

/* Decode: the whole layer for `tokens` rows of x processed one at a time, in
 * order (batch 1 each): out[t] = x[t] + sum_i w_i * down_i(SwiGLU(gate_i h,
 * up_i h)). ids/weights as fmx_moe_route. Matches the reference within its
 * own rounding (bit-identical except where two libm exp() results differ). */
int fmx_moe_decode(const fmx_moe_layer *layer, const float *x, float *out, uint32_t tokens,
                   uint32_t *ids, float *weights, void *workspace, uint64_t workspace_bytes,
                   void *stream);

/* fmx_moe_decode for callers that cannot allocate device memory (code under
 * HIP graph capture, serving loops, harnesses that forbid hipMalloc). No
 * counterpart in the reference. It allocates nothing: its workspace is a
 * device array of FMX_STATIC_SCRATCH_BYTES inside the library, one per GPU,
 * held until the process ends. A layer whose decode workspace
 * (fmx_moe_workspace_bytes(layer, 1)) exceeds that is refused with
 * FMX_ERR_SHAPE_MISMATCH before anything is launched. `status` (device, 4
 * bytes, may be NULL) receives the error word fmx_moe_status would read
 * (cleared first; bit 0: a non-finite router score, INTERNAL_ERROR; bit 1: an
 * expert id out of range, INVALID_ARGUMENT). Every call on one GPU shares
 * that GPU's array: calls that overlap on one GPU (two streams, two threads)
 * race and must be ordered by the caller. Results equal fmx_moe_decode's bit
 * for bit. */
#define FMX_STATIC_SCRATCH_BYTES (4u << 20)
int fmx_moe_decode_static(const fmx_moe_layer *layer, const float *x, float *out, uint32_t tokens,
                          uint32_t *ids, float *weights, uint32_t *status, void *stream);

/* Instrumented fmx_moe_decode (no reference counterpart; for measurement):
 * the same launches on `stream`, timed with HIP events: kernel_ms[0] sums the
 * interval between events recorded before and after each routing launch;
 * kernel_ms[1] and kernel_ms[2] sum the gate/up and down kernels' own
 * execution, between events their launches record at kernel start and end
 * (hipExtLaunchKernelGGL). Milliseconds over all tokens. Synchronises the
 * stream. */
int fmx_moe_decode_timed(const fmx_moe_layer *layer, const float *x, float *out, uint32_t tokens,
                         uint32_t *ids, float *weights, void *workspace, uint64_t workspace_bytes,
                         void *stream, double *kernel_ms);

/* Prefill: the whole layer for `tokens` rows of x ([tokens x hidden]) at once.
 * Routing is bit-identical to fmx_moe_route (ids / weights [tokens x top_k]);
 * the experts run as grouped GEMMs on bf16 MFMA over per-expert token lists
 * (fmx_moe_bucket's order): each lane loads its weight row's packed blocks
 * and dequantises them in registers into the MFMA's bf16 B operand, while the
 * gathered activations pass through LDS; outputs match the reference within
 * 2e-2 relative (bf16 operands, f32 accumulation). The reference has no batched MoE path: it runs its decode
 * step once per prompt token (engine.cpp:1870, 2395-2399); this replaces that
 * loop. Shapes the GEMMs do not tile (and F32 experts) run the decode expert
 * kernels token by token instead, on the GPU. */
uint64_t fmx_moe_prefill_workspace_bytes(const fmx_moe_layer *layer, uint32_t tokens);
int fmx_moe_prefill(const fmx_moe_layer *layer, const float *x, float *out, uint32_t tokens,
                    uint32_t *ids, float *weights, void *workspace, uint64_t workspace_bytes,
                    void *stream);

/* Instrumented fmx_moe_prefill (no reference counterpart; for measurement):
 * the same launches on `stream`; kernel_ms[0] and kernel_ms[1] receive the
 * gate/up and the down grouped GEMM's own execution time, between events
 * their launches record at kernel start and end (hipExtLaunchKernelGGL), in
 * milliseconds. Synchronises the stream. FMX_ERR_SHAPE_MISMATCH when the
 * grouped GEMMs do not run (no tokens, or a shape they do not tile). */
int fmx_moe_prefill_timed(const fmx_moe_layer *layer, const float *x, float *out, uint32_t tokens,
                          uint32_t *ids, float *weights, void *workspace, uint64_t workspace_bytes,
                          void *stream, double *kernel_ms);

/* Device error word written by the routing kernels (non-finite score or an
 * expert id out of range): reads and clears it, blocking on `stream`. */
int fmx_moe_status(void *workspace, void *stream);

/* The error word of `workspace` queued for copy into *host_word and cleared,
 * in stream order, without waiting: *host_word holds it once the stream has
 * been synchronised (host_word from fmx_host_alloc, so the copy runs
 * asynchronously), and fmx_moe_status_of turns it into the status
 * fmx_moe_status returns. Lets a caller that synchronises for its outputs
 * anyway read the word in the same wait. No counterpart in the reference,
 * whose kernels raise on the host. */
int fmx_moe_status_copy(void *workspace, uint32_t *host_word, void *stream);
int fmx_moe_status_of(uint32_t word);

/* Per-expert token lists from a routing table ids[tokens x top_k] (device):
 * offsets[experts+1], token_list/rank_list[tokens*top_k] as the reference's
 * routing record (engine.cpp:1707) inverted: tokens ascending within each
 * expert, with the rank at which each chose it. Deterministic (no atomic slot
 * grabs). experts <= 256. A token's ids must be distinct, as top-k makes them
 * (engine.cpp:395-411). An id >= experts, or a token that lists one expert
 * twice, is reported as FMX_ERR_INVALID_ARGUMENT by fmx_moe_status on the same
 * workspace (>= 256 bytes); the lists are then not meaningful. */
int fmx_moe_bucket(const uint32_t *ids, uint32_t tokens, uint32_t top_k, uint32_t experts,
                   uint32_t *offsets, uint32_t *token_list, uint32_t *rank_list, void *workspace,
                   uint64_t workspace_bytes, void *stream);

/* Decode attention of one token over its `positions` cached positions, the
 * full-context multi-head / grouped-query case of the engine's attention loop
 * (engine.cpp:1360-1420; replaces its per-head host loop behind
 * fm::HipBackend::attention). kv: the layer's cache on the device, position
 * t's row at kv + t * row_stride floats holding every kv head's key, the
 * values at + v_offset; q and out: [heads x head_dim] floats; scale: the
 * score scale (1 / sqrt(head_dim)). Per head: scores float(double dot * scale)
 * with the dot summed in index order, the engine's softmax (float maximum,
 * double exponentials summed in position order), values summed in double in
 * position order. Only exp is the device's own (within an ulp of the host
 * libm's). heads % kv_heads == 0, head_dim <= 256 and % 4 == 0, positions
 * <= 8192, pointers 16-byte aligned. workspace (>= 256 bytes): its first
 * word receives the error word; a non-finite score (INTERNAL_ERROR in the
 * engine) is reported by fmx_moe_status on it. */
int fmx_attention_decode(const float *q, const float *kv, uint64_t row_stride, uint32_t v_offset,
                         uint32_t heads, uint32_t kv_heads, uint32_t head_dim, uint32_t positions,
                         double scale, float *out, void *workspace, uint64_t workspace_bytes, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* FMX_H */
