// fmx_internal.hpp — shared host and device helpers of libfmx (gfx950).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstring>

#include "fmx.h"

namespace fmx {

// ------------------------------------------------------------------ host --

// Host-side fault state (fm::BackendFault semantics, backend.cpp:258-277).
int current_fault();
void consume_fault(int fault);
// FMX_ERR_DEVICE_LOSS when a device loss is injected, else FMX_OK.
int fault_gate();

#define FMX_HIP_TRY(expr)                                                        \
    do {                                                                         \
        hipError_t fmx_e_ = (expr);                                              \
        if (fmx_e_ != hipSuccess) return ::fmx::status_of_hip(fmx_e_);           \
    } while (0)

#define FMX_LAUNCH_CHECK()                                                       \
    do {                                                                         \
        hipError_t fmx_e_ = hipGetLastError();                                   \
        if (fmx_e_ != hipSuccess) return ::fmx::status_of_hip(fmx_e_);           \
    } while (0)

int status_of_hip(hipError_t e);

// attention.hip: fmx_attention_decode after its pointer checks.
int attention_decode(const float *q, const float *kv, uint64_t row_stride, uint32_t v_offset, uint32_t heads,
                     uint32_t kv_heads, uint32_t head_dim, uint32_t positions, double scale, float *out,
                     uint32_t *status, hipStream_t s);

// Raises kernel `fn`'s dynamic LDS limit to `bytes` when above the 64 KiB
// default (gfx950 workgroups may use up to 160 KiB).
int allow_lds(const void *fn, size_t bytes);

__host__ __device__ inline uint64_t align_up(uint64_t v, uint64_t a) { return (v + a - 1) / a * a; }
__host__ __device__ inline uint32_t div_up(uint32_t a, uint32_t b) { return (a + b - 1) / b; }

// Packed layout of one [rows x cols] matrix: two regions, scales then quants,
// each 256-byte aligned. A "chunk" is what one lane loads per row per step
// (16 bytes of quants); 8 lanes load a row's 128-byte chunk together.
struct PackedGeometry {
    uint32_t type_id = 0;
    uint32_t rows = 0, cols = 0;
    uint32_t blocks = 0;          // quant blocks (Q4_K: super-blocks) per row
    uint32_t blocks_padded = 0;   // rounded up to whole chunks
    uint32_t chunks = 0;          // per row
    uint64_t scale_row_bytes = 0; // bytes of region A per row
    uint64_t scale_bytes = 0;     // region A, aligned
    uint64_t quant_bytes = 0;     // region B
    uint64_t total = 0;
};

// Fills `g`; FMX_ERR_UNSUPPORTED_QUANTISATION / FMX_ERR_SHAPE_MISMATCH on bad input.
int packed_geometry(uint32_t type_id, uint32_t rows, uint32_t cols, PackedGeometry *g);

// Raw block geometry (gguf.cpp:58-106) for the four types.
int raw_geometry(uint32_t type_id, uint32_t *block_size, uint32_t *block_bytes);

// Device error word bits (fmx_moe_status).
enum : uint32_t { STATUS_NONFINITE_SCORE = 1u, STATUS_BAD_EXPERT = 2u };

// ---------------------------------------------------------------- device --

// IEEE binary16 bits -> float. The hardware conversion is exact for every
// half, subnormals included (tests check all 65536 encodings).
__device__ __forceinline__ float half_bits_to_float(uint32_t bits16) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(bits16)));
}

__device__ __forceinline__ float fma_rn(float a, float b, float c) { return __builtin_fmaf(a, b, c); }

// Bytes 2w and 2w + 1 of a dword read as OCP E4M3 fp8 values (one
// v_cvt_pk_f32_fp8). A byte below 16 is the fp8 value byte * 2^-9 exactly.
template <bool kHighWord>
__device__ __forceinline__ float2 fp8_pair(uint32_t v) {
    typedef float f2 __attribute__((ext_vector_type(2)));
    const f2 r = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(v), kHighWord);
    return make_float2(r.x, r.y);
}

// Bytes 0, 1 (or, kHighWord, 2, 3) of v, each below 16, as the integers they
// hold, in one instruction: read as fp8 a byte below 16 is byte * 2^-9
// exactly, and v_cvt_scalef32_pk_f32_fp8 multiplies by the power of two in
// its scale operand's exponent (2^9), so the floats are exact whatever the
// other operand of the products they feed (all 16 values in every byte
// position checked on the GPU).
template <bool kHighWord>
__device__ __forceinline__ float2 nibble_pair(uint32_t v) {
    typedef float f2 __attribute__((ext_vector_type(2)));
    const f2 r = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(v, 0x1p9f, kHighWord);
    return make_float2(r.x, r.y);
}

// Value held by lane (lane ^ M), M in {1, 2, 4, 8}, by DPP moves inside each
// row of 16 lanes (VALU only; a shuffle through ds_bpermute would take the
// LDS pipeline and a wait): M = 1, 2 as quad permutations; M = 4 as
// row_shr:4 (lanes 4-7 of each 8 take lane - 4) overwritten on banks 0 and 2
// (lanes 0-3, 8-11) by row_shl:4 (lane + 4); M = 8 as row_ror:8.
template <int M>
__device__ __forceinline__ uint32_t lane_xor_u32(uint32_t v) {
    const int b = static_cast<int>(v);
    int r;
    // (every lane has its source lane for M = 1, 2, 8, so bound_ctrl changes
    // nothing there; set, it lets the compiler fold the move into the
    // instruction that consumes it, e.g. v_add_f32_dpp)
    if constexpr (M == 1) {
        r = __builtin_amdgcn_mov_dpp(b, 0xB1, 0xF, 0xF, true); // quad_perm [1,0,3,2]
    } else if constexpr (M == 2) {
        r = __builtin_amdgcn_mov_dpp(b, 0x4E, 0xF, 0xF, true); // quad_perm [2,3,0,1]
    } else if constexpr (M == 4) {
        const int hi = __builtin_amdgcn_mov_dpp(b, 0x114, 0xF, 0xF, false); // row_shr:4
        r = __builtin_amdgcn_update_dpp(hi, b, 0x104, 0xF, 0x5, false);     // row_shl:4, banks 0, 2
    } else {
        static_assert(M == 8, "lane_xor: mask 1, 2, 4 or 8");
        r = __builtin_amdgcn_mov_dpp(b, 0x128, 0xF, 0xF, true); // row_ror:8
    }
    return static_cast<uint32_t>(r);
}
template <int M>
__device__ __forceinline__ float lane_xor(float v) {
    return __builtin_bit_cast(float, lane_xor_u32<M>(__builtin_bit_cast(uint32_t, v)));
}
template <int M>
__device__ __forceinline__ uint64_t lane_xor_u64(uint64_t v) {
    return (static_cast<uint64_t>(lane_xor_u32<M>(static_cast<uint32_t>(v >> 32))) << 32) |
           lane_xor_u32<M>(static_cast<uint32_t>(v));
}

// The values of lanes i and i ^ M (M = 16 or 32), the lower lane's first,
// through the gfx950 permlane swaps (VALU): given v in both operands,
// v_permlane32_swap leaves v[i & 31] and v[32 + (i & 31)], v_permlane16_swap
// the even and the odd 16-lane row of i's half. A commutative operation on
// the two gives every lane the result of op(v_i, v_(i ^ M)).
template <int M>
__device__ __forceinline__ void lane_pair_u32(uint32_t v, uint32_t &a, uint32_t &b) {
    if constexpr (M == 32) {
        const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
        a = r[0];
        b = r[1];
    } else {
        static_assert(M == 16, "lane_pair: mask 16 or 32");
        const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
        a = r[0];
        b = r[1];
    }
}
template <int M>
__device__ __forceinline__ void lane_pair_u64(uint64_t v, uint64_t &a, uint64_t &b) {
    uint32_t alo, blo, ahi, bhi;
    lane_pair_u32<M>(static_cast<uint32_t>(v), alo, blo);
    lane_pair_u32<M>(static_cast<uint32_t>(v >> 32), ahi, bhi);
    a = (static_cast<uint64_t>(ahi) << 32) | alo;
    b = (static_cast<uint64_t>(bhi) << 32) | blo;
}

// Horizontal sum of t_l over the 8 lanes l = lane & 7 in the tree of the
// reference's _mm256 reduction: s_i = t_i + t_{i+4}; (s0 + s1) + (s2 + s3).
// Addition is commutative, so every lane of the group ends with the same bits.
__device__ __forceinline__ float hsum8_lanes(float t) {
    const float s = t + lane_xor<4>(t);
    const float a = s + lane_xor<1>(s);
    return a + lane_xor<2>(a);
}

// Lane M's value in every lane of each 16-lane row (DPP row_newbcast:M;
// bound_ctrl set so the move can fold into the instruction that consumes it).
template <uint32_t M>
__device__ __forceinline__ float row_bcast(float v) {
    static_assert(M < 16, "a lane of the 16-lane row");
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x150 + M, 0xF, 0xF, true));
}

// hsum8_lanes' value in lanes 0-3 of each 8-lane group only (the other four
// hold sums that mix in the neighbouring group), for callers that read lane
// 0 of each group: the first stage takes lane i + 4 by a rotation of the
// 16-lane row (row_ror:12: lane i reads lane (i - 12) mod 16) instead of the
// two masked moves of lane_xor<4>, so all three stages fold into DPP adds.
__device__ __forceinline__ float hsum8_first(float t) {
    const float r = __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, t), 0x12C, 0xF, 0xF, true));
    const float s = t + r;
    const float a = s + lane_xor<1>(s);
    return a + lane_xor<2>(a);
}

// Global-memory loads through an address-space-1 pointer. Expert slots are
// reached through a table of generic pointers, which the compiler would
// otherwise read with FLAT instructions; FLAT loads count against the LDS
// wait counter too, so every wait for an LDS read would also drain the
// weight prefetch.
typedef unsigned int fmx_u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int fmx_u32x2 __attribute__((ext_vector_type(2)));
typedef const __attribute__((address_space(1))) fmx_u32x4 fmx_global_u32x4;
typedef const __attribute__((address_space(1))) fmx_u32x2 fmx_global_u32x2;

__device__ __forceinline__ uint4 ld16(const void *p) {
    const fmx_u32x4 v = *(fmx_global_u32x4 *)(p);
    return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ uint2 ld8(const void *p) {
    const fmx_u32x2 v = *(fmx_global_u32x2 *)(p);
    return make_uint2(v.x, v.y);
}

// The same loads marked non-temporal (the nt cache policy: streamed data,
// read once), for the decode kernels' weight quants, so the expert stream
// does not evict what the token's kernels read again (the block scales that
// consecutive chunks share, the activations, h). Mixtral-shaped decode per
// 1000 tokens: Q4_0 53.9 -> 52.2 ms, Q8_0 88.4 -> 83.0 ms, Q4_K unchanged.
// The prefill GEMMs keep plain loads (nt: 0.74 -> 0.85 ms for 512 Q8_0
// tokens).
__device__ __forceinline__ uint4 ld16nt(const void *p) {
    const fmx_u32x4 v = __builtin_nontemporal_load((fmx_global_u32x4 *)(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ uint2 ld8nt(const void *p) {
    const fmx_u32x2 v = __builtin_nontemporal_load((fmx_global_u32x2 *)(p));
    return make_uint2(v.x, v.y);
}

__device__ __forceinline__ float ldf_nt(const float *p) {
    return __builtin_nontemporal_load((const __attribute__((address_space(1))) float *)(p));
}

// 6-bit scale/min pair j of a Q4_K super-block (quant.cpp:63-71).
__device__ __forceinline__ void k4_scale_min(int j, const uint8_t *q, uint32_t &sc, uint32_t &m) {
    if (j < 4) {
        sc = q[j] & 63u;
        m = q[j + 4] & 63u;
    } else {
        sc = (q[j + 4] & 0x0Fu) | ((q[j - 4] >> 6) << 4);
        m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
    }
}

} // namespace fmx
