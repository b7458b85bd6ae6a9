// quant.hip — block geometry, dequantisation and the packed device layout.
//
// Dequantisation follows dequantize_block (quant.cpp:163-371) for F32, Q4_0,
// Q8_0, Q4_K and Q6_K. Every product there is exact in float (Q4_0/Q8_0: an
// 11-bit half times a small integer; Q4_K: d*sc <= 17 bits times a nibble;
// Q6_K: d*sc <= 18 bits times |q| <= 32), so the only rounding is Q4_K's final
// subtraction and the decoded values are the reference's bit for bit.
#include "fmx_internal.hpp"

namespace fmx {

int raw_geometry(uint32_t type_id, uint32_t *block_size, uint32_t *block_bytes) {
    uint32_t bs, bb;
    switch (type_id) {
    case FMX_TYPE_F32: bs = 1; bb = 4; break;
    case FMX_TYPE_Q4_0: bs = 32; bb = 18; break;
    case FMX_TYPE_Q8_0: bs = 32; bb = 34; break;
    case FMX_TYPE_Q4_K: bs = 256; bb = 144; break;
    case FMX_TYPE_Q6_K: bs = 256; bb = 210; break;
    default: return FMX_ERR_UNSUPPORTED_QUANTISATION;
    }
    if (block_size) *block_size = bs;
    if (block_bytes) *block_bytes = bb;
    return FMX_OK;
}

// Packed layouts (one [rows x cols] matrix):
//   Q4_0  A: f16 d[rows][Bp]             B: [rows][Bp/8][lane 0..7][16 B]
//         lane l's 16 B for blocks 8c..8c+7: bytes (2j, 2j+1) = (qs[l], qs[8+l])
//         of block 8c+j, i.e. the nibbles of elements l, 16+l and 8+l, 24+l.
//   Q8_0  A: f16 d[rows][Bp]             B: [rows][Bp/4][lane][16 B]
//         lane l's bytes 4j..4j+3 = qs[l], qs[8+l], qs[16+l], qs[24+l] of block 4c+j.
//   Q4_K  A: [rows][S][16 B] header (d, dmin, 12 B scales) B: [rows][S][lane][16 B]
//         lane l's bytes 4g+k = qs[32g + 8k + l] (group g, k = 0..3).
//   F32   raw row-major, no packing.
//   Q6_K  raw rows (its matvec and batched product read the GGUF blocks).
// Block-type layouts end with kPackedTail spare bytes: the decode streams
// request up to 8 chunks (1 KiB) past a row's last chunk before they know the
// row has ended, and the last row's requests must stay inside the allocation.
constexpr uint64_t kPackedTail = 4096;

int packed_geometry(uint32_t type_id, uint32_t rows, uint32_t cols, PackedGeometry *g) {
    uint32_t bs, bb;
    int rc = raw_geometry(type_id, &bs, &bb);
    if (rc) return rc;
    if (rows == 0 || cols == 0) return FMX_ERR_INVALID_ARGUMENT;
    if (cols % bs) return FMX_ERR_SHAPE_MISMATCH;
    PackedGeometry p;
    p.type_id = type_id;
    p.rows = rows;
    p.cols = cols;
    p.blocks = cols / bs;
    switch (type_id) {
    case FMX_TYPE_F32:
        p.blocks_padded = p.blocks;
        p.chunks = 0;
        p.total = static_cast<uint64_t>(rows) * cols * 4;
        break;
    case FMX_TYPE_Q4_0:
    case FMX_TYPE_Q8_0: {
        const uint32_t per_chunk = type_id == FMX_TYPE_Q4_0 ? 8 : 4;
        p.blocks_padded = div_up(p.blocks, per_chunk) * per_chunk;
        p.chunks = p.blocks_padded / per_chunk;
        p.scale_row_bytes = static_cast<uint64_t>(p.blocks_padded) * 2;
        p.scale_bytes = align_up(p.scale_row_bytes * rows, 256);
        p.quant_bytes = static_cast<uint64_t>(rows) * p.chunks * 128;
        p.total = p.scale_bytes + align_up(p.quant_bytes, 256) + kPackedTail;
        break;
    }
    case FMX_TYPE_Q4_K:
        p.blocks_padded = p.blocks;
        p.chunks = p.blocks;
        p.scale_row_bytes = static_cast<uint64_t>(p.blocks) * 16;
        p.scale_bytes = align_up(p.scale_row_bytes * rows, 256);
        p.quant_bytes = static_cast<uint64_t>(rows) * p.chunks * 128;
        p.total = p.scale_bytes + align_up(p.quant_bytes, 256) + kPackedTail;
        break;
    case FMX_TYPE_Q6_K:
        p.blocks_padded = p.blocks;
        p.chunks = p.blocks;
        p.quant_bytes = static_cast<uint64_t>(rows) * p.blocks * bb;
        p.total = p.quant_bytes;
        break;
    }
    *g = p;
    return FMX_OK;
}

namespace {

// One thread per (row, chunk, lane): gathers that lane's 16 bytes.
__global__ void pack_q4_0_kernel(const uint8_t *__restrict__ raw, uint8_t *__restrict__ packed,
                                 uint32_t rows, uint32_t blocks, uint32_t blocks_padded,
                                 uint32_t chunks, uint64_t scale_bytes) {
    const uint64_t gid = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    const uint64_t total = static_cast<uint64_t>(rows) * chunks * 8;
    if (gid >= total) return;
    const uint32_t l = gid & 7;
    const uint64_t rc = gid >> 3;
    const uint32_t c = rc % chunks;
    const uint32_t r = rc / chunks;
    const uint8_t *row = raw + static_cast<uint64_t>(r) * blocks * 18;
    uint8_t out[16];
    uint8_t sc[2] = {0, 0};
    for (int j = 0; j < 8; ++j) {
        const uint32_t b = c * 8 + j;
        if (b < blocks) {
            const uint8_t *blk = row + static_cast<uint64_t>(b) * 18;
            out[2 * j] = blk[2 + l];
            out[2 * j + 1] = blk[2 + 8 + l];
            if (l == 0) {
                uint8_t *scales = packed + static_cast<uint64_t>(r) * blocks_padded * 2;
                scales[2 * b] = blk[0];
                scales[2 * b + 1] = blk[1];
            }
        } else {
            out[2 * j] = 0;
            out[2 * j + 1] = 0;
            if (l == 0) {
                uint8_t *scales = packed + static_cast<uint64_t>(r) * blocks_padded * 2;
                scales[2 * b] = sc[0];
                scales[2 * b + 1] = sc[1];
            }
        }
    }
    uint8_t *dst = packed + scale_bytes + (rc * 8 + l) * 16;
    for (int i = 0; i < 16; ++i) dst[i] = out[i];
}

__global__ void pack_q8_0_kernel(const uint8_t *__restrict__ raw, uint8_t *__restrict__ packed,
                                 uint32_t rows, uint32_t blocks, uint32_t blocks_padded,
                                 uint32_t chunks, uint64_t scale_bytes) {
    const uint64_t gid = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    const uint64_t total = static_cast<uint64_t>(rows) * chunks * 8;
    if (gid >= total) return;
    const uint32_t l = gid & 7;
    const uint64_t rc = gid >> 3;
    const uint32_t c = rc % chunks;
    const uint32_t r = rc / chunks;
    const uint8_t *row = raw + static_cast<uint64_t>(r) * blocks * 34;
    uint8_t *scales = packed + static_cast<uint64_t>(r) * blocks_padded * 2;
    uint8_t *dst = packed + scale_bytes + (rc * 8 + l) * 16;
    for (int j = 0; j < 4; ++j) {
        const uint32_t b = c * 4 + j;
        const bool real = b < blocks;
        const uint8_t *blk = row + static_cast<uint64_t>(b) * 34;
        for (int k = 0; k < 4; ++k) dst[4 * j + k] = real ? blk[2 + 8 * k + l] : 0;
        if (l == 0) {
            scales[2 * b] = real ? blk[0] : 0;
            scales[2 * b + 1] = real ? blk[1] : 0;
        }
    }
}

__global__ void pack_q4_k_kernel(const uint8_t *__restrict__ raw, uint8_t *__restrict__ packed,
                                 uint32_t rows, uint32_t blocks, uint64_t scale_bytes) {
    const uint64_t gid = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    const uint64_t total = static_cast<uint64_t>(rows) * blocks * 8;
    if (gid >= total) return;
    const uint32_t l = gid & 7;
    const uint64_t rb = gid >> 3; // row * blocks + block
    const uint8_t *blk = raw + rb * 144;
    uint8_t *dst = packed + scale_bytes + (rb * 8 + l) * 16;
    for (int g = 0; g < 4; ++g)
        for (int k = 0; k < 4; ++k) dst[4 * g + k] = blk[16 + 32 * g + 8 * k + l];
    if (l < 4) {
        uint8_t *hdr = packed + rb * 16;
        for (int i = 0; i < 4; ++i) hdr[4 * l + i] = blk[4 * l + i];
    }
}

// Q6_K (quant.cpp:347-371): two halves of 128 elements; in a half, l < 32
// gives elements l, l+32, l+64, l+96 from the low / high nibbles of ql[l] and
// ql[l+32] and the four bit pairs of qh[l], with sub-block scales
// sc[l/16 + 0, 2, 4, 6]; value (d * sc) * (q - 32).
__device__ inline void q6_k_block(const uint8_t *blk, float *o) {
    const float d = half_bits_to_float(blk[208] | (blk[209] << 8));
    for (int n = 0; n < 2; ++n) {
        const uint8_t *ql = blk + 64 * n, *qh = blk + 128 + 32 * n;
        const int8_t *sc = reinterpret_cast<const int8_t *>(blk + 192 + 8 * n);
        float *y = o + 128 * n;
        for (int l = 0; l < 32; ++l) {
            const int is = l / 16;
            const int q1 = static_cast<int>((ql[l] & 0x0F) | (((qh[l] >> 0) & 3) << 4)) - 32;
            const int q2 = static_cast<int>((ql[l + 32] & 0x0F) | (((qh[l] >> 2) & 3) << 4)) - 32;
            const int q3 = static_cast<int>((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
            const int q4 = static_cast<int>((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
            y[l] = d * static_cast<float>(sc[is]) * static_cast<float>(q1);
            y[l + 32] = d * static_cast<float>(sc[is + 2]) * static_cast<float>(q2);
            y[l + 64] = d * static_cast<float>(sc[is + 4]) * static_cast<float>(q3);
            y[l + 96] = d * static_cast<float>(sc[is + 6]) * static_cast<float>(q4);
        }
    }
}

// One thread per block (dequantize_block).
__global__ void dequant_kernel(uint32_t type_id, const uint8_t *__restrict__ raw,
                               float *__restrict__ dst, uint64_t blocks) {
    const uint64_t b = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (b >= blocks) return;
    switch (type_id) {
    case FMX_TYPE_F32: {
        float v;
        memcpy(&v, raw + b * 4, 4);
        dst[b] = v;
        break;
    }
    case FMX_TYPE_Q4_0: {
        const uint8_t *blk = raw + b * 18;
        const float d = half_bits_to_float(blk[0] | (blk[1] << 8));
        float *o = dst + b * 32;
        for (int j = 0; j < 16; ++j) {
            o[j] = d * static_cast<float>(static_cast<int>(blk[2 + j] & 0x0F) - 8);
            o[j + 16] = d * static_cast<float>(static_cast<int>(blk[2 + j] >> 4) - 8);
        }
        break;
    }
    case FMX_TYPE_Q8_0: {
        const uint8_t *blk = raw + b * 34;
        const float d = half_bits_to_float(blk[0] | (blk[1] << 8));
        float *o = dst + b * 32;
        for (int j = 0; j < 32; ++j) o[j] = d * static_cast<float>(static_cast<int8_t>(blk[2 + j]));
        break;
    }
    case FMX_TYPE_Q4_K: {
        const uint8_t *blk = raw + b * 144;
        const float d = half_bits_to_float(blk[0] | (blk[1] << 8));
        const float dmin = half_bits_to_float(blk[2] | (blk[3] << 8));
        const uint8_t *scales = blk + 4;
        const uint8_t *qs = blk + 16;
        float *o = dst + b * 256;
        for (int g = 0; g < 4; ++g) {
            uint32_t sc, m;
            k4_scale_min(2 * g, scales, sc, m);
            const float d1 = d * static_cast<float>(sc), m1 = dmin * static_cast<float>(m);
            k4_scale_min(2 * g + 1, scales, sc, m);
            const float d2 = d * static_cast<float>(sc), m2 = dmin * static_cast<float>(m);
            for (int l = 0; l < 32; ++l) o[64 * g + l] = d1 * static_cast<float>(qs[32 * g + l] & 0x0F) - m1;
            for (int l = 0; l < 32; ++l) o[64 * g + 32 + l] = d2 * static_cast<float>(qs[32 * g + l] >> 4) - m2;
        }
        break;
    }
    case FMX_TYPE_Q6_K:
        q6_k_block(raw + b * 210, dst + b * 256);
        break;
    default:
        break;
    }
}

} // namespace
} // namespace fmx

using namespace fmx;

extern "C" int fmx_quant_geometry(uint32_t type_id, uint32_t *block_size, uint32_t *block_bytes) {
    return raw_geometry(type_id, block_size, block_bytes);
}

extern "C" uint64_t fmx_packed_bytes(uint32_t type_id, uint32_t rows, uint32_t cols) {
    PackedGeometry g;
    if (packed_geometry(type_id, rows, cols, &g)) return 0;
    return g.total;
}

extern "C" int fmx_pack(uint32_t type_id, const void *raw, void *packed, uint32_t rows,
                        uint32_t cols, void *stream) {
    if (int rc = fault_gate()) return rc;
    PackedGeometry g;
    if (int rc = packed_geometry(type_id, rows, cols, &g)) return rc;
    if (!raw || !packed) return FMX_ERR_INVALID_ARGUMENT;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const uint8_t *src = static_cast<const uint8_t *>(raw);
    uint8_t *dst = static_cast<uint8_t *>(packed);
    const uint32_t threads = 256;
    switch (type_id) {
    case FMX_TYPE_F32:
    case FMX_TYPE_Q6_K:
        FMX_HIP_TRY(hipMemcpyAsync(dst, src, g.total, hipMemcpyDeviceToDevice, s));
        return FMX_OK;
    case FMX_TYPE_Q4_0: {
        const uint64_t n = static_cast<uint64_t>(rows) * g.chunks * 8;
        hipLaunchKernelGGL(pack_q4_0_kernel, dim3(static_cast<uint32_t>((n + threads - 1) / threads)),
                           dim3(threads), 0, s, src, dst, rows, g.blocks, g.blocks_padded, g.chunks,
                           g.scale_bytes);
        break;
    }
    case FMX_TYPE_Q8_0: {
        const uint64_t n = static_cast<uint64_t>(rows) * g.chunks * 8;
        hipLaunchKernelGGL(pack_q8_0_kernel, dim3(static_cast<uint32_t>((n + threads - 1) / threads)),
                           dim3(threads), 0, s, src, dst, rows, g.blocks, g.blocks_padded, g.chunks,
                           g.scale_bytes);
        break;
    }
    case FMX_TYPE_Q4_K: {
        const uint64_t n = static_cast<uint64_t>(rows) * g.blocks * 8;
        hipLaunchKernelGGL(pack_q4_k_kernel, dim3(static_cast<uint32_t>((n + threads - 1) / threads)),
                           dim3(threads), 0, s, src, dst, rows, g.blocks, g.scale_bytes);
        break;
    }
    }
    FMX_LAUNCH_CHECK();
    return FMX_OK;
}

extern "C" int fmx_dequantize(uint32_t type_id, const void *raw, float *dst, uint64_t count,
                              void *stream) {
    if (int rc = fault_gate()) return rc;
    uint32_t bs, bb;
    if (int rc = raw_geometry(type_id, &bs, &bb)) return rc;
    if (count % bs) return FMX_ERR_SHAPE_MISMATCH;
    if (count == 0) return FMX_OK;
    if (!raw || !dst) return FMX_ERR_INVALID_ARGUMENT;
    const uint64_t blocks = count / bs;
    const uint32_t threads = 256;
    hipLaunchKernelGGL(dequant_kernel, dim3(static_cast<uint32_t>((blocks + threads - 1) / threads)),
                       dim3(threads), 0, static_cast<hipStream_t>(stream), type_id,
                       static_cast<const uint8_t *>(raw), dst, blocks);
    FMX_LAUNCH_CHECK();
    return FMX_OK;
}
