"""numpy statement of libfmx's packed device layout (include/fmx.h, quant.hip).

Used to check fmx_pack's output byte for byte and, on the CPU, that the layout
is a pure permutation of the raw GGUF bytes (unpack(pack(raw)) == raw).
"""
import numpy as np

Q4_0, Q8_0, Q4_K, F32, Q6_K = 2, 8, 12, 0, 14
# zero bytes after a block-type layout (room for the decode streams' prefetch)
PACKED_TAIL = 4096


def _align(v, a=256):
    return (v + a - 1) // a * a


def pack(type_id: int, raw: np.ndarray, rows: int, cols: int) -> np.ndarray:
    raw = np.ascontiguousarray(raw, np.uint8).reshape(rows, -1)
    if type_id in (F32, Q6_K):  # raw rows
        return raw.reshape(-1).copy()
    if type_id in (Q4_0, Q8_0):
        bb, per = (18, 8) if type_id == Q4_0 else (34, 4)
        nb = cols // 32
        bp = -(-nb // per) * per
        chunks = bp // per
        blk = np.zeros((rows, bp, bb), np.uint8)
        blk[:, :nb] = raw.reshape(rows, nb, bb)
        scales = blk[:, :, 0:2].reshape(rows, bp * 2)
        qs = blk[:, :, 2:].reshape(rows, chunks, per, bb - 2)
        lanes = np.empty((rows, chunks, 8, 16), np.uint8)
        for l in range(8):
            if type_id == Q4_0:
                # bytes (2j, 2j+1) = (qs[l], qs[8+l]) of block j of the chunk
                lanes[:, :, l, 0::2] = qs[:, :, :, l]
                lanes[:, :, l, 1::2] = qs[:, :, :, 8 + l]
            else:
                # bytes 4j + k = qs[8k + l] of block j
                for k in range(4):
                    lanes[:, :, l, k::4] = qs[:, :, :, 8 * k + l]
        sbytes = _align(rows * bp * 2)
        out = np.zeros(sbytes + _align(lanes.size) + PACKED_TAIL, np.uint8)
        out[:rows * bp * 2] = scales.reshape(-1)
        out[sbytes:sbytes + lanes.size] = lanes.reshape(-1)
        return out
    if type_id == Q4_K:
        nb = cols // 256
        blk = raw.reshape(rows, nb, 144)
        hdr = blk[:, :, 0:16]
        qs = blk[:, :, 16:].reshape(rows, nb, 4, 4, 8)  # [g][k][l]
        lanes = np.transpose(qs, (0, 1, 4, 2, 3)).reshape(rows, nb, 8, 16)  # [l][g*4+k]
        sbytes = _align(rows * nb * 16)
        out = np.zeros(sbytes + _align(lanes.size) + PACKED_TAIL, np.uint8)
        out[:rows * nb * 16] = hdr.reshape(-1)
        out[sbytes:sbytes + lanes.size] = lanes.reshape(-1)
        return out
    raise ValueError(type_id)


def unpack(type_id: int, packed: np.ndarray, rows: int, cols: int) -> np.ndarray:
    if type_id in (F32, Q6_K):
        return packed.reshape(rows, -1).copy()
    if type_id in (Q4_0, Q8_0):
        bb, per = (18, 8) if type_id == Q4_0 else (34, 4)
        nb = cols // 32
        bp = -(-nb // per) * per
        chunks = bp // per
        sbytes = _align(rows * bp * 2)
        scales = packed[:rows * bp * 2].reshape(rows, bp, 2)
        lanes = packed[sbytes:sbytes + rows * chunks * 128].reshape(rows, chunks, 8, 16)
        qs = np.empty((rows, chunks, per, bb - 2), np.uint8)
        for l in range(8):
            if type_id == Q4_0:
                qs[:, :, :, l] = lanes[:, :, l, 0::2]
                qs[:, :, :, 8 + l] = lanes[:, :, l, 1::2]
            else:
                for k in range(4):
                    qs[:, :, :, 8 * k + l] = lanes[:, :, l, k::4]
        blk = np.concatenate([scales, qs.reshape(rows, bp, bb - 2)], axis=2)
        return blk[:, :nb].reshape(rows, nb * bb)
    if type_id == Q4_K:
        nb = cols // 256
        sbytes = _align(rows * nb * 16)
        hdr = packed[:rows * nb * 16].reshape(rows, nb, 16)
        lanes = packed[sbytes:sbytes + rows * nb * 128].reshape(rows, nb, 8, 4, 4)  # [l][g][k]
        qs = np.transpose(lanes, (0, 1, 3, 4, 2)).reshape(rows, nb, 128)
        return np.concatenate([hdr, qs], axis=2).reshape(rows, nb * 144)
    raise ValueError(type_id)
