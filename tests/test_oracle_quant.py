"""The oracle's block decoders and row dots, pinned against the reference's own
fixture (quant_reference.bin), closed forms, and the reference's dequantise-
then-gemv_scalar identity (tests/unit/tests.cpp:1546-1661)."""
import struct
from pathlib import Path

import numpy as np
import pytest

import fmoracle as fo

GOLDEN = Path(__file__).resolve().parent / "golden"


def read_quant_reference():
    b = (GOLDEN / "quant_reference.bin").read_bytes()
    assert b[:5] == b"FMQR1"
    (count,) = struct.unpack_from("<I", b, 8)
    pos, recs = 12, []
    while pos < len(b):
        t, bb, nf = struct.unpack_from("<III", b, pos)
        pos += 12
        raw = np.frombuffer(b, np.uint8, bb, pos).copy()
        pos += bb
        exp = np.frombuffer(b, np.float32, nf, pos).copy()
        pos += 4 * nf
        recs.append((t, raw, exp))
    assert len(recs) == count == 36
    return recs


def test_fp16_all_encodings_match_ieee():
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    want = h.view(np.float16).astype(np.float32)
    got = np.array([fo.fp16_to_f32(int(v)) for v in h], np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))
    # NaN payloads are carried (quant.cpp:41-42): bits = sign | 0x7F800000 | m << 13.
    # Returning a float through ctypes quiets signalling NaNs, so the quiet bit
    # is ignored.
    hb = h[nan].astype(np.uint32)
    exp_bits = ((hb & 0x8000) << 16) | 0x7F800000 | ((hb & 0x3FF) << 13)
    quiet = np.uint32(0x00400000)
    assert np.array_equal(got[nan].view(np.uint32) | quiet, exp_bits | quiet)


@pytest.mark.parametrize("type_id", [0, 2, 8, 12, 14])
def test_dequant_matches_reference_fixture(type_id):
    recs = [r for r in read_quant_reference() if r[0] == type_id]
    assert recs, f"fixture has a record for type {type_id}"
    for t, raw, exp in recs:
        got = fo.dequantize(t, raw, exp.size)
        # 1e-6 relative is the reference test's bar; these types decode exactly
        assert np.array_equal(got.view(np.uint32), exp.view(np.uint32))


def test_q4_0_closed_form_every_nibble():
    # each byte value in every position, scale 2^-4: value = (q - 8)/16 exactly
    blk = np.zeros((16, 18), np.uint8)
    blk[:, 0:2] = np.frombuffer(np.float16(0.0625).tobytes(), np.uint8)
    for i in range(16):
        blk[i, 2:] = (np.arange(16) + 16 * i) % 256
    got = fo.dequantize(2, blk, 16 * 32).reshape(16, 32)
    for i in range(16):
        byte = (np.arange(16) + 16 * i) % 256
        assert np.array_equal(got[i, :16], ((byte & 15).astype(np.float32) - 8) * np.float32(0.0625))
        assert np.array_equal(got[i, 16:], ((byte >> 4).astype(np.float32) - 8) * np.float32(0.0625))


def test_q8_0_closed_form_every_int8():
    blk = np.zeros((8, 34), np.uint8)
    d = np.float16(-3.5)
    blk[:, 0:2] = np.frombuffer(d.tobytes(), np.uint8)
    q = np.arange(256, dtype=np.uint8).reshape(8, 32)
    blk[:, 2:] = q
    got = fo.dequantize(8, blk, 256)
    assert np.array_equal(got, q.reshape(-1).view(np.int8).astype(np.float32) * np.float32(d))


def _k4_pairs(sc):
    out = []
    for j in range(8):
        if j < 4:
            out.append((sc[j] & 63, sc[j + 4] & 63))
        else:
            out.append(((sc[j + 4] & 0xF) | ((sc[j - 4] >> 6) << 4), (sc[j + 4] >> 4) | ((sc[j] >> 6) << 4)))
    return out


def test_q4_k_closed_form_every_scale_code():
    # Every 6-bit (sc, m) code at every sub-block position, against
    # value = (d*sc)*q - dmin*m computed in float64 then rounded once.
    rng = np.random.default_rng(5)
    for trial in range(64):
        blk = np.frombuffer(rng.bytes(144), np.uint8).copy()
        blk[0:2] = np.frombuffer(np.float16(rng.uniform(1e-3, 0.1)).tobytes(), np.uint8)
        blk[2:4] = np.frombuffer(np.float16(rng.uniform(1e-3, 0.1)).tobytes(), np.uint8)
        # force codes trial and 63 - trial into the eight pairs
        codes = [(trial + 7 * j) % 64 for j in range(8)]
        ms = [(63 - trial + 5 * j) % 64 for j in range(8)]
        sc = np.zeros(12, np.uint8)
        for j in range(4):
            sc[j] = (codes[j] & 63) | ((codes[j + 4] >> 4) << 6)
            sc[j + 4] = (ms[j] & 63) | ((ms[j + 4] >> 4) << 6)
            sc[j + 8] = (codes[j + 4] & 15) | ((ms[j + 4] & 15) << 4)
        blk[4:16] = sc
        assert _k4_pairs(sc) == list(zip(codes, ms))
        d = np.float64(np.frombuffer(blk[0:2].tobytes(), np.float16)[0])
        dmin = np.float64(np.frombuffer(blk[2:4].tobytes(), np.float16)[0])
        got = fo.dequantize(12, blk, 256)
        want = np.empty(256, np.float32)
        qs = blk[16:]
        for g in range(4):
            for half in range(2):
                s, m = codes[2 * g + half], ms[2 * g + half]
                q = (qs[32 * g:32 * g + 32] >> (4 * half)) & 15
                want[64 * g + 32 * half:64 * g + 32 * half + 32] = (
                    (d * s) * q.astype(np.float64) - dmin * m).astype(np.float32)
        assert np.array_equal(got, want)


def _reference_style_weights(type_id, out_dim=9):
    # tests.cpp:1549-1601: LCG bytes, every block's scale field set to 2^-4
    bs, bb = fo.GEOMETRY[type_id]
    in_dim = bs * 2 if type_id else 2
    w = np.empty(out_dim * (in_dim // bs) * bb, np.uint8)
    state = (0xBEEF0000 + type_id) & 0xFFFFFFFF
    for i in range(w.size):
        state = (state * 1664525 + 1013904223) & 0xFFFFFFFF
        w[i] = (state >> 16) & 0xFF
    blocks = w.reshape(-1, bb)
    if type_id == 0:
        blocks[:] = np.frombuffer(np.float32(0.0625).tobytes(), np.uint8)
    else:
        blocks[:, 0:2] = np.frombuffer(np.float16(0.0625).tobytes(), np.uint8)
        if type_id == 12:
            blocks[:, 2:4] = np.frombuffer(np.float16(0.0625).tobytes(), np.uint8)
    x = (((np.arange(in_dim) % 7) - 3) * 0.25).astype(np.float32)
    return w, x, out_dim, in_dim


@pytest.mark.parametrize("type_id", [0, 2, 8, 12])
@pytest.mark.parametrize("isa", [fo.ISA_SCALAR, fo.ISA_AVX2])
def test_gemv_equals_dequantise_then_scalar_gemv(type_id, isa):
    w, x, out_dim, in_dim = _reference_style_weights(type_id)
    dense = fo.dequantize(type_id, w, out_dim * in_dim).reshape(out_dim, in_dim)
    ref = fo.gemv(0, dense.view(np.uint8), x, out_dim, in_dim, fo.ISA_SCALAR)
    got = fo.gemv(type_id, w, x, out_dim, in_dim, isa)
    worst = np.abs(got.astype(np.float64) - ref).max() / max(np.abs(ref).max(), 1e-30)
    assert worst < 1e-5


def test_gemv_rejects_bad_shapes_and_types():
    w = np.zeros(18, np.uint8)
    x = np.zeros(33, np.float32)
    with pytest.raises(fo.OracleError) as e:
        fo.gemv(2, w, x, 1, 33)
    assert e.value.status == 3  # SHAPE_MISMATCH
    with pytest.raises(fo.OracleError) as e:
        fo.gemv(3, w, x, 1, 32)
    assert e.value.status == 2  # UNSUPPORTED_QUANTISATION
