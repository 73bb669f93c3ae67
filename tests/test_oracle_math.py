"""Checks of the oracle that the golden vectors leave open, fixed by mathematics:
fp16 widening over all 65536 inputs, codebook tables, RMSNorm/RoPE/INT8 closed
forms, and a matvec against numpy on the oracle's own decoded weights."""
import os
import re

import numpy as np
import pytest

import qxo

GRIDS_H = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "qx-mini-c_amd", "csrc", "qx_grids.h")


def test_fp16_all_65536():
    h = np.arange(65536, dtype=np.uint16)
    ref = h.view(np.float16).astype(np.float32)
    exp31 = ((h >> 10) & 31) == 31
    ref[exp31] = np.where((h[exp31] & 0x8000) != 0, -65504.0, 65504.0)
    got = np.array([qxo.fp16_to_f32(int(v)) for v in h], np.float32)
    assert got.view(np.uint32).tobytes() == ref.view(np.uint32).tobytes()


def _grid_tables():
    src = open(GRIDS_H).read()
    p2 = [int(x, 16) for x in re.search(r"qx_iq2xs_packed\[512\] = \{(.*?)\};", src, re.S).group(1).replace(",", " ").split()]
    p3 = [int(x, 16) for x in re.search(r"qx_iq3xxs_packed\[256\] = \{(.*?)\};", src, re.S).group(1).replace(",", " ").split()]
    f2 = int(re.search(r"QX_IQ2XS_GRID_FNV (0x[0-9a-f]+)", src).group(1), 16)
    f3 = int(re.search(r"QX_IQ3XXS_GRID_FNV (0x[0-9a-f]+)", src).group(1), 16)
    g2 = np.array([[[8, 25, 43][(c >> (2 * j)) & 3] for j in range(8)] for c in p2], np.uint8)
    g3 = np.array([[[4, 12, 20, 28, 36, 44, 52, 62][(c >> (3 * j)) & 7] for j in range(4)] for c in p3], np.uint8)
    return g2, g3, f2, f3


def _grid_tables_s():
    src = open(GRIDS_H).read()
    p2 = [int(x, 16) for x in re.search(r"qx_iq2s_packed\[1024\] = \{(.*?)\};", src, re.S).group(1).replace(",", " ").split()]
    p3 = [int(x, 16) for x in re.search(r"qx_iq3s_packed\[512\] = \{(.*?)\};", src, re.S).group(1).replace(",", " ").split()]
    f2 = int(re.search(r"QX_IQ2S_GRID_FNV (0x[0-9a-f]+)", src).group(1), 16)
    f3 = int(re.search(r"QX_IQ3S_GRID_FNV (0x[0-9a-f]+)", src).group(1), 16)
    g2 = np.array([[[8, 25, 43][(c >> (2 * j)) & 3] for j in range(8)] for c in p2], np.uint8)
    g3 = np.array([[[1, 3, 5, 7, 9, 11, 13, 15][(c >> (3 * j)) & 7] for j in range(4)] for c in p3], np.uint8)
    return g2, g3, f2, f3


def test_iq2s_iq3s_grid_expansion_matches_recorded_fnv():
    g2, g3, f2, f3 = _grid_tables_s()
    assert qxo.fnv1a64(g2) == f2 and qxo.fnv1a64(g3) == f3
    assert len({bytes(r) for r in g2}) == 1024 and len({bytes(r) for r in g3}) == 512


def test_grid_expansion_matches_recorded_fnv():
    g2, g3, f2, f3 = _grid_tables()
    assert qxo.fnv1a64(g2) == f2 and qxo.fnv1a64(g3) == f3
    assert len({bytes(r) for r in g2}) == 512 and len({bytes(r) for r in g3}) == 256


@pytest.mark.skipif(not os.path.exists("/root/reference/src/qx_iq2xs_tables.inc"), reason="reference tables not present")
def test_grids_equal_reference_tables():
    src = open("/root/reference/src/qx_iq2xs_tables.inc").read()

    def arr(name):
        m = re.search(name + r"\[\d+\]\s*=\s*\{(.*?)\};", src, re.S)
        return [int(x, 0) for x in re.findall(r"0x[0-9a-fA-F]+|\d+", m.group(1))]
    g2, g3, _, _ = _grid_tables()
    assert [int.from_bytes(bytes(r), "little") for r in g2] == arr("qx_iq2xs_grid")
    assert [int.from_bytes(bytes(r), "little") for r in g3] == arr("qx_iq3xxs_grid")
    assert arr("qx_ksigns_iq2xs") == [i | ((bin(i).count("1") & 1) << 7) for i in range(128)]
    g2s, g3s, _, _ = _grid_tables_s()
    assert [int.from_bytes(bytes(r), "little") for r in g2s] == arr("qx_iq2s_grid")
    assert [int.from_bytes(bytes(r), "little") for r in g3s] == arr("qx_iq3s_grid")


def _iq4_block(d16, ls, nib):
    """IQ4_XS block with fp16 d, per-sub-block 6-bit ls and nibble codes nib[256]."""
    b = np.zeros(136, np.uint8)
    b[0], b[1] = d16 & 255, d16 >> 8
    sh = 0
    for ib in range(8):
        sh |= ((ls[ib] >> 4) & 3) << (2 * ib)
        b[4 + ib // 2] |= (ls[ib] & 15) << (4 * (ib % 2))
    b[2], b[3] = sh & 255, sh >> 8
    for ib in range(8):
        for j in range(16):
            b[8 + 16 * ib + j] = nib[32 * ib + j] | (nib[32 * ib + 16 + j] << 4)
    return b


def test_iq4_closed_form():
    kv = [-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113]
    rng = np.random.default_rng(3)
    ls = rng.integers(0, 64, 8)
    nib = rng.integers(0, 16, 256)
    d16 = int(np.float16(0.25).view(np.uint16))
    v = qxo.decode_block(23, _iq4_block(d16, ls, nib))
    want = np.array([np.float32(0.25) * np.float32(ls[i // 32] - 32) * np.float32(kv[nib[i]]) for i in range(256)], np.float32)
    assert np.array_equal(v, want)


def test_matvec_equals_double_dot_of_decoded_rows():
    rng = np.random.default_rng(5)
    rows, dims = 7, 512
    raw = rng.integers(0, 256, size=(rows * dims // 256, 136), dtype=np.uint8)
    raw[:, 0], raw[:, 1] = 0x00, 0x20          # d = fp16 0x2000 (2^-7)
    x = rng.standard_normal(dims).astype(np.float32)
    y = np.zeros(rows, np.float32)
    qxo._o.qxo_matvec(23, raw.ctypes.data_as(qxo.vp), rows, dims, x.ctypes.data_as(qxo.vp), y.ctypes.data_as(qxo.vp))
    w = np.concatenate([qxo.decode_block(23, b) for b in raw]).reshape(rows, dims).astype(np.float64)
    want = np.array([float(np.float32(sum(float(a) * float(b) for a, b in zip(w[r], x)))) for r in range(rows)], np.float32)
    assert np.array_equal(y, want)


def test_rmsnorm_constant_vector():
    # x = c everywhere, w = 1: y = (float)(c / sqrt(c^2 + 1e-6))
    x = np.full(2048, 3.0, np.float32)
    w = np.ones(2048, np.float32)
    y = np.zeros(2048, np.float32)
    qxo._o.qxo_rmsnorm.argtypes = [qxo.vp, qxo.vp, qxo.vp, qxo.u32, qxo.vp]
    qxo._o.qxo_rmsnorm(x.ctypes.data_as(qxo.vp), w.ctypes.data_as(qxo.vp), y.ctypes.data_as(qxo.vp), 2048, None)
    assert np.all(y == np.float32(3.0 / np.sqrt(9.0 + 1e-6)))


def test_rope_position_zero_is_identity_and_rotation_preserves_pair_norms():
    qxo._o.qxo_rope.argtypes = [qxo.vp, qxo.u32, qxo.u32, qxo.u32, qxo.ctypes.c_double]
    v = np.random.default_rng(9).standard_normal(4 * 128).astype(np.float32)
    a = v.copy()
    qxo._o.qxo_rope(a.ctypes.data_as(qxo.vp), 4, 128, 0, 1e6)
    assert np.array_equal(a, v)
    b = v.copy()
    qxo._o.qxo_rope(b.ctypes.data_as(qxo.vp), 4, 128, 777, 1e6)
    v2, b2 = v.reshape(4, 2, 64).astype(np.float64), b.reshape(4, 2, 64).astype(np.float64)
    assert np.allclose(np.hypot(v2[:, 0], v2[:, 1]), np.hypot(b2[:, 0], b2[:, 1]), rtol=1e-6)
    # pair 0 has frequency 1: angle = pos radians
    c, s = np.cos(777.0), np.sin(777.0)
    assert b[0] == np.float32(float(v[0]) * c - float(v[64]) * s)


def test_int8_quantize_properties():
    qxo._o.qxo_quantize_int8.argtypes = [qxo.vp, qxo.vp, qxo.u32]
    qxo._o.qxo_quantize_int8.restype = qxo.ctypes.c_float
    x = np.random.default_rng(1).standard_normal(512).astype(np.float32)
    x[10] = np.inf
    q = np.zeros(512, np.int8)
    s = qxo._o.qxo_quantize_int8(x.ctypes.data_as(qxo.vp), q.ctypes.data_as(qxo.vp), 512)
    fin = np.isfinite(x)
    assert s == np.float32(np.abs(x[fin]).max()) / np.float32(127.0)
    assert q[10] == 0 and np.abs(q).max() == 127
    assert np.array_equal(q[fin], np.clip(np.rint(x[fin] / np.float32(s)), -127, 127).astype(np.int8))
    z = np.zeros(512, np.float32)
    assert qxo._o.qxo_quantize_int8(z.ctypes.data_as(qxo.vp), q.ctypes.data_as(qxo.vp), 512) == 1.0


def test_int8_quantize_ties_round_half_even():
    """numpy's rint is round-half-even, like lrintf in the default mode: with max 127 the
    scale is exactly 1 and the codes of k + 0.5 are the even neighbours."""
    x = np.float32([127.0, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 126.5, -126.5])
    codes, scale = qxo.quantize_int8(x)
    assert scale == np.float32(1.0)
    assert list(codes) == [127, 0, 2, 2, 0, -2, -2, 126, -126]
