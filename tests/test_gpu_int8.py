"""The device INT8 KV quantizer bit for bit against the oracle's (reference
qx_quantize_int8_vector, src/qx_format.c:4449-4463; the oracle's is pinned to the reference
by the state-loop goldens' KV checksums).  qxg_int8_quantize runs the same device functions
(int8_mag, int8_scale, int8_code) that every kernel appending a KV row uses.  Integer output:
codes and scale must be identical, including values exactly half-way between two codes,
the +-127 clamp, non-finite values and all-zero rows."""
import numpy as np
import pytest

import qxg
import qxo

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    c = qxg.Context(0)
    yield c
    c.close()


def rows():
    rng = np.random.default_rng(4449)
    out = {}
    for s in (1e-30, 1e-3, 1.0, 37.5, 1e4, 3e38):
        with np.errstate(over="ignore"):   # the largest scale overflows some values to +-inf on purpose
            out[f"normal*{s:g}"] = (rng.standard_normal(512) * s).astype(np.float32)
    # max 127 -> scale exactly 1: x = k + 0.5 sits on a rounding tie (round-half-even)
    t = np.arange(-127, 127, dtype=np.float32)[:254] + np.float32(0.5)
    out["ties_scale1"] = np.concatenate([t, np.float32([127.0, -127.0, 0.5, -0.5, 1.5, -1.5, 2.5, -2.5])]).astype(np.float32)
    # a scale that is not a power of two: x = (k + 0.5) * scale, the quotient lands next to a tie
    sc = np.float32(100.0) / np.float32(127.0)
    k = np.arange(-126, 127, dtype=np.float32)
    out["near_ties"] = np.concatenate([(k + np.float32(0.5)) * sc, np.float32([100.0, -100.0])]).astype(np.float32)
    # non-finite values are excluded from the maximum and coded 0
    x = rng.standard_normal(512).astype(np.float32)
    x[[3, 77, 200]] = [np.nan, np.inf, -np.inf]
    out["nonfinite"] = x
    out["zeros"] = np.zeros(512, np.float32)
    out["subnormal"] = (rng.standard_normal(512) * 1e-42).astype(np.float32)
    # a single outlier: everything else rounds towards 0
    x = (rng.standard_normal(512) * 1e-3).astype(np.float32)
    x[10] = -5e3
    out["outlier"] = x
    out["short_row"] = rng.standard_normal(37).astype(np.float32)
    return out


@pytest.mark.parametrize("name", sorted(rows()))
def test_int8_quantizer_bit_exact(ctx, name):
    x = rows()[name]
    codes, scale = ctx.int8_quantize(x)
    ocodes, oscale = qxo.quantize_int8(x)
    assert np.float32(scale).view(np.uint32) == np.float32(oscale).view(np.uint32), (name, scale, oscale)
    assert np.array_equal(codes, ocodes), (name, np.flatnonzero(codes != ocodes)[:8])


def test_int8_ties_round_half_even(ctx):
    """With scale 1 the codes of k + 0.5 are the even neighbours (lrintf in the default mode)."""
    x = np.float32([127.0, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 126.5, -126.5])
    codes, scale = ctx.int8_quantize(x)
    assert scale == np.float32(1.0)
    assert list(codes) == [127, 0, 2, 2, 0, -2, -2, 126, -126]
