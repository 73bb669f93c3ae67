"""What the decode's activation digits cost, on the CPU: an emulation of the scheme the HIP
decode kernels use for every matvec input (qxg_dev.h digits8: per 32-value group, the
values as integers X = rint(y * 2^k) with k = 22 - e, 2^(e-1) <= max |y| < 2^e, so each
value carries 2^-23 of its group's maximum as rounding error; weight codes and digit
planes then multiply exactly).

The MoE half of a layer (reference src/qx_format.c:5198-5317) is recomputed from the
oracle's own dequantized expert rows and its own routing, once exactly (which must equal
the oracle bit for bit, pinning the emulation) and once with the x' and h digits
truncated as the device truncates them.  On the planted single x1000 channels the
truncation stays far inside the 1e-5 bar; on the compound stress pattern (groups of x'
spanning ~2.6e3, of h ~6e4, expert outputs cancelling in channel 13) it alone exceeds it,
which is why the persistent-path stress test holds that half to 5e-5."""
import numpy as np
import pytest

import qxg
import qxo
from helpers import rel_l2

LAYERS, VOCAB, EXPERTS = 4, 8192, 128
PROMPT = [5, 900, 17]


def digits(y, group=32):
    """The device's truncation of a vector to 22-bit digits per 32-value group (each result
    is an integer of at most 22 bits times a power of two, so exact in f32)."""
    y = np.asarray(y, np.float32).reshape(-1, group).astype(np.float64)
    out = np.zeros_like(y)
    for i, row in enumerate(y):
        mx = np.abs(row).max()
        if mx == 0:
            continue
        _, e = np.frexp(np.float32(mx))
        k = min(22 - int(e), 126)
        out[i] = np.rint(row * 2.0 ** k) * 2.0 ** -k
    return out.reshape(-1).astype(np.float32)


def _perm(hi, lo, sel):
    """v_perm_b32 for selector bytes 0..7 (bytes of lo, then hi) and 0x0c (zero)."""
    src = [(lo >> (8 * i)) & 255 for i in range(4)] + [(hi >> (8 * i)) & 255 for i in range(4)]
    out = np.zeros_like(lo)
    for i in range(4):
        s = (sel >> (8 * i)) & 255
        out |= (np.zeros_like(lo) if s == 0x0C else src[s]) << (8 * i)
    return out


def test_digit_planes_from_one_subtraction():
    """digits8's split of X (|X| <= 2^22) into signed bytes L, M, H with X = 65536 H + 256 M
    + L: taken from the bytes of X + 0x808080 (each digit + 128) and packed four values a word
    by its byte transpose, the planes equal the sequential peel (L = sext(X mod 256), then M
    from (X - L) / 256, then H), for every X in range."""
    X = np.arange(-(1 << 22), (1 << 22) + 1, dtype=np.int64)
    sext = lambda v: ((v & 255) ^ 128) - 128
    L = sext(X)
    X1 = (X - L) >> 8
    M = sext(X1)
    H = (X1 - M) >> 8
    assert np.array_equal(65536 * H + 256 * M + L, X)
    assert H.min() >= -128 and H.max() <= 127
    xb = X + 0x808080
    assert xb.min() >= 0 and xb.max() < (1 << 24)
    for d, sh in ((L, 0), (M, 8), (H, 16)):
        assert np.array_equal(((xb >> sh) & 255) - 128, d)
    # the byte transpose of four consecutive values (the device's perm selectors)
    rng = np.random.default_rng(5)
    v = [(rng.integers(-(1 << 22), (1 << 22) + 1, 4096) + 0x808080).astype(np.uint64) for _ in range(4)]
    t0, t1 = _perm(v[1], v[0], 0x05010400), _perm(v[3], v[2], 0x05010400)
    u0, u1 = _perm(v[1], v[0], 0x0C0C0602), _perm(v[3], v[2], 0x0C0C0602)
    planes = (_perm(t1, t0, 0x05040100) ^ 0x80808080, _perm(t1, t0, 0x07060302) ^ 0x80808080,
              _perm(u1, u0, 0x05040100) ^ 0x80808080)
    for byte, plane in enumerate(planes):
        want = sum(((((v[j] >> (8 * byte)) & 255) - 128) & 255) << (8 * j) for j in range(4))
        assert np.array_equal(plane, want)


def expert_matvec(om, name, e, rows, in_dims, block_bytes, x):
    """(float) of the double dot of expert e's rows with f32 x: the oracle's matvec, the
    reference's arithmetic (src/qx_format.c:4739-4787)."""
    t, _, raw = om.tensor(name)
    n = rows * (in_dims // 256) * block_bytes
    return qxo.matvec(t, raw[int(e) * n:(int(e) + 1) * n], rows, in_dims, x)


def moe_emulated(om, layer, ffn_inp, trunc_x, trunc_h):
    """(emulated MoE output, oracle MoE output) on ffn_inp: the oracle's normalised input,
    routing and weights, its f32 casts of gate, up, h and each expert's down output, and its
    rank-ordered f32 weighted sum (src/qx_format.c:5296-5309)."""
    _, moe, ids, w = om.moe_layer(layer, ffn_inp)
    st, _ = om.moe_stage(layer, ffn_inp, EXPERTS)
    x = digits(st["ffn_norm"]) if trunc_x else st["ffn_norm"]
    hs = []
    for r in range(8):
        g = expert_matvec(om, f"blk.{layer}.ffn_gate_exps.weight", ids[r], 768, 2048, 74, x).astype(np.float64)
        u = expert_matvec(om, f"blk.{layer}.ffn_up_exps.weight", ids[r], 768, 2048, 74, x).astype(np.float64)
        with np.errstate(over="ignore"):
            hs.append((g / (1.0 + np.exp(-g)) * u).astype(np.float32))
    h = np.concatenate(hs)
    h = digits(h) if trunc_h else h
    out = np.zeros(2048, np.float32)
    for r in range(8):
        y = expert_matvec(om, f"blk.{layer}.ffn_down_exps.weight", ids[r], 2048, 768, 98, h[768 * r:768 * (r + 1)])
        out = (out + (w[r] * y.astype(np.float64)).astype(np.float32)).astype(np.float32)
    return out, moe


def chain_inputs(om, upto_pos):
    """The oracle's own ffn inputs of every layer at positions 0..upto_pos of PROMPT."""
    kv = qxo.KV(LAYERS, 8)
    res = {}
    for pos in range(upto_pos + 1):
        x = om.embed(PROMPT[pos])
        for l in range(LAYERS):
            a, _, _ = qxo.attention_layer(om, l, pos, kv, x)
            fi = (x + a).astype(np.float32)
            res[(pos, l)] = fi
            x, _, _, _ = om.moe_layer(l, fi)
    return res


@pytest.fixture(scope="module", params=[1, 2], ids=["single", "stress"])
def model(request, tmp_path_factory):
    p = tmp_path_factory.mktemp("digits") / f"outliers{request.param}.qxf"
    qxg.generate_model(p, layers=LAYERS, vocab=VOCAB, experts=EXPERTS, seed=71, outliers=request.param)
    om = qxo.Model(p)
    yield om, request.param
    om.close()


def test_digit_truncation_of_the_moe_half(model):
    om, pattern = model
    if pattern == 1:
        cells = chain_inputs(om, 1)                      # positions 0 and 1, every layer
    else:
        cells = {(2, 3): chain_inputs(om, 2)[(2, 3)]}   # the stress cell the GPU test met
    for (pos, l), fi in cells.items():
        exact, moe = moe_emulated(om, l, fi, False, False)
        assert np.array_equal(exact, moe), (pos, l)      # the emulation is the oracle's arithmetic
        ex = rel_l2(moe_emulated(om, l, fi, True, False)[0], moe)
        eh = rel_l2(moe_emulated(om, l, fi, False, True)[0], moe)
        if pattern == 1:
            assert ex <= 2e-6 and eh <= 2e-6, (pos, l, ex, eh)
        else:
            assert ex > 1e-5 and eh > 1e-5, (pos, l, ex, eh)
            assert ex < 5e-5 and eh < 5e-5, (pos, l, ex, eh)
