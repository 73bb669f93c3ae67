"""q8_k_compat activation mode on the HIP path (reference --activation q8_k_compat:
Q8_K activations and integer dots for the projections, experts and Q6_K head).

Bars: the device Q8_K quantizer is byte-identical to the reference probe's blocks and
to the oracle.  Matvec outputs whose input reaches the quantizer bit-identical (Q/K/V
and gate/up on the normed residual, the head) are within 1e-5 relative L2.  Outputs
that re-quantize a device-computed intermediate (O projection of the attention
context, down projection of h) may see a code one step apart where the two inputs
straddle a rounding boundary: about 1e-5 of the values, each worth ~5e-4 of the
output's norm, so those are held to REQ_TOL = 2e-3 (a wrong block scale, sign or
rounding rule costs 1e-2 or more).  Those two projections are also replayed on the same
input - the oracle's Q8_K O projection of the device's own context, its down projection of
the device's own h per rank - and held to 1e-5."""
import ctypes
import json
import os

import numpy as np
import pytest

import qxo
import qxg
from helpers import REL_L2, rel_l2, seeded_kv, seeded_normal, topk_consistent

pytestmark = pytest.mark.gpu
GOLDEN = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "golden.json")))
REQ_TOL = 2e-3


@pytest.fixture(scope="module")
def ctx():
    c = qxg.Context(0)
    yield c
    c.close()


def _probe_input(inject, values):
    i = np.arange(values)
    if inject == "positive":
        return (i % 127).astype(np.float32) / np.float32(127.0)
    if inject == "negative":
        return -((i % 127).astype(np.float32) / np.float32(127.0))
    if inject == "edge":
        return np.where(i % 2 == 1, 1.0, -1.0).astype(np.float32)
    if inject == "zero":
        return np.zeros(values, np.float32)
    return ((i % 251).astype(np.int32) - 125).astype(np.float32) / np.float32(127.0)


def test_q8k_quantizer_matches_reference_probe(ctx):
    """The reference's q8-k-activation-probe inputs: block bytes' FNV identical."""
    for key, want in GOLDEN["q8k_activation"].items():
        inject, values = key.split("/")
        b = ctx.q8k_quantize(_probe_input(inject, int(values)))
        assert str(qxo.fnv1a64(b)) == want["checksum"], key


def test_q8k_quantizer_bit_exact_vs_oracle(ctx):
    rng = np.random.default_rng(8)
    cases = [rng.standard_normal(4096).astype(np.float32),
             (rng.standard_normal(2048) * 1e-30).astype(np.float32),        # tiny scales
             np.repeat(rng.standard_normal(16), 16).astype(np.float32),     # ties of the largest magnitude
             np.concatenate([np.full(256, -3.0), np.full(256, 3.0)]).astype(np.float32),
             ((rng.integers(-254, 255, 768) + 0.5) / 127.0 * 2).astype(np.float32)]   # half-way codes
    t = np.zeros(256, np.float32); t[7] = -2.0; t[9] = 2.0                  # first of equal magnitudes wins
    cases.append(t)
    for x in cases:
        assert ctx.q8k_quantize(x).tobytes() == qxo.quantize_q8k(x).tobytes()


def test_q8k_quantizer_rejects_like_reference(ctx):
    for bad in (np.nan, np.inf):
        x = _probe_input("none", 512)
        x[300] = bad
        with pytest.raises(qxg.QxgError, match="NaN or Inf"):
            ctx.q8k_quantize(x)
    with pytest.raises(qxg.QxgError, match="multiple of 256"):
        ctx.q8k_quantize(np.zeros(300, np.float32))
    with pytest.raises(qxg.QxgError, match="too small"):
        ctx.q8k_quantize(np.zeros(4352, np.float32))


@pytest.fixture(scope="module")
def models(tmp_path_factory):
    d = tmp_path_factory.mktemp("q8")
    base, mix, head = d / "base.qxf", d / "mix.qxf", d / "head.qxf"
    qxg.generate_model(base, layers=1, vocab=1024, experts=128, seed=22)
    qxg.generate_model(mix, layers=4, vocab=4096, experts=32, seed=66, mix=1)
    qxg.generate_model(head, layers=0, vocab=151936, embedding=False, head=True, seed=11)
    return {"base": base, "mix": mix, "head": head}


@pytest.mark.parametrize("which,layer", [("base", 0), ("mix", 0), ("mix", 1), ("mix", 2), ("mix", 3)])
def test_q8k_attention_layer(ctx, models, which, layer):
    ctx.load(models[which])
    ctx.set_activation("q8_k_compat")
    try:
        layers = 1 if which == "base" else 4
        pos = 45
        ctx.kv_create(layers, 128)
        okv = qxo.KV(layers, 128)
        k, v, ks, vs = seeded_kv(70 + layer, pos)
        ctx.kv_write(layer, 0, k, v, ks, vs)
        okv.k[layer, :pos], okv.v[layer, :pos], okv.ks[layer, :pos], okv.vs[layer, :pos] = k, v, ks, vs
        x = seeded_normal(80 + layer)
        a, kqv, vcur = ctx.attention_layer(layer, pos, x)
        om = qxo.Model(models[which], activation="q8_k_compat")
        oa, okqv, ovcur = qxo.attention_layer(om, layer, pos, okv, x)
        om.close()
        om_o = qxo.Model(models[which], activation="q8_k_compat")
        assert rel_l2(vcur, ovcur) <= REL_L2, rel_l2(vcur, ovcur)
        assert rel_l2(kqv, okqv) <= REL_L2, rel_l2(kqv, okqv)
        assert rel_l2(a, oa) <= REQ_TOL, rel_l2(a, oa)
        # same input: the oracle's Q8_K O projection of the device's own context
        t, _, wo = om_o.tensor(f"blk.{layer}.attn_output.weight")
        so = qxo.matvec_q8k(t, wo, 2048, 4096, kqv)
        assert so is not None and rel_l2(a, so) <= REL_L2, rel_l2(a, so)
        # f32 and q8_k_compat really differ (the mode switch is live)
        ctx.set_activation("f32")
        ctx.kv_create(layers, 128)
        ctx.kv_write(layer, 0, k, v, ks, vs)
        a32, _, _ = ctx.attention_layer(layer, pos, x)
        assert rel_l2(a32, oa) > 10 * rel_l2(a, oa)
        om_o.close()
    finally:
        ctx.set_activation("f32")


@pytest.mark.parametrize("which,layer", [("base", 0), ("mix", 0), ("mix", 1), ("mix", 2), ("mix", 3)])
def test_q8k_moe_layer(ctx, models, which, layer):
    ctx.load(models[which])
    ctx.set_activation("q8_k_compat")
    try:
        om = qxo.Model(models[which], activation="q8_k_compat")
        for seed in (90, 91):
            x = seeded_normal(seed + 10 * layer)
            y, moe, ids, w = ctx.moe_layer(layer, x)
            oy, omoe, oids, ow = om.moe_layer(layer, x)
            assert list(ids) == list(oids)
            assert np.allclose(w, ow, rtol=1e-9, atol=0)
            assert rel_l2(moe, omoe) <= REQ_TOL, rel_l2(moe, omoe)
            assert rel_l2(y, oy) <= REQ_TOL
            # same input: the oracle's Q8_K down projection of the device's own h, per rank
            st, sids = ctx.moe_stage(layer, x)
            t, _, wd = om.tensor(f"blk.{layer}.ffn_down_exps.weight")
            per_expert = len(wd) // ctx.info.experts
            for r in range(8):
                e = int(sids[r])
                h = st["ffn_moe_swiglu"][768 * r:768 * (r + 1)]
                sd = qxo.matvec_q8k(t, wd[e * per_expert:(e + 1) * per_expert], 2048, 768, h, expert=True)
                gd = st["ffn_moe_down"][2048 * r:2048 * (r + 1)]
                assert sd is not None and rel_l2(gd, sd) <= REL_L2, (r, rel_l2(gd, sd))
        om.close()
    finally:
        ctx.set_activation("f32")


def test_q8k_final_head_config1(ctx, models):
    ctx.load(models["head"], verify=False)
    ctx.set_activation("q8_k_compat")
    try:
        om = qxo.Model(models["head"], activation="q8_k_compat")
        for seed in (1, 2):
            x = seeded_normal(seed)
            _, lg, ids, tl = ctx.final_head(x, 8)
            _, olg, oids, otl = om.final_head(x, 151936, 8)
            assert rel_l2(lg, olg) <= REL_L2, rel_l2(lg, olg)
            ok, why = topk_consistent(ids, oids, olg)
            assert ok, why
        om.close()
    finally:
        ctx.set_activation("f32")


def test_q8k_decode_greedy_and_replay(ctx, models):
    """Embedding + 4 mixed layers + head, 4 steps fed the oracle's tokens; the
    replayed device loop then matches the eager q8 steps token for token."""
    ctx.load(models["mix"])
    ctx.set_activation("q8_k_compat")
    try:
        ctx.kv_create(4, 16)
        om = qxo.Model(models["mix"], activation="q8_k_compat")
        okv = qxo.KV(4, 16)
        tok = 29
        for s in range(4):
            res, lay, lg, ids, tl = ctx.decode_token(tok, s, True, 4, want_layers=True, want_logits=True)
            ores, olay, olg, oids, otl = qxo.decode_token(om, tok, s, okv, 4, True, 4096, 4)
            assert rel_l2(lay, olay) <= REQ_TOL, (s, rel_l2(lay, olay))
            assert rel_l2(lg, olg) <= REQ_TOL
            ok, why = topk_consistent(ids[:1], oids[:1], olg, margin=0.05)
            assert ok, why
            tok = int(oids[0])
        om.close()
        ctx.kv_create(4, 16)
        eager, t = [], 29
        for s in range(5):
            _, _, _, ids, _ = ctx.decode_token(t, s, True, 1)
            t = int(ids[0])
            eager.append(t)
        for rep in range(2):
            ctx.kv_create(4, 16)
            gen, _ = ctx.generate([29], 5)
            assert list(gen) == eager, rep
    finally:
        ctx.set_activation("f32")


def test_q8k_failures_report_and_clear(ctx, models):
    """A non-finite activation fails the call with the reference's message (f32 mode
    zeroes it instead); the next call succeeds; prefill runs as decode steps."""
    ctx.load(models["base"])
    ctx.set_activation("q8_k_compat")
    try:
        x = seeded_normal(5)
        x[100] = np.nan
        with pytest.raises(qxg.QxgError, match="Q8_K activation contains NaN or Inf"):
            ctx.moe_layer(0, x)
        y, _, _, _ = ctx.moe_layer(0, seeded_normal(5))
        assert np.isfinite(y).all()
        # prefill in this mode runs the one-kernel-per-phase decode kernels token by token:
        # equal to the decode steps of that path
        ctx.set_layer_path(0)
        ctx.kv_create(1, 8)
        res, _, ids, _, _ = ctx.prefill(np.array([1, 2, 3], np.uint32), 0, True, 2, want_residual=True)
        ctx.kv_create(1, 8)
        for s, tok in enumerate((1, 2, 3)):
            r, _, _, i2, _ = ctx.decode_token(tok, s, s == 2, 2)
            assert np.array_equal(res[s], r)
        assert list(ids) == list(i2)
        err = ctypes.create_string_buffer(256)
        assert not qxg._g.qxg_set_activation(ctx._c, 7, err, 256)   # the C entry point rejects unknown formats
        assert b"unsupported activation" in err.value
    finally:
        ctx.set_layer_path(1)
        ctx.set_activation("f32")


def test_q8k_cli_probe_matches_reference(tmp_path):
    """qxqxf q8-k-activation-probe prints the reference CLI's JSON for the same inputs."""
    import subprocess
    exe = os.path.join(os.path.dirname(qxg.__file__), "bin", "qxqxf")
    for key in ("none/256", "edge/512", "negative/4096"):   # one child process each, run one after another
        want = GOLDEN["q8k_activation"][key]
        inject, values = key.split("/")
        r = subprocess.run([exe, "q8-k-activation-probe", "--values", values, "--inject", inject],
                           capture_output=True, text=True, timeout=60)
        assert r.returncode == 0, r.stderr
        j = json.loads(r.stdout)
        assert str(j["checksum"]) == want["checksum"] and j["quant_sum"] == want["quant_sum"], key
        assert j["first_scale"] == want["first_scale"] and j["block_bytes"] == 292
        # the reference's keys, in its order (src/qx_format.c:4331-4343)
        assert list(j) == ["probe", "activation_format", "values", "blocks", "block_bytes", "workspace_bytes",
                           "first_scale", "quant_sum", "finite", "block_hex", "checksum"], list(j)
    r = subprocess.run([exe, "q8-k-activation-probe", "--values", "256", "--inject", "nan"], capture_output=True,
                       text=True, timeout=60)
    assert r.returncode == 1 and "NaN or Inf" in r.stderr
