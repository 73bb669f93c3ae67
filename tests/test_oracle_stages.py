"""The oracle's stage probes, snapshot resume, residual replay and layer prefix against
golden vectors captured from the reference's own CLI compiled in this container
(tests/golden/make_golden.py), plus the f32 -> fp16 conversion against numpy's IEEE
binary16 cast.  Every float output is compared bit for bit (FNV-1a-64 of the f32
bytes); the probe sums to the 9 significant digits the reference prints."""
import json
import os

import numpy as np
import pytest

import qxo
import qxg

GOLDEN = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "golden.json")))
GOLDEN_DIR = os.path.join(os.path.dirname(__file__), "golden")
PHASES = ["input", "v-cur", "kqv-out", "ffn-inp", "ffn-moe-out", "output"]
ATTN_SIDECARS = ["attn_norm", "Vcur", "kqv_out", "attn_out", "ffn_inp"]


def stage_input(k, layer, scale):
    """make_golden.stage_input: the seeded input of a stage-probe or replay case"""
    seed = 1000 * (ord(k) - ord("A")) + layer
    return (np.random.default_rng(seed).standard_normal(2048) * scale).astype(np.float32)


@pytest.fixture(scope="module")
def paths(tmp_path_factory):
    d = tmp_path_factory.mktemp("stages")
    out = {}
    for k, spec in GOLDEN["models"].items():
        out[k] = d / f"{k}.qxf"
        qxg.generate_model(out[k], **spec)
    return out


def fnv(v):
    return str(qxo.fnv1a64(np.ascontiguousarray(v, np.float32)))


def test_fp16_conversion_matches_ieee():
    """qxo_f32_to_fp16 (the reference's conversion restated) equals numpy's
    round-to-nearest-even binary16 cast: normals, subnormals, ties, overflow."""
    rng = np.random.default_rng(5)
    vals = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * np.float32(3.0),
        (rng.standard_normal(20000) * 1e-5).astype(np.float32),          # binary16 subnormals
        (rng.standard_normal(2000) * 7e4).astype(np.float32),            # overflow to infinity
        np.float32(1.0) + np.arange(-64, 64, dtype=np.float32) * np.float32(2.0 ** -11),   # exact ties
        np.array([0.0, -0.0, 65504.0, 65519.0, 65520.0, 2 ** -24, 2 ** -25, 3 * 2 ** -26, np.inf, -np.inf],
                 np.float32)])
    want = vals.astype(np.float16).view(np.uint16)
    got = np.array([qxo.f32_to_fp16(v) for v in vals], np.uint16)
    assert np.array_equal(got, want)
    assert qxo.f32_to_fp16(np.float32(np.nan)) == 0x7E00


@pytest.mark.parametrize("key", sorted(GOLDEN["attention_stage"]))
def test_attention_stage_matches_reference(paths, key):
    k, layer, act, kv = key.split("/")
    layer = int(layer)
    g = GOLDEN["attention_stage"][key]
    m = qxo.Model(paths[k], activation=act)
    r = m.attention_stage(layer, stage_input(k, layer, 1.0), f16_kv=(kv == "f16"))
    m.close()
    assert r is not None
    for name, v in zip(ATTN_SIDECARS, r[:5]):
        assert fnv(v) == g["sidecars"][name], (key, name)
    assert float(f"{r[5][0]:.9g}") == g["v_probe"] and float(f"{r[5][1]:.9g}") == g["output_probe"]


@pytest.mark.parametrize("key", sorted(GOLDEN["moe_stage"]))
def test_moe_stage_matches_reference(paths, key):
    k, layer, act = key.split("/")
    layer = int(layer)
    g = GOLDEN["moe_stage"][key]
    m = qxo.Model(paths[k], activation=act)
    r = m.moe_stage(layer, stage_input(k, layer, 1.0), GOLDEN["models"][k]["experts"])
    m.close()
    assert r is not None
    vec, ids = r
    for name, v in vec.items():
        assert fnv(v) == g["sidecars"][name], (key, name)
    assert [int(i) for i in ids] == g["selected_experts"]
    assert [float(f"{w:.9g}") for w in vec["ffn_moe_weights_norm"]] == g["routing_weights"]


def replay_steps(m, kv, tokens, pos0, layers, start=0, x0=None):
    """the state loop's per-step, per-layer stages (dumps by phase), from position pos0"""
    out = []
    for s, tok in enumerate(tokens):
        x = m.embed(tok) if x0 is None else x0.copy()
        step = {}
        for layer in range(start, layers):
            got = {"input": x.copy()}
            a, kqv, vcur = qxo.attention_layer(m, layer, pos0 + s, kv, x)
            got["v-cur"], got["kqv-out"] = vcur, kqv
            x = x + a
            got["ffn-inp"] = x.copy()
            y, moe, ids, w = m.moe_layer(layer, x)
            got["ffn-moe-out"], got["output"] = moe, y
            got["ids"] = [int(i) for i in ids]
            x = y
            step[layer] = got
        out.append(step)
    return out


@pytest.mark.parametrize("k", ["A", "B", "C"])
def test_resume_from_reference_snapshot(paths, k):
    """--kv-snapshot-in: the reference's own QXKVSNP1 file restores the cache (positions
    [0, position_base)), and the continuation's every dump matches the reference's."""
    g = GOLDEN["state_loop_resume"][k]
    layers = GOLDEN["models"][k]["layers"]
    kk, vv, ks, vs, pos, nt = qxg.kvsnap_read(os.path.join(GOLDEN_DIR, f"kvsnap_{k}.bin"), layers, 8, 1)
    assert (pos, nt) == (g["position_base"], g["prompt_token"])
    kv = qxo.KV(layers, 8)
    kv.k[:], kv.v[:], kv.ks[:], kv.vs[:] = kk, vv, ks, vs
    m = qxo.Model(paths[k])
    steps = replay_steps(m, kv, g["input_tokens"], pos, layers)
    m.close()
    for s, step in enumerate(steps):
        for layer, got in step.items():
            for ph in PHASES:
                assert fnv(got[ph]) == g["dumps"][f"{s}/{layer}/{ph}"], (k, s, layer, ph)
            assert got["ids"] == g["selected_experts"][s][layer]
            assert str(qxo.fnv1a64(kv.k[layer, pos + s])) == g["k_checksums"][s][layer]


@pytest.mark.parametrize("k", ["B", "C"])
def test_residual_replay_matches_reference(paths, k):
    """--start-layer S --residual-in: one token from an injected residual through layers
    S.. of a fresh cache (src/qx_format.c:6021-6025, 6260-6268)."""
    g = GOLDEN["state_loop_replay"][k]
    layers = GOLDEN["models"][k]["layers"]
    x0 = stage_input(k, 100 + g["start_layer"], g["input_scale"])
    assert str(qxo.fnv1a64(x0)) == g["residual_checksum"]
    m = qxo.Model(paths[k])
    kv = qxo.KV(layers, 8)
    (step,) = replay_steps(m, kv, [17], 0, layers, start=g["start_layer"], x0=x0)
    m.close()
    assert sorted(step) == g["layers"]
    for layer, got in step.items():
        for ph in PHASES:
            assert fnv(got[ph]) == g["dumps"][f"{layer}/{ph}"], (k, layer, ph)
    assert [step[layer]["ids"] for layer in g["layers"]] == g["selected_experts"]


def test_layer_prefix_matches_reference(paths):
    """--layers 1 on a 2-layer file: only layer 0 runs, with the full model's tensors
    (step 0; later inputs come from the token scan)."""
    g = GOLDEN["state_loop_prefix"]["B"]
    assert g["layers"] == 1
    m = qxo.Model(paths["B"])
    (step,) = replay_steps(m, qxo.KV(1, 8), [17], 0, 1)
    m.close()
    for ph in PHASES:
        assert fnv(step[0][ph]) == g["dumps"][f"0/0/{ph}"], ph
