"""The oracle (oracle/qxo.c) against golden vectors captured from the reference's
own CLI compiled in this container (tests/golden/make_golden.py).  Models are
regenerated from their seeds, so the same bytes are checked on any machine."""
import json
import os

import numpy as np
import pytest

import qxo
import qxg

GOLDEN = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "golden.json")))
BB = {12: 144, 14: 210, 17: 74, 18: 98, 23: 136}
BB_ALL = {**BB, 13: 176, 21: 110, 22: 82}
PHASES = ["input", "v-cur", "kqv-out", "ffn-inp", "ffn-moe-out", "output"]


@pytest.fixture(scope="module")
def models(tmp_path_factory):
    d = tmp_path_factory.mktemp("golden")
    out = {}
    for k, spec in GOLDEN["models"].items():
        p = d / f"{k}.qxf"
        qxg.generate_model(p, **spec)
        out[k] = qxo.Model(p)
    yield out
    for m in out.values():
        m.close()


def test_decode_block_matches_reference(models):
    BB.update({13: 176, 21: 110, 22: 82})
    for key, want in GOLDEN["decode_block"].items():
        k, _, rest = key.rpartition(":")
        m = models[k or "A"]
        name, b = rest.split("#")
        t, dims, raw = m.tensor(name)
        v = qxo.decode_block(t, raw[int(b) * BB[t]:(int(b) + 1) * BB[t]])
        assert str(qxo.fnv1a64(v)) == want["f32_checksum"], key


def test_final_head_matches_reference(models):
    for key, want in GOLDEN["final_head"].items():
        k, seed = key.split("/seed")
        x = np.random.default_rng(int(seed)).standard_normal(2048).astype(np.float32)
        vocab = GOLDEN["models"][k]["vocab"]
        nrm, lg, ids, tl = models[k].final_head(x, vocab, 8)
        assert str(qxo.fnv1a64(nrm)) == want["normalized_checksum"]
        assert str(qxo.fnv1a64(lg)) == want["logits_checksum"]
        assert int(ids[0]) == want["argmax_token"]
        assert float(tl[0]) == pytest.approx(want["argmax_logit"], rel=0, abs=0)
        # ranks 2..8 too: the reference's logits ordered by (value desc, index asc)
        assert [int(i) for i in ids] == want["top8_by_float"], key
        assert [float(v) for v in lg[:4]] == want["logits_sample"], key


@pytest.mark.parametrize("k", ["A", "B", "C"])
def test_state_loop_layer_dumps_match_reference(models, k):
    """Per step and layer: input, v-cur, kqv-out, ffn-inp, ffn-moe-out, output are
    bit-identical to the reference's --dump-residuals files (INT8 KV, double
    softmax, MoE with double router)."""
    g = GOLDEN["state_loop"][k]
    m = models[k]
    layers = GOLDEN["models"][k]["layers"]
    kv = qxo.KV(layers, g["ctx"])
    for s, tok in enumerate(g["input_tokens"]):
        x = m.embed(tok)
        for layer in range(layers):
            got = {"input": x.copy()}
            a, kqv, vcur = qxo.attention_layer(m, layer, s, kv, x)
            got["v-cur"], got["kqv-out"] = vcur, kqv
            x = x + a
            got["ffn-inp"] = x.copy()
            y, moe, ids, w = m.moe_layer(layer, x)
            got["ffn-moe-out"], got["output"] = moe, y
            x = y
            for ph in PHASES:
                assert str(qxo.fnv1a64(got[ph])) == g["dumps"][f"{s}/{layer}/{ph}"], (s, layer, ph)


def test_long_state_loop_matches_reference(models):
    """64 greedy steps at ctx 64 (softmax over up to 64 cached INT8 positions): every
    step's dumps bit-identical to the reference's, the same tokens and routed experts."""
    g = GOLDEN["state_loop_long"]
    m = models[g["model"]]
    kv = qxo.KV(1, g["ctx"])
    for s, tok in enumerate(g["input_tokens"]):
        x = m.embed(tok)
        got = {"input": x.copy()}
        a, kqv, vcur = qxo.attention_layer(m, 0, s, kv, x)
        got["v-cur"], got["kqv-out"] = vcur, kqv
        x = x + a
        got["ffn-inp"] = x.copy()
        y, moe, ids, w = m.moe_layer(0, x)
        got["ffn-moe-out"], got["output"] = moe, y
        assert [int(i) for i in ids] == g["selected_experts"][s], s
        for ph in PHASES:
            assert str(qxo.fnv1a64(got[ph])) == g["dumps"][f"{s}/0/{ph}"], (s, ph)


def _q8_probe_input(inject, values):
    """The q8-k-activation-probe's own input vectors (reference src/qx_format.c:4315-4323)."""
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


def test_q8k_activation_blocks_match_reference():
    """Q8_K blocks (d, 256 codes, 16 sums) byte-identical to the reference probe's."""
    for key, want in GOLDEN["q8k_activation"].items():
        inject, values = key.split("/")
        b = qxo.quantize_q8k(_q8_probe_input(inject, int(values)))
        assert str(qxo.fnv1a64(b)) == want["checksum"], key
        codes = b.reshape(-1, qxo.Q8K_BYTES)[:, 4:260].view(np.int8)
        assert int(codes.astype(np.int64).sum()) == want["quant_sum"], key
        assert float(b[:4].view(np.float32)[0]) == pytest.approx(want["first_scale"], rel=1e-8)


def test_q8k_quantize_rejects_non_finite():
    for bad in (np.nan, np.inf, -np.inf):
        x = _q8_probe_input("none", 256)
        x[128] = bad
        assert qxo.quantize_q8k(x) is None


def test_q8k_expert_dots_match_reference(models):
    """One expert row per format of model C (IQ2_XS, IQ3_XXS, IQ2_S, IQ4_XS, IQ3_S)."""
    m = models["C"]
    for key, want in GOLDEN["q8k_expert_dot"].items():
        name, rest = key.split("#")
        e, r = (int(v) for v in rest.split("/"))
        t, dims, raw = m.tensor(name)
        assert t == want["ggml_type"]
        n = int(dims[0])
        row_bytes = (n // 256) * BB_ALL[t]
        off = (e * int(dims[1]) + r) * row_bytes
        x = np.random.default_rng(n).standard_normal(n).astype(np.float32)
        y = qxo.matvec_q8k(t, raw[off:off + row_bytes], 1, n, x, expert=True)
        assert y[0] == np.float32(want["dot"]), key   # 9 significant digits identify a float exactly


def test_q8k_final_head_matches_reference(tmp_path):
    for key, want in GOLDEN["q8k_final_head"].items():
        k, seed = key.split("/seed")
        p = tmp_path / f"{k}.qxf"
        if not p.exists():
            qxg.generate_model(p, **GOLDEN["models"][k])
        m = qxo.Model(p, activation="q8_k_compat")
        x = np.random.default_rng(int(seed)).standard_normal(2048).astype(np.float32)
        _, lg, ids, tl = m.final_head(x, GOLDEN["models"][k]["vocab"], 8)
        m.close()
        assert str(qxo.fnv1a64(lg)) == want["logits_checksum"], key
        assert int(ids[0]) == want["argmax_token"] and float(tl[0]) == want["argmax_logit"]


@pytest.mark.parametrize("k", ["A", "B", "C"])
def test_q8k_state_loop_layer_dumps_match_reference(tmp_path, k):
    """--activation q8_k_compat: every per-layer dump bit-identical to the reference's."""
    g = GOLDEN["q8k_state_loop"][k]
    p = tmp_path / f"{k}.qxf"
    qxg.generate_model(p, **GOLDEN["models"][k])
    m = qxo.Model(p, activation="q8_k_compat")
    layers = GOLDEN["models"][k]["layers"]
    kv = qxo.KV(layers, g["ctx"])
    for s, tok in enumerate(g["input_tokens"]):
        x = m.embed(tok)
        for layer in range(layers):
            got = {"input": x.copy()}
            a, kqv, vcur = qxo.attention_layer(m, layer, s, kv, x)
            got["v-cur"], got["kqv-out"] = vcur, kqv
            x = x + a
            got["ffn-inp"] = x.copy()
            y, moe, ids, w = m.moe_layer(layer, x)
            got["ffn-moe-out"], got["output"] = moe, y
            x = y
            for ph in PHASES:
                assert str(qxo.fnv1a64(got[ph])) == g["dumps"][f"{s}/{layer}/{ph}"], (s, layer, ph)
    m.close()
