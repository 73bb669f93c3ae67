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
