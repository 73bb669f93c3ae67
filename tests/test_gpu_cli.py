"""The qxqxf CLI on the GPU: state-loop-probe with --dump-residuals in both activation
modes, each per-layer dump checked against the oracle run on the same input tokens
(the reference's Python tests drive its CLI the same way, through subprocess).  Without
--final-head (which needs the full Qwen3-30B-A3B manifest, tested at size) the next
token comes from the reference's token scan, as in its own state loop."""
import json
import os
import subprocess

import numpy as np
import pytest

import qxo
import qxg
from helpers import REL_L2, rel_l2

pytestmark = pytest.mark.gpu
EXE = os.path.join(os.path.dirname(qxg.__file__), "bin", "qxqxf")
PHASES = ["input", "v-cur", "kqv-out", "ffn-inp", "ffn-moe-out", "output"]


@pytest.mark.parametrize("act,tol", [("f32", REL_L2), ("q8_k_compat", 2e-3)])
def test_state_loop_probe_dumps(tmp_path, act, tol):
    """Each stage is replayed by the oracle on the CLI's own dumped input of that stage
    (same-input chaining: the attention on "input" with a KV cache the oracle builds
    from those inputs, the MoE on "ffn-inp"), so every stage meets its bar alone."""
    model = tmp_path / "m.qxf"
    qxg.generate_model(model, layers=2, vocab=1024, experts=16, seed=1234, mix=1)
    dd = tmp_path / "dumps"
    dd.mkdir()
    r = subprocess.run([EXE, "state-loop-probe", "--in", str(model), "--prompt-token", "17", "--steps", "3", "--layers",
                        "2", "--ctx", "8", "--kv", "int8", "--full-moe", "--activation", act, "--dump-residuals", str(dd)],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    j = json.loads(r.stdout)
    assert j["activation_format"] == act
    toks = [t["input_token"] for t in j["tokens"]]
    m = qxo.Model(model, activation=act)
    kv = qxo.KV(2, 8)
    dump = lambda s, layer, ph: np.fromfile(dd / f"step-{s}-layer-{layer}-{ph}.f32", np.float32)
    worst = {}
    for s, tok in enumerate(toks):
        assert rel_l2(dump(s, 0, "input"), m.embed(tok)) == 0.0
        for layer in range(2):
            x = dump(s, layer, "input")
            a, kqv, vcur = qxo.attention_layer(m, layer, s, kv, x)
            got = {"v-cur": (dump(s, layer, "v-cur"), vcur), "kqv-out": (dump(s, layer, "kqv-out"), kqv),
                   "ffn-inp": (dump(s, layer, "ffn-inp"), x + a)}
            y, moe, _, _ = m.moe_layer(layer, dump(s, layer, "ffn-inp"))
            got["ffn-moe-out"] = (dump(s, layer, "ffn-moe-out"), moe)
            got["output"] = (dump(s, layer, "output"), y)
            for ph, (g, ref) in got.items():
                e = rel_l2(g, ref)
                worst[ph] = max(worst.get(ph, 0.0), e)
                assert e <= tol, (act, s, layer, ph, e)
            if layer == 0:
                assert rel_l2(dump(s, 1, "input"), dump(s, 0, "output")) == 0.0
    m.close()
    print(act, {k: f"{v:.2e}" for k, v in worst.items()})


def test_long_state_loop_probe_vs_reference(tmp_path):
    """The reference's 64-step loop at ctx 64 (golden state_loop_long, model A) through this
    CLI: the same input tokens and routed experts as the reference, and every step's
    attention and MoE replayed by the oracle on the CLI's own dumped inputs (1e-5)."""
    GOLDEN = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "golden.json")))
    g = GOLDEN["state_loop_long"]
    model = tmp_path / "a.qxf"
    qxg.generate_model(model, **GOLDEN["models"][g["model"]])
    dd = tmp_path / "dumps"
    dd.mkdir()
    r = subprocess.run([EXE, "state-loop-probe", "--in", str(model), "--prompt-token", "17", "--steps", str(g["steps"]),
                        "--layers", "1", "--ctx", str(g["ctx"]), "--kv", "int8", "--full-moe", "--dump-residuals", str(dd)],
                       capture_output=True, text=True, timeout=240)
    assert r.returncode == 0, r.stderr
    j = json.loads(r.stdout)
    assert [t["input_token"] for t in j["tokens"]] == g["input_tokens"]
    assert [t["layers"][0]["selected_experts"] for t in j["tokens"]] == g["selected_experts"]
    m = qxo.Model(model)
    kv = qxo.KV(1, g["ctx"])
    dump = lambda s, ph: np.fromfile(dd / f"step-{s}-layer-0-{ph}.f32", np.float32)
    worst = 0.0
    for s in range(g["steps"]):
        a, kqv, vcur = qxo.attention_layer(m, 0, s, kv, dump(s, "input"))
        y, moe, _, _ = m.moe_layer(0, dump(s, "ffn-inp"))
        for got, ref in ((dump(s, "kqv-out"), kqv), (dump(s, "ffn-inp"), dump(s, "input") + a), (dump(s, "output"), y)):
            e = rel_l2(got, ref)
            worst = max(worst, e)
            assert e <= REL_L2, (s, e)
    m.close()
    print(f"64-step loop: worst same-input rel L2 {worst:.2e}")
