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


def test_state_loop_one_launch_matches_layer_seams(tmp_path):
    """Without residual dumps the state loop runs each step as one qxg_decode_token launch
    (the persistent decode on this benchmark-mix model) and rebuilds every layer's JSON entry
    from the step's records; with --dump-residuals it runs the per-layer seams.  Both give the
    same tokens and routed experts, the same layer-0 input checksum, and per-layer vector
    norms, scales and softmax sums within the bars; --bench times the device steps."""
    model = tmp_path / "m.qxf"
    qxg.generate_model(model, layers=2, vocab=1024, experts=16, seed=4321)
    base = [EXE, "state-loop-probe", "--in", str(model), "--prompt-token", "17", "--steps", "6", "--layers", "2", "--ctx",
            "16", "--kv", "int8", "--full-moe"]
    r1 = subprocess.run(base + ["--bench"], capture_output=True, text=True, timeout=120)
    assert r1.returncode == 0, r1.stderr
    dd = tmp_path / "dumps"
    dd.mkdir()
    r2 = subprocess.run(base + ["--dump-residuals", str(dd)], capture_output=True, text=True, timeout=120)
    assert r2.returncode == 0, r2.stderr
    one, seams = json.loads(r1.stdout), json.loads(r2.stdout)
    assert one["bench"]["timed"] == "device_steps" and one["bench"]["tokens_per_second"] > 0
    assert len(one["tokens"]) == len(seams["tokens"]) == 6
    for t1, t2 in zip(one["tokens"], seams["tokens"]):
        assert t1["input_token"] == t2["input_token"] and t1.get("selected_token") == t2.get("selected_token")
        assert t1["residual_checksum"] == t2["residual_checksum"]   # the embedding row, exact
        for l1, l2 in zip(t1["layers"], t2["layers"]):
            assert l1["selected_experts"] == l2["selected_experts"], (t1["step"], l1["layer"])
            assert np.allclose(l1["routing_weights"], l2["routing_weights"], rtol=1e-5, atol=0)
            for k in ("attention_output_vector_l2", "moe_output_l2", "k_scale", "v_scale"):
                assert abs(l1[k] / l2[k] - 1.0) <= REL_L2, (t1["step"], l1["layer"], k, l1[k], l2[k])
            for k in ("softmax_sum", "softmax_sum_min", "softmax_sum_max"):
                assert abs(l1[k] - 1.0) < 1e-6, (t1["step"], l1["layer"], k, l1[k])


def test_persistent_decode_in_a_second_process(tmp_path):
    """The runtime grants cooperative launches on a GPU to one process at a time: after this
    process has run the persistent decode, a child's cooperative launch is refused
    (hipErrorIllegalState) for as long as this process lives.  The child's decode then
    launches the same kernel plainly and gives the tokens this process's decode gives."""
    model = tmp_path / "m.qxf"
    qxg.generate_model(model, layers=2, vocab=1024, experts=16, seed=4321)
    c = qxg.Context(0)
    try:
        c.set_layer_path(1)
        c.load(model)
        assert c.persistent_path()
        c.kv_create(2, 16)
        c.generate([17], 3)   # a cooperative launch in this process
        r = subprocess.run([EXE, "state-loop-probe", "--in", str(model), "--prompt-token", "17", "--steps", "6", "--layers",
                            "2", "--ctx", "16", "--kv", "int8", "--full-moe"], capture_output=True, text=True, timeout=120)
        assert r.returncode == 0, r.stderr
        j = json.loads(r.stdout)
        c.kv_create(2, 16)
        tok = 17
        for t in j["tokens"]:
            assert t["input_token"] == tok
            _, lay, _, _, _ = c.decode_token(tok, t["position"], False, 1, want_layers=True)
            assert t["residual_checksum_after"] == qxg.fnv1a64(lay[-1]), t["step"]
            tok = t["selected_token"]
    finally:
        c.close()
