"""Writes tests/golden/golden.json from the reference CLI compiled in this container
(oracle/_ref/qxqxf, built by `make -C oracle ref` from /root/reference sources).

Inputs are QXF1 models written by this build's seeded generator
(qx-mini-c_amd/host/qxgen.c), so a test can regenerate identical bytes anywhere.
Only numeric summaries are stored: FNV-1a-64 of the reference's f32 outputs,
argmax/top tokens and a few sampled values; plus the reference's QXKVSNP1 KV
snapshots of the state-loop runs (kvsnap_*.bin, a few KB each).  Re-run here after changing the
generator:  python3 tests/golden/make_golden.py
"""
import json
import os
import re
import subprocess
import sys
import tempfile

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, os.path.join(ROOT, "qx-mini-c_amd"))
import qxg  # noqa: E402

REF = os.path.join(ROOT, "oracle", "_ref", "qxqxf")
GOLDEN_DIR = os.path.dirname(os.path.abspath(__file__))

# model specs used by the golden checks (layers, vocab, experts, seed)
MODELS = {
    "A": dict(layers=1, vocab=1024, experts=16, seed=1234),
    "B": dict(layers=2, vocab=2048, experts=128, seed=77),
    # the real checkpoint's per-layer quant mix: Q5_K v/o, IQ2_S gate/up, IQ4_XS and IQ3_S down
    "C": dict(layers=4, vocab=1024, experts=16, seed=4321, mix=1),
}
DECODE_BLOCKS_C = [("blk.1.attn_v.weight", [0, 3, 4095]), ("blk.3.attn_output.weight", [0, 7, 32767]),
                   ("blk.1.ffn_gate_exps.weight", [0, 5, 98303]), ("blk.3.ffn_up_exps.weight", [11]),
                   ("blk.2.ffn_down_exps.weight", [0, 9, 98303]), ("blk.1.ffn_down_exps.weight", [4, 98303])]
DECODE_BLOCKS = [("token_embd.weight", [0, 1, 4095]), ("output.weight", [0, 7, 8191]),
                 ("blk.0.attn_q.weight", [0, 3, 32767]), ("blk.0.attn_output.weight", [5]),
                 ("blk.0.ffn_gate_exps.weight", [0, 1, 98303]), ("blk.0.ffn_up_exps.weight", [12345]),
                 ("blk.0.ffn_down_exps.weight", [0, 2, 98303])]
PHASES = ["input", "v-cur", "kqv-out", "ffn-inp", "ffn-moe-out", "output"]
# q8_k_compat: expert rows of every expert format in model C (layer l % 4 picks the mix)
Q8_EXPERT_DOTS = [("blk.0.ffn_gate_exps.weight", 2048), ("blk.0.ffn_down_exps.weight", 768),
                  ("blk.1.ffn_up_exps.weight", 2048), ("blk.1.ffn_down_exps.weight", 768),
                  ("blk.2.ffn_down_exps.weight", 768)]
Q8_INJECT = ["none", "positive", "negative", "edge", "zero"]
# stage probes: (model, layer) pairs; model C's layer l takes quant mix l % 4
STAGE_CASES = [("A", 0), ("B", 1), ("C", 0), ("C", 1), ("C", 2), ("C", 3)]
ATTN_SIDECARS = ["attn_norm", "Vcur", "kqv_out", "attn_out", "ffn_inp"]
MOE_SIDECARS = ["ffn_norm", "ffn_moe_logits", "ffn_moe_probs", "ffn_moe_topk", "ffn_moe_weights",
                "ffn_moe_weights_sum", "ffn_moe_weights_norm", "ffn_moe_gate", "ffn_moe_up", "ffn_moe_swiglu",
                "ffn_moe_down", "ffn_moe_weighted"]


def stage_input(k, layer, scale):
    """the seeded layer / ffn input of a stage-probe case"""
    seed = 1000 * (ord(k) - ord("A")) + layer
    return (np.random.default_rng(seed).standard_normal(2048) * scale).astype(np.float32)


def run(args):
    r = subprocess.run([REF] + args, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"{args[0]} failed: {r.stderr}")
    return r.stdout


def fnv_file(path):
    return qxg.fnv1a64(np.fromfile(path, np.uint8))


def main():
    if not os.path.exists(REF):
        sys.exit(f"{REF} missing: run make -C oracle ref (needs /root/reference)")
    out = {"models": MODELS, "decode_block": {}, "final_head": {}, "state_loop": {},
           "q8k_activation": {}, "q8k_expert_dot": {}, "q8k_final_head": {}, "q8k_state_loop": {}}
    # Q8_K activation blocks of the probe's own inputs (src/qx_format.c:4304-4345)
    for inj in Q8_INJECT:
        for values in (256, 512, 4096):
            j = json.loads(run(["q8-k-activation-probe", "--values", str(values), "--inject", inj]))
            out["q8k_activation"][f"{inj}/{values}"] = {"checksum": str(j["checksum"]), "quant_sum": j["quant_sum"],
                                                        "first_scale": j["first_scale"]}
    with tempfile.TemporaryDirectory() as d:
        paths = {}
        for k, spec in MODELS.items():
            paths[k] = os.path.join(d, f"{k}.qxf")
            qxg.generate_model(paths[k], **spec)
        # block decoders (reference decode-block, src/qx_format.c:2219-2264)
        for name, blocks in DECODE_BLOCKS:
            for b in blocks:
                j = json.loads(run(["decode-block", "--in", paths["A"], "--name", name, "--block", str(b)]))
                out["decode_block"][f"{name}#{b}"] = {"f32_checksum": str(j["f32_checksum"]),
                                                       "first8": j["first8"]}
        for name, blocks in DECODE_BLOCKS_C:
            for b in blocks:
                j = json.loads(run(["decode-block", "--in", paths["C"], "--name", name, "--block", str(b)]))
                out["decode_block"][f"C:{name}#{b}"] = {"f32_checksum": str(j["f32_checksum"]), "first8": j["first8"]}
        # final head probe (src/qx_format.c:5369-5411) on seeded residuals
        for k in ("A", "B"):
            for seed in (1, 2):
                x = np.random.default_rng(seed).standard_normal(2048).astype(np.float32)
                rp = os.path.join(d, f"r{k}{seed}.f32")
                x.tofile(rp)
                od = os.path.join(d, f"h{k}{seed}")
                os.mkdir(od)
                j = json.loads(run(["final-head-probe", "--in", paths[k], "--residual", rp, "--out-dir", od]))
                lg = np.fromfile(os.path.join(od, "logits.f32"), np.float32)
                order = np.lexsort((np.arange(len(lg)), -lg.astype(np.float64)))[:8]
                out["final_head"][f"{k}/seed{seed}"] = {
                    "normalized_checksum": str(j["normalized_checksum"]), "logits_checksum": str(j["logits_checksum"]),
                    "argmax_token": j["argmax_token"], "argmax_logit": j["argmax_logit"],
                    "top8_by_float": [int(i) for i in order], "logits_sample": [float(v) for v in lg[:4]]}
        # q8_k_compat: single expert rows (src/qx_format.c:5413-5470) and the Q6_K head
        for name, n in Q8_EXPERT_DOTS:
            ap = os.path.join(d, f"act{n}.f32")
            np.random.default_rng(n).standard_normal(n).astype(np.float32).tofile(ap)
            for e, r in ((0, 0), (3, 5), (15, 767 if n == 2048 else 2047)):
                j = json.loads(run(["expert-q8-k-dot-probe", "--in", paths["C"], "--name", name, "--expert", str(e),
                                    "--row", str(r), "--activation", ap]))
                out["q8k_expert_dot"][f"{name}#{e}/{r}"] = {"ggml_type": j["ggml_type"], "dot": j["dot"]}
        for k in ("A", "B"):
            for seed in (1, 2):
                rp = os.path.join(d, f"r{k}{seed}.f32")
                od = os.path.join(d, f"q{k}{seed}")
                os.mkdir(od)
                j = json.loads(run(["final-head-probe", "--in", paths[k], "--residual", rp, "--out-dir", od,
                                    "--activation", "q8_k_compat"]))
                out["q8k_final_head"][f"{k}/seed{seed}"] = {
                    "logits_checksum": str(j["logits_checksum"]), "argmax_token": j["argmax_token"],
                    "argmax_logit": j["argmax_logit"]}
        for k, steps in (("A", 5), ("B", 3), ("C", 3)):
            dd = os.path.join(d, f"q{k}")
            os.mkdir(dd)
            layers = MODELS[k]["layers"]
            txt = run(["state-loop-probe", "--in", paths[k], "--prompt-token", "17", "--steps", str(steps),
                       "--layers", str(layers), "--ctx", "8", "--kv", "int8", "--full-moe", "--activation",
                       "q8_k_compat", "--dump-residuals", dd])
            toks = [int(t) for t in re.findall(r'"input_token": (\d+)', txt)]
            dumps = {f"{s}/{layer}/{ph}": str(fnv_file(os.path.join(dd, f"step-{s}-layer-{layer}-{ph}.f32")))
                     for s in range(steps) for layer in range(layers) for ph in PHASES}
            out["q8k_state_loop"][k] = {"input_tokens": toks, "steps": steps, "ctx": 8, "dumps": dumps}
        # full-MoE state loop with INT8 KV and per-layer dumps (src/qx_format.c:5970-6719)
        for k, steps in (("A", 5), ("B", 4), ("C", 3)):
            dd = os.path.join(d, f"s{k}")
            os.mkdir(dd)
            layers = MODELS[k]["layers"]
            snap = os.path.join(GOLDEN_DIR, f"kvsnap_{k}.bin")
            txt = run(["state-loop-probe", "--in", paths[k], "--prompt-token", "17", "--steps", str(steps),
                       "--layers", str(layers), "--ctx", "8", "--kv", "int8", "--full-moe", "--dump-residuals", dd,
                       "--kv-snapshot-out", snap])
            hdr = np.fromfile(snap, np.uint32, count=12)
            out.setdefault("kv_snapshot", {})[k] = {
                "file": os.path.basename(snap), "final_token": int(re.search(r'"final_token": (\d+)', txt).group(1)),
                "positions": int(hdr[4]), "seed": int(hdr[11]), "bytes": os.path.getsize(snap)}
            toks = [int(t) for t in re.findall(r'"input_token": (\d+)', txt)]
            experts = [[int(e) for e in re.findall(r"\d+", m)]
                       for m in re.findall(r'"selected_experts": \[([0-9, ]*)\]', txt)]
            dumps = {}
            for s in range(steps):
                for layer in range(layers):
                    for ph in PHASES:
                        dumps[f"{s}/{layer}/{ph}"] = str(fnv_file(os.path.join(dd, f"step-{s}-layer-{layer}-{ph}.f32")))
            out["state_loop"][k] = {"input_tokens": toks, "steps": steps, "ctx": 8, "dumps": dumps,
                                    "selected_experts": experts}
        # a long state loop: 64 greedy steps at ctx 64 on model A, so the reference pins the
        # attention softmax over many positions (every step's per-layer dumps)
        dd = os.path.join(d, "slong")
        os.mkdir(dd)
        txt = run(["state-loop-probe", "--in", paths["A"], "--prompt-token", "17", "--steps", "64", "--layers", "1",
                   "--ctx", "64", "--kv", "int8", "--full-moe", "--dump-residuals", dd])
        out["state_loop_long"] = {
            "model": "A", "steps": 64, "ctx": 64,
            "input_tokens": [int(t) for t in re.findall(r'"input_token": (\d+)', txt)],
            "selected_experts": [[int(e) for e in re.findall(r"\d+", m)]
                                 for m in re.findall(r'"selected_experts": \[([0-9, ]*)\]', txt)],
            "dumps": {f"{s_}/0/{ph}": str(fnv_file(os.path.join(dd, f"step-{s_}-layer-0-{ph}.f32")))
                      for s_ in range(64) for ph in PHASES}}
        # attention and MoE stage probes (src/qx_format.c:5478-5725) on seeded inputs
        out["attention_stage"], out["moe_stage"] = {}, {}
        for k, layer in STAGE_CASES:
            x = stage_input(k, layer, 1.0)
            xp = os.path.join(d, f"stage{k}{layer}.f32")
            x.tofile(xp)
            for act in ("f32", "q8_k_compat"):
                for kv in ("f32", "f16"):
                    od = os.path.join(d, f"as{k}{layer}{act}{kv}")
                    os.mkdir(od)
                    j = json.loads(run(["attention-stage-probe", "--in", paths[k], "--layer", str(layer), "--layer-in", xp,
                                        "--out-dir", od, "--activation", act, "--kv", kv]))
                    j["sidecars"] = {n: str(fnv_file(os.path.join(od, f"{n}-{layer}.f32"))) for n in ATTN_SIDECARS}
                    out["attention_stage"][f"{k}/{layer}/{act}/{kv}"] = j
                od = os.path.join(d, f"ms{k}{layer}{act}")
                os.mkdir(od)
                j = json.loads(run(["moe-stage-probe", "--in", paths[k], "--layer", str(layer), "--ffn-inp", xp,
                                    "--out-dir", od, "--activation", act]))
                j["sidecars"] = {n: str(fnv_file(os.path.join(od, f"{n}-{layer}.f32"))) for n in MOE_SIDECARS}
                out["moe_stage"][f"{k}/{layer}/{act}"] = j
        # state loop variants: resume from the reference's own snapshots (the continuation
        # token must be the snapshot's next token, src/qx_format.c:6165-6177), residual
        # replay from a layer (--start-layer/--residual-in, :6021-6025, 6260-6268), a layer
        # prefix (--layers below the manifest's), and the reference's error messages
        out["state_loop_resume"], out["state_loop_replay"], out["state_loop_prefix"], out["state_loop_errors"] = {}, {}, {}, {}
        for k, steps in (("A", 2), ("B", 2), ("C", 2)):
            layers = MODELS[k]["layers"]
            snap = os.path.join(GOLDEN_DIR, f"kvsnap_{k}.bin")
            nt = out["kv_snapshot"][k]["final_token"]
            dd = os.path.join(d, f"r{k}")
            os.mkdir(dd)
            txt = run(["state-loop-probe", "--in", paths[k], "--prompt-token", str(nt), "--steps", str(steps),
                       "--layers", str(layers), "--ctx", "8", "--kv", "int8", "--full-moe", "--dump-residuals", dd,
                       "--kv-snapshot-in", snap])
            j = json.loads(txt)
            pb = j["position_base"]
            dumps = {f"{s_}/{layer}/{ph}": str(fnv_file(os.path.join(dd, f"step-{pb + s_}-layer-{layer}-{ph}.f32")))
                     for s_ in range(steps) for layer in range(layers) for ph in PHASES}
            out["state_loop_resume"][k] = {
                "prompt_token": nt, "steps": steps, "position_base": pb, "final_token": j["final_token"],
                "input_tokens": [t["input_token"] for t in j["tokens"]],
                "selected_experts": [[ly["selected_experts"] for ly in t["layers"]] for t in j["tokens"]],
                "k_checksums": [[str(ly["k_checksum"]) for ly in t["layers"]] for t in j["tokens"]],
                "dumps": dumps}
        for k, start in (("B", 1), ("C", 2)):
            layers = MODELS[k]["layers"]
            x = stage_input(k, 100 + start, 0.5)
            xp = os.path.join(d, f"replay{k}.f32")
            x.tofile(xp)
            dd = os.path.join(d, f"p{k}")
            os.mkdir(dd)
            j = json.loads(run(["state-loop-probe", "--in", paths[k], "--prompt-token", "17", "--steps", "1",
                                "--layers", str(layers), "--ctx", "8", "--kv", "int8", "--full-moe", "--dump-residuals", dd,
                                "--start-layer", str(start), "--residual-in", xp]))
            t0 = j["tokens"][0]
            out["state_loop_replay"][k] = {
                "start_layer": start, "input_scale": 0.5, "residual_checksum": str(t0["residual_checksum"]),
                "layers": [ly["layer"] for ly in t0["layers"]],
                "selected_experts": [ly["selected_experts"] for ly in t0["layers"]],
                "residual_output_checksums": [str(ly["residual_output_checksum"]) for ly in t0["layers"]],
                "dumps": {f"{layer}/{ph}": str(fnv_file(os.path.join(dd, f"step-0-layer-{layer}-{ph}.f32")))
                          for layer in range(start, layers) for ph in PHASES}}
        dd = os.path.join(d, "prefixB")
        os.mkdir(dd)
        j = json.loads(run(["state-loop-probe", "--in", paths["B"], "--prompt-token", "17", "--steps", "2", "--layers", "1",
                            "--ctx", "8", "--kv", "int8", "--full-moe", "--dump-residuals", dd]))
        out["state_loop_prefix"]["B"] = {
            "layers": j["layers"], "final_token": j["final_token"], "top_keys": sorted(j.keys()),
            "step_keys": sorted(j["tokens"][0].keys()), "layer_keys": sorted(j["tokens"][0]["layers"][0].keys()),
            "dumps": {f"{s_}/0/{ph}": str(fnv_file(os.path.join(dd, f"step-{s_}-layer-0-{ph}.f32")))
                      for s_ in range(2) for ph in PHASES}}
        def err_of(args):
            r = subprocess.run([REF] + args, capture_output=True, text=True)
            return r.returncode, r.stderr.strip()
        base = ["state-loop-probe", "--in", paths["A"], "--steps", "1", "--layers", "1", "--ctx", "8", "--kv", "int8",
                "--full-moe"]
        snapA = os.path.join(GOLDEN_DIR, "kvsnap_A.bin")
        out["state_loop_errors"] = {
            "token_mismatch": err_of(base + ["--prompt-token", "3", "--kv-snapshot-in", snapA]),
            "replay_two_steps": err_of(["state-loop-probe", "--in", paths["A"], "--steps", "2", "--layers", "1", "--ctx", "8",
                                        "--kv", "int8", "--full-moe", "--prompt-token", "17", "--start-layer", "0",
                                        "--residual-in", os.path.join(d, "replayB.f32")]),
            "replay_start_beyond": err_of(base + ["--prompt-token", "17", "--start-layer", "1", "--residual-in",
                                                  os.path.join(d, "replayB.f32")]),
            "ctx_too_small": err_of(base + ["--prompt-token", str(out["kv_snapshot"]["A"]["final_token"]),
                                            "--kv-snapshot-in", snapA, "--ctx", "4"]),
        }
    dst = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden.json")
    with open(dst, "w") as f:
        json.dump(out, f, indent=1, sort_keys=True)
    print(f"wrote {dst}")


if __name__ == "__main__":
    main()
