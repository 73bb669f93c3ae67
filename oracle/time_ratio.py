"""ORACLE — test infrastructure only.  Times the clean-room oracle (liboracle.so) against
the reference CLI compiled from its own sources (oracle/_ref/qxqxf) on the same generated
QXF1 file: a greedy state loop with full MoE, INT8 KV and the final head, one thread each.
Prints one JSON line with both wall times per token and their ratio, and checks that the two
produce the same greedy tokens.  Needs oracle/_ref/qxqxf (built here from /root/reference by
`make -C oracle ref`); used to calibrate the CPU baseline that bench.py reports.

    python oracle/time_ratio.py [--layers 4] [--steps 3]
"""
import argparse
import json
import os
import re
import subprocess
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
sys.path.insert(0, HERE)
sys.path.insert(0, os.path.join(ROOT, "qx-mini-c_amd"))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--steps", type=int, default=2)
    ap.add_argument("--prompt-token", type=int, default=17)
    args = ap.parse_args()
    ref = os.path.join(HERE, "_ref", "qxqxf")
    if not os.path.exists(ref):
        sys.exit("oracle/_ref/qxqxf is not built (make -C oracle ref, with /root/reference present)")
    import qxg
    import qxo
    V, L = 151936, 48   # the reference's final head requires the exact Qwen3-30B-A3B manifest
    model = qxg.MemModel(L, V, 128, True, True, seed=11)   # in-memory file; the child opens /proc/<pid>/fd/N
    try:
        path = model.path.replace("/proc/self/", f"/proc/{os.getpid()}/")
        cmd = [ref, "state-loop-probe", "--in", path, "--prompt-token", str(args.prompt_token), "--steps", str(args.steps),
               "--layers", str(L), "--ctx", "16", "--kv", "int8", "--full-moe", "--final-head", "--top-n", "1"]
        t0 = time.perf_counter()
        r = subprocess.run(cmd, capture_output=True, text=True, check=True)
        ref_s = time.perf_counter() - t0
        ref_tokens = [int(t) for t in re.findall(r'"input_token": (\d+)', r.stdout)]
        m = qxo.Model(path)
        kv = qxo.KV(L, 16)
        tok, toks = args.prompt_token, []
        t0 = time.perf_counter()
        for step in range(args.steps):
            toks.append(tok)
            _, _, _, ids, _ = qxo.decode_token(m, tok, step, kv, L, True, V, 1)
            tok = int(ids[0])
        ora_s = time.perf_counter() - t0
        m.close()
    finally:
        model.close()
    print(json.dumps({"layers": L, "steps": args.steps, "reference_s_per_token": round(ref_s / args.steps, 4),
                      "oracle_s_per_token": round(ora_s / args.steps, 4), "oracle_over_reference": round(ora_s / ref_s, 4),
                      "reference_includes": "process start, file open, per-call tensor checksum verification",
                      "same_tokens": toks == ref_tokens[:len(toks)], "tokens": toks, "reference_tokens": ref_tokens}))


if __name__ == "__main__":
    main()
