"""Batch-1 decode benchmark of the 48-layer Qwen3-30B-A3B-shaped random-init model
(config 4 of the hot path) on one MI355X, with the roofline of the dominant
kernel and the oracle's CPU time on a bounded sample of the same workload.

A step is one greedy decode token: Q4_K embedding, 48 x (attention with INT8 KV +
top-8 MoE), output RMSNorm and the full Q6_K head with argmax fed back on the
device.  Prints one JSON line."""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "qx-mini-c_amd"))

HBM_PEAK_GBS = 8000.0
LAYERS, VOCAB, EXPERTS = 48, 151936, 128
# algorithmic bytes (weights read once per use; 74/98/136/210/144-byte blocks)
GATE_UP_WEIGHTS = 8 * 2 * 768 * 8 * 74          # 8 experts x (gate, up) x 768 rows x 8 blocks
DOWN_WEIGHTS = 8 * 2048 * 3 * 98
ATTN_WEIGHTS = (4096 + 512 + 512) * 8 * 136 + 2048 * 16 * 136
ROUTER = 128 * 2048 * 4
NORMS = 2048 * 4 * 2 + 128 * 4 * 2
LAYER_BYTES = GATE_UP_WEIGHTS + DOWN_WEIGHTS + ATTN_WEIGHTS + ROUTER + NORMS      # 23,184,384
HEAD_BYTES = VOCAB * 8 * 210
TOKEN_BYTES = LAYERS * LAYER_BYTES + HEAD_BYTES + 2048 * 4 + 8 * 144            # 1,368,112,256
KERNEL_BYTES = {
    # weights + activations read + outputs written, per launch
    "gate_up": GATE_UP_WEIGHTS + 2048 * 4 * 2 + 8 * 768 * 4,
    "down": DOWN_WEIGHTS + 8 * 768 * 4 + 2048 * 4 * 2,
    "qkv": (4096 + 512 + 512) * 8 * 136 + 2048 * 4 * 2 + 5120 * 4,
    "oproj": 2048 * 16 * 136 + 4096 * 4 + 2048 * 4 * 2,
    "head": HEAD_BYTES + 2048 * 4 * 2 + VOCAB * 4,
    # the persistent decode kernel: one launch runs every step of a generate call (all 48
    # layers and the head per token); per-launch bytes are formed in main() from the steps
    # and the KV rows read
    "layers": TOKEN_BYTES,
}


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def kv_bytes(p0, n):
    """INT8 K+V rows (512 B each) and two f32 scales per position, 48 layers, positions p0..p0+n-1."""
    return sum(LAYERS * (p + 1) * 1032 for p in range(p0, p0 + n))


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(model_path, prompt_kv, first_token, p0, budget_s):
    """The oracle (oracle/qxo.c, scalar, one thread) decoding the GPU's first timed positions:
    its KV cache holds the prompt's rows as the GPU wrote them (positions 0..p0-1), and it
    decodes from the GPU's first generated token at positions p0, p0 + 1, ... within budget_s.
    Also times one FNV-1a 64 pass over the Q6_K head tensor: the reference verifies that
    checksum on every final-head call (src/qx_format.c:3631-3632), which neither the oracle nor
    the GPU path repeats per token; the "with_head_fnv" rate adds it to each token."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import qxo
    m = qxo.Model(model_path)
    kv = qxo.KV(LAYERS, p0 + 8)
    for l, (k, v, ks, vs) in enumerate(prompt_kv):
        kv.k[l, :p0], kv.v[l, :p0], kv.ks[l, :p0], kv.vs[l, :p0] = k, v, ks, vs
    done, t0, c0 = 0, time.perf_counter(), time.process_time()
    tok = first_token
    while done < 2:
        _, _, _, ids, _ = qxo.decode_token(m, tok, p0 + done, kv, LAYERS, True, VOCAB, 1)
        tok = int(ids[0])
        done += 1
        if time.perf_counter() - t0 > budget_s:
            break
    wall, cpu = time.perf_counter() - t0, time.process_time() - c0
    _, _, head = m.tensor("output.weight")
    t1 = time.perf_counter()
    qxo.fnv1a64(head)
    fnv_s = time.perf_counter() - t1
    m.close()
    return {"value": done / wall, "unit": "tok/s", "cores": 1, "kind": "port", "cpu": cpu_model(),
            "with_head_fnv": round(done / (wall + done * fnv_s), 5), "head_fnv_s": round(fnv_s, 4),
            "sample": f"{done} greedy decode tokens at positions {p0}..{p0 + done - 1} of the same model, the GPU's "
                      f"first timed positions (prompt KV rows taken from the GPU; oracle/qxo.c, scalar, 1 thread); "
                      f"wall {wall:.2f} s, process CPU {cpu:.2f} s"}


def measured_traffic_ratio(kernel):
    """HBM bytes over algorithmic bytes of `kernel` from the committed rocprofv3 --pmc summary
    (FETCH_SIZE + WRITE_SIZE, each scaled by the same counter's reading for a plain device
    copy of known size, divided by the profiled launch's algorithmic bytes): (ratio, file), or
    (None, None) when no summary is committed for it.  The ratio carries over to a launch of
    another step count (the counted excess is per token), so `traffic` is this run's
    algorithmic bytes times it."""
    key = f"traffic_ratio[{kernel}]="
    for name in ("decode_config4_persistent_traffic.md", "decode_config4_per_phase_traffic.md"):
        path = os.path.join(ROOT, "profiles", name)
        if not os.path.exists(path):
            continue
        with open(path) as f:
            for line in f:
                if line.startswith(key):
                    return float(line[len(key):]), f"profiles/{name}"
    return None, None


def copy_calibration(mib):
    """Copies a mib-MiB device buffer 4 times (and fills it once): the known-size
    kernels whose FETCH_SIZE / WRITE_SIZE readings scale the decode kernels' counters."""
    import torch
    n = mib << 20
    a = torch.empty(n, dtype=torch.uint8, device="cuda:0")
    a.fill_(1)
    b = torch.empty_like(a)
    for _ in range(4):
        b.copy_(a)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes": n, "copies": 4}), flush=True)


# config 5: algorithmic flops of one layer's expert GEMMs over T tokens (8 assignments each)
def expert_flops(t):
    return {"pf_gate_up": 2.0 * t * 8 * 2 * 768 * 2048, "pf_down": 2.0 * t * 8 * 2048 * 768}


def prefill_leg(ctx, args):
    """Config 5: batched prefill of T seeded ids, then greedy decode from the prefilled
    INT8 KV.  The expert gate/up GEMM is timed in situ (event pairs around each of its
    48 launches) for the MFMA roofline."""
    T, G = args.prefill_tokens, args.prefill_decode
    ids = np.random.default_rng(args.seed + 5).integers(0, VOCAB, size=T).astype(np.uint32)
    ctx.kv_create(LAYERS, T + G + 1)
    ctx.prefill(ids, 0, True, 1)                                      # warmup
    ctx.kv_create(LAYERS, T + G + 1)
    ctx.profile_kernel(qxg_kernels()["pf_gate_up"])
    _, _, first, _, ms_prof = ctx.prefill(ids, 0, True, 1)
    launches, kern_ms = ctx.profile_result()
    ctx.profile_kernel(-1)
    ctx.kv_create(LAYERS, T + G + 1)
    t0 = time.perf_counter()
    _, _, first2, _, ms = ctx.prefill(ids, 0, True, 1)
    wall = time.perf_counter() - t0
    assert int(first2[0]) == int(first[0]), "prefill result changed between identical runs"
    toks, dec_ms = ctx.generate([int(first2[0])], G - 1, T)
    avg = kern_ms / 1e3 / max(launches, 1)
    fl = expert_flops(T)["pf_gate_up"]
    expert_bytes = LAYERS * EXPERTS * (2 * 768 * 8 * 74 + 2048 * 3 * 98)
    log(f"prefill {T} tokens: {wall * 1e3:.2f} ms wall, {ms:.2f} ms device; gate/up {launches} launches "
        f"avg {avg * 1e6:.1f} us; decode {G - 1} tokens after it: {dec_ms:.2f} ms")
    return {
        "workload": f"config5: prefill of {T} seeded token ids (uniform in [0,{VOCAB})) through the same 48-layer "
                    f"model, head on the last, then {G} greedy tokens (the first from the prefill head)",
        "tokens": T, "ms": round(wall * 1e3, 3), "device_ms": round(ms, 3), "tok_s": round(T / wall, 1),
        "dtype": "fp16 MFMA (codes exact; activations split hi+lo), f32 accumulation",
        "roofline": {"bound": "mfma", "kernel": "pf_gate_up", "achieved": round(fl / avg / 1e12, 2),
                     "peak": 2500.0, "unit": "TFLOP/s", "frac": round(fl / avg / 1e12 / 2500.0, 4),
                     "flops_per_launch": fl, "avg_launch_us": round(avg * 1e6, 2), "launches": launches,
                     "note": "algorithmic flops 2*M*N*K (M = 8T assignments); the split activations make the "
                             "matrix cores execute 2x these, plus padding of each expert to 32 rows"},
        "expert_weights_GBs": round(expert_bytes / (ms / 1e3) / 1e9, 1),
        "decode_after": {"steps": G - 1, "tok_s": round((G - 1) / (dec_ms / 1e3), 1),
                         "positions": f"{T}..{T + G - 2}"},
    }


def qxg_kernels():
    import qxg
    return qxg.KERNELS


def long_context_leg(ctx, args):
    """Decode at the end of the 4096-long context (config 5's "4096-long INT8 KV"): the
    cache holds seeded INT8 rows at positions 0..p0-1 of every layer, then one persistent
    launch generates n greedy tokens at positions p0..4095; the KV rows read per token grow
    to 203 MB at position 4095, counted in the roofline."""
    n = args.long_steps
    p0 = 4096 - n
    rng = np.random.default_rng(args.seed + 9)
    ctx.kv_create(LAYERS, 4096)
    t0 = time.perf_counter()
    for layer in range(LAYERS):
        k = rng.integers(-127, 128, size=(p0, 512), dtype=np.int8)
        v = rng.integers(-127, 128, size=(p0, 512), dtype=np.int8)
        ks = (rng.uniform(0.5, 2.0, size=p0) / 127.0).astype(np.float32)
        vs = (rng.uniform(0.5, 2.0, size=p0) / 127.0).astype(np.float32)
        ctx.kv_write(layer, 0, k, v, ks, vs)
    log(f"long context: seeded {p0} INT8 rows x {LAYERS} layers in {time.perf_counter() - t0:.1f} s")
    ctx.generate([11], n, p0)                      # warmup (rewrites rows p0.. itself)
    t0 = time.perf_counter()
    toks, dev_ms = ctx.generate([11], n, p0)
    wall = time.perf_counter() - t0
    tok_s = n / wall
    token_bytes = TOKEN_BYTES + kv_bytes(p0, n) / n
    log(f"long context: {n} tokens at positions {p0}..4095: {wall * 1e3:.2f} ms wall ({tok_s:.1f} tok/s)")
    return {"workload": f"{n} greedy tokens at positions {p0}..4095 over a seeded INT8 KV cache of the same model "
                        f"(4096-long context)", "positions": f"{p0}..4095", "steps": n,
            "tok_s": round(tok_s, 1), "ms_per_token": round(wall * 1e3 / n, 4),
            "algorithmic_bytes_per_token": int(token_bytes),
            "frac": round(token_bytes * tok_s / 1e9 / HBM_PEAK_GBS, 4)}


def mix_decode_leg(args):
    """Decode on the real checkpoint's per-layer quant mix (layer l % 4: Q5_K or IQ4_XS V/O,
    IQ2_S or IQ2_XS gate/up, IQ3_XXS / IQ4_XS / IQ3_S down): these layers decode one kernel per
    phase (replayed step graph)."""
    import qxg
    model = qxg.MemModel(LAYERS, VOCAB, EXPERTS, True, True, seed=args.seed, mix=1)
    ctx = qxg.Context(0)
    ctx.load(model.path, verify=False)
    prompt = np.random.default_rng(args.seed).integers(0, VOCAB, size=8).astype(np.uint32)
    n = args.mix_steps
    ctx.kv_create(LAYERS, 8 + 2 * n + 1)
    first, _ = ctx.generate(prompt, 1, 0)
    ctx.generate([int(first[0])], n, 8)            # warmup (records the step graph)
    ctx.kv_create(LAYERS, 8 + 2 * n + 1)
    first, _ = ctx.generate(prompt, 1, 0)
    t0 = time.perf_counter()
    ctx.generate([int(first[0])], n, 8)
    wall = time.perf_counter() - t0
    ctx.close()
    model.close()
    log(f"real-mix decode: {n} tokens in {wall * 1e3:.2f} ms ({n / wall:.1f} tok/s)")
    return {"workload": f"{n} greedy tokens at positions 8..{7 + n} after an 8-token prompt, the 48-layer model in "
                        "the real checkpoint's per-layer formats", "steps": n, "tok_s": round(n / wall, 1),
            "ms_per_token": round(wall * 1e3 / n, 4), "layer_path": "per_phase (graph replay)"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=64)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--roofline-kernel", default=None, choices=sorted(KERNEL_BYTES),
                    help="kernel timed in situ for the roofline (default: layers on the persistent path, else gate_up)")
    ap.add_argument("--layer-path", type=int, default=1, choices=[0, 1],
                    help="0: one kernel per phase; 1: the persistent decode kernel (default)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-budget", type=float, default=25.0)
    ap.add_argument("--seed", type=int, default=1)
    ap.add_argument("--prefill-tokens", type=int, default=512,
                    help="config 5 leg: batched prefill of this many seeded token ids (0: skip)")
    ap.add_argument("--prefill-decode", type=int, default=128,
                    help="greedy tokens generated after the prefill (the first comes from the prefill's head)")
    ap.add_argument("--prefill-only", action="store_true",
                    help="run only the config 5 prefill leg (profiling aid; prints that leg's JSON)")
    ap.add_argument("--real-mix", action="store_true",
                    help="with --prefill-only: the model in the real checkpoint's per-layer formats (layer l %% 4: "
                         "Q5_K or IQ4_XS attention V/O, IQ2_S or IQ2_XS gate/up, IQ3_XXS, IQ4_XS or IQ3_S down)")
    ap.add_argument("--long-steps", type=int, default=128,
                    help="long-context leg: greedy tokens at positions 4096-N..4095 over a seeded KV (0: skip)")
    ap.add_argument("--mix-steps", type=int, default=32,
                    help="real-mix decode leg: greedy tokens on the real checkpoint's per-layer formats (0: skip)")
    ap.add_argument("--attention-chunks", type=int, default=0, metavar="N",
                    help="persistent decode: attend by kv head and chunk from N = pos + 1 positions on "
                         "(0: the library default; 1: always; 4097: never)")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only copy a MIB-sized device buffer (HBM counter calibration) and exit")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: this build has no multi-GPU path (asked for --gpus {args.gpus}); "
              "run with --gpus 1", file=sys.stderr)
        sys.exit(1)
    if args.copy_calibration:
        copy_calibration(args.copy_calibration)
        return
    if args.real_mix and not args.prefill_only:
        sys.exit("--real-mix measures the prefill leg only (use it with --prefill-only)")
    import qxg

    prompt_len = 8
    if prompt_len + max(args.steps, args.warmup) > 4096:
        sys.exit("steps exceed the 4096-token context")
    ctx_tokens = prompt_len + max(args.steps, args.warmup) + 1
    prompt = np.random.default_rng(args.seed).integers(0, VOCAB, size=prompt_len).astype(np.uint32)

    t0 = time.perf_counter()
    model = qxg.MemModel(LAYERS, VOCAB, EXPERTS, True, True, seed=args.seed, mix=1 if args.real_mix else 0)
    log(f"generated the {LAYERS}-layer model in memory in {time.perf_counter() - t0:.1f} s ({model.path})")
    ctx = qxg.Context(0)
    ctx.set_layer_path(args.layer_path)
    if args.attention_chunks:
        ctx.set_attention_chunks(args.attention_chunks)
    if args.roofline_kernel is None:
        args.roofline_kernel = "layers" if args.layer_path else "gate_up"
    t0 = time.perf_counter()
    info = ctx.load(model.path, verify=False)
    log(f"uploaded {info.tensors} tensors, {info.tensor_bytes / 1e9:.3f} GB in {time.perf_counter() - t0:.1f} s")

    if args.prefill_only:
        leg = prefill_leg(ctx, args)
        if args.real_mix:
            leg["quant_mix"] = ("real checkpoint per-layer formats: Q5_K/IQ4_XS attn V/O, IQ2_S/IQ2_XS gate/up, "
                                "IQ3_XXS/IQ4_XS/IQ3_S down (layer l % 4)")
        ctx.close()
        model.close()
        print(json.dumps({"prefill": leg}), flush=True)
        return

    def prefill():
        ctx.kv_create(LAYERS, ctx_tokens)
        first, _ = ctx.generate(prompt, 1, 0)          # 8 steps, last one yields the first token
        return int(first[0])

    # warmup
    first = prefill()
    ctx.generate([first], max(args.warmup, 1), prompt_len)
    log(f"warmup done ({args.warmup} tokens)")
    # timed: K decode tokens at positions 8 .. 8+K-1, in-situ events around the roofline kernel
    first = prefill()
    which = qxg.KERNELS[args.roofline_kernel]
    ctx.profile_kernel(which)
    t0 = time.perf_counter()
    toks, dev_ms = ctx.generate([first], args.steps, prompt_len)
    wall = time.perf_counter() - t0
    launches, kern_ms = ctx.profile_result()
    ctx.profile_kernel(-1)
    log(f"timed {args.steps} tokens: device {dev_ms:.2f} ms, wall {wall * 1e3:.2f} ms; "
        f"{args.roofline_kernel}: {launches} launches, {kern_ms:.2f} ms")
    # same region without event pairs, for the headline number
    first = prefill()
    t0 = time.perf_counter()
    toks2, dev_ms2 = ctx.generate([first], args.steps, prompt_len)
    wall2 = time.perf_counter() - t0
    assert list(toks2) == list(toks), "greedy sequence changed between identical runs"
    tok_s = args.steps / wall2
    avg_kernel_s = kern_ms / 1e3 / max(launches, 1)
    kb = KERNEL_BYTES[args.roofline_kernel]
    if args.roofline_kernel == "layers":   # every step of the call, plus the INT8 KV rows read at positions 8..8+K-1
        kb = TOKEN_BYTES * args.steps + kv_bytes(prompt_len, args.steps)
    achieved = kb / avg_kernel_s / 1e9
    ratio, ratio_src = measured_traffic_ratio(args.roofline_kernel)
    token_bytes = TOKEN_BYTES + kv_bytes(prompt_len, args.steps) / args.steps
    out = {
        "metric": "batch-1 decode tok/s (48 layers + Q6_K head)",
        "value": round(tok_s, 3),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall2 * 1e3 / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32 result; activations as 22-bit block-fixed-point int8 digit planes x exact integer weight "
                 "codes (int32 v_dot4 sums), f32/f64 combination and softmax",
        "data": "synthetic: seeded random-init QXF1 (generator qxgen.c), seeded 8-token prompt",
        "config": {"workload": "config4: Qwen3-30B-A3B-shaped decode, 48 layers + Q6_K head 2048x151936, "
                               "greedy tokens after an 8-token prompt, INT8 KV",
                   "layers": LAYERS, "vocab": VOCAB, "experts": EXPERTS, "top_k": 8, "prompt_tokens": prompt_len,
                   "quant_mix": "IQ4_XS attn, IQ2_XS gate/up, IQ3_XXS down, Q6_K head, Q4_K embedding",
                   "kv": "int8", "parallelism": "none (1 GPU)",
                   "layer_path": "persistent" if args.layer_path else "per_phase"},
        "roofline": {"bound": "hbm", "kernel": args.roofline_kernel, "achieved": round(achieved, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": round(ratio * kb) if ratio else None, "traffic_ratio": ratio,
                     "traffic_note": (f"HBM bytes of this launch = its algorithmic bytes x the FETCH_SIZE+WRITE_SIZE "
                                      f"ratio measured in {ratio_src}") if ratio else None,
                     "bytes_per_launch": kb, "avg_launch_us": round(avg_kernel_s * 1e6, 3), "launches": launches},
        "token_roofline": {"algorithmic_bytes_per_token": int(token_bytes),
                           "achieved_GBs": round(token_bytes * tok_s / 1e9, 1),
                           "frac": round(token_bytes * tok_s / 1e9 / HBM_PEAK_GBS, 4),
                           "device_ms_per_token": round(dev_ms2 / args.steps, 4)},
        "first_tokens": [int(t) for t in toks[:8]],
    }
    prompt_kv = None
    if not args.no_cpu_baseline:   # the prompt's KV rows as the GPU writes them, for the CPU baseline
        first = prefill()
        prompt_kv = [ctx.kv_read(l, 0, prompt_len) for l in range(LAYERS)]
    if args.prefill_tokens:
        out["prefill"] = prefill_leg(ctx, args)
    if args.long_steps and args.layer_path:
        out["long_context"] = long_context_leg(ctx, args)
    ctx.close()
    if args.mix_steps:
        out["real_mix_decode"] = mix_decode_leg(args)
    if not args.no_cpu_baseline:
        log("cpu baseline (oracle, 1 thread) ...")
        out["cpu_baseline"] = cpu_baseline(model.path, prompt_kv, first, prompt_len, args.cpu_budget)
    else:
        out["cpu_baseline"] = None
    model.close()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
