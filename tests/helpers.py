"""Shared checks for the parity tests (tolerances come from the hot-path contract:
bit-exact dequant; F32 outputs within 1e-5 relative L2; top-k identical except
where the oracle's own margin is below 1e-4)."""
import numpy as np

REL_L2 = 1e-5
TIE_MARGIN = 1e-4


def rel_l2(a, ref):
    a = np.asarray(a, np.float64)
    ref = np.asarray(ref, np.float64)
    den = np.linalg.norm(ref)
    return float(np.linalg.norm(a - ref) / (den if den > 0 else 1.0))


def topk_consistent(gpu_ids, ref_ids, ref_logits_all, margin=TIE_MARGIN):
    """GPU top-k must equal the oracle's; a mismatch at rank r is allowed only when
    the oracle's logits of the two ids involved differ by less than `margin`."""
    gpu_ids = [int(i) for i in gpu_ids]
    ref_ids = [int(i) for i in ref_ids]
    for r, (g, o) in enumerate(zip(gpu_ids, ref_ids)):
        if g == o:
            continue
        if abs(float(ref_logits_all[g]) - float(ref_logits_all[o])) >= margin:
            return False, f"rank {r}: gpu {g} ({ref_logits_all[g]}) vs oracle {o} ({ref_logits_all[o]})"
    return True, ""


def seeded_normal(seed, n=2048):
    return np.random.default_rng(seed).standard_normal(n).astype(np.float32)


def seeded_kv(seed, count):
    """Seeded INT8 KV rows and positive scales, handed identically to both sides."""
    rng = np.random.default_rng(seed)
    k = rng.integers(-127, 128, size=(count, 512), dtype=np.int8)
    v = rng.integers(-127, 128, size=(count, 512), dtype=np.int8)
    ks = (rng.uniform(0.5, 2.0, size=count) / 127.0).astype(np.float32)
    vs = (rng.uniform(0.5, 2.0, size=count) / 127.0).astype(np.float32)
    return k, v, ks, vs
