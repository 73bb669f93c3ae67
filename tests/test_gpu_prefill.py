"""Batched prefill (config 5's path) against the oracle: same-input replay of one layer
over many tokens (each token's attention and MoE recomputed by the oracle on the GPU's
own inputs), the full prefill against the oracle's token-by-token steps, and chunked
prefill against the GPU's own decode path.  Runs through the C ABI (include/qxg.h)."""
import numpy as np
import pytest

import qxo
import qxg
from helpers import REL_L2, rel_l2, seeded_kv, topk_consistent

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    c = qxg.Context(0)
    yield c
    c.close()


@pytest.mark.parametrize("experts,n,p0", [(16, 48, 0), (128, 40, 100), (8, 70, 3)])
def test_prefill_layer_replay(ctx, tmp_path, experts, n, p0):
    """n tokens through one layer at positions p0..p0+n-1 (earlier positions hold seeded
    INT8 rows).  experts=16/8 put 24..70 tokens on an expert (several row tiles, ragged
    last tile); experts=128 leaves most experts empty."""
    p = tmp_path / f"l{experts}.qxf"
    qxg.generate_model(p, layers=1, vocab=1024, experts=experts, seed=60 + experts)
    ctx.load(p)
    ctx.kv_create(1, 256)
    okv = qxo.KV(1, 256)
    if p0:
        k, v, ks, vs = seeded_kv(70, p0)
        ctx.kv_write(0, 0, k, v, ks, vs)
        okv.k[0, :p0], okv.v[0, :p0], okv.ks[0, :p0], okv.vs[0, :p0] = k, v, ks, vs
    x = np.random.default_rng(80 + n).standard_normal((n, 2048)).astype(np.float32)
    x[3] *= 1e-3   # rows of very different magnitude share the GEMM tiles
    x[5] *= 300.0
    fi, moe, out = ctx.prefill_layer(0, p0, x)
    om = qxo.Model(p)
    fi_ref = np.zeros_like(x)
    for t in range(n):
        a, _, _ = qxo.attention_layer(om, 0, p0 + t, okv, x[t])
        fi_ref[t] = x[t] + a
    assert rel_l2(fi, fi_ref) <= REL_L2, rel_l2(fi, fi_ref)
    for t in (0, n // 2, n - 1):
        assert rel_l2(fi[t], fi_ref[t]) <= REL_L2, (t, rel_l2(fi[t], fi_ref[t]))
    out_ref = np.zeros_like(x)
    moe_ref = np.zeros_like(x)
    for t in range(n):   # same-input replay of the MoE half on the GPU's ffn input
        y, m, _, _ = om.moe_layer(0, fi[t])
        out_ref[t], moe_ref[t] = y, m
    om.close()
    assert rel_l2(moe, moe_ref) <= REL_L2, rel_l2(moe, moe_ref)
    assert rel_l2(out, out_ref) <= REL_L2, rel_l2(out, out_ref)
    for t in range(n):
        assert rel_l2(moe[t], moe_ref[t]) <= REL_L2, (t, rel_l2(moe[t], moe_ref[t]))
    gk, gv, gks, gvs = ctx.kv_read(0, p0, n)
    assert np.abs(gk.astype(int) - okv.k[0, p0:p0 + n].astype(int)).max() <= 1
    assert np.abs(gv.astype(int) - okv.v[0, p0:p0 + n].astype(int)).max() <= 1
    assert np.abs(gks / okv.ks[0, p0:p0 + n] - 1).max() < 1e-5
    assert np.abs(gvs / okv.vs[0, p0:p0 + n] - 1).max() < 1e-5


def test_prefill_matches_token_steps(ctx, tmp_path):
    """Embedding + 2 layers over a 37-token prompt, head on the last token, against the
    oracle's token-by-token steps; then greedy decode continues from the prefilled cache
    and gives the tokens of the all-decode path."""
    p = tmp_path / "two.qxf"
    qxg.generate_model(p, layers=2, vocab=4096, experts=32, seed=44)
    ctx.load(p)
    prompt = np.random.default_rng(5).integers(0, 4096, size=37).astype(np.uint32)
    n = len(prompt)
    ctx.kv_create(2, 64)
    res, lg, ids, tl, ms = ctx.prefill(prompt, 0, True, 8, want_residual=True, want_logits=True)
    assert ms > 0
    om = qxo.Model(p)
    okv = qxo.KV(2, 64)
    ores = np.zeros((n, 2048), np.float32)
    for t in range(n):
        last = t == n - 1
        r, _, olg, oids, otl = qxo.decode_token(om, int(prompt[t]), t, okv, 2, last, 4096, 8)
        ores[t] = r
    om.close()
    assert rel_l2(res, ores) <= 1e-4, rel_l2(res, ores)
    assert rel_l2(lg, olg) <= 1e-4, rel_l2(lg, olg)
    ok, why = topk_consistent(ids, oids, olg)
    assert ok, why
    gk, gv, gks, _ = ctx.kv_read(1, 0, n)
    assert np.abs(gks / okv.ks[1, :n] - 1).max() < 1e-3
    # prefill + decode == decode only (tokens of the greedy continuation)
    gen_pf, _ = ctx.generate([int(ids[0])], 5, pos0=n)
    ctx.kv_create(2, 64)
    gen_dec, _ = ctx.generate(prompt, 6)
    assert [int(ids[0])] + list(gen_pf) == list(gen_dec)


def test_prefill_chunks_vs_decode_path(ctx, tmp_path):
    """600 tokens: two chunks (512 + 88) whose second attends over the first; the last
    token's residual and logits agree with the decode path's on the same prompt."""
    p = tmp_path / "chunk.qxf"
    qxg.generate_model(p, layers=2, vocab=2048, experts=16, seed=91)
    ctx.load(p)
    prompt = np.random.default_rng(9).integers(0, 2048, size=600).astype(np.uint32)
    ctx.kv_create(2, 640)
    res, lg, ids, _, _ = ctx.prefill(prompt, 0, True, 8, want_residual=True, want_logits=True)
    ctx.kv_create(2, 640)
    ctx.generate(prompt[:599], 1)
    dres, _, dlg, dids, _ = ctx.decode_token(int(prompt[599]), 599, True, 8, want_logits=True)
    assert rel_l2(res[599], dres) <= 1e-4, rel_l2(res[599], dres)
    assert rel_l2(lg, dlg) <= 1e-4, rel_l2(lg, dlg)
    ok, why = topk_consistent(ids, dids, dlg)
    assert ok, why
