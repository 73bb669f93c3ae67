"""The real checkpoint's per-layer quant mix on the HIP decode path: layer l % 4 of the
mixed generator model uses (attention V/O, gate/up, down) =
0: IQ4_XS, IQ2_XS, IQ3_XXS;  1: Q5_K, IQ2_S, IQ4_XS;  2: IQ4_XS, IQ2_XS, IQ3_S;
3: Q5_K, IQ2_S, IQ3_S.  Each layer's attention and MoE halves, and a greedy decode
through all four layers, are compared with the oracle on the same seeded inputs."""
import numpy as np
import pytest

import qxo
import qxg
from helpers import REL_L2, rel_l2, seeded_kv, seeded_normal, topk_consistent

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    """The persistent decode is asked for (the default); a mixed model runs one kernel per
    phase regardless."""
    c = qxg.Context(0)
    c.set_layer_path(1)
    yield c
    c.close()


@pytest.fixture(scope="module")
def mix_model(tmp_path_factory):
    p = tmp_path_factory.mktemp("mix") / "mix.qxf"
    qxg.generate_model(p, layers=4, vocab=4096, experts=32, embedding=True, head=True, seed=66, mix=1)
    return p


@pytest.mark.parametrize("layer", [0, 1, 2, 3])
def test_mix_attention_layer(ctx, mix_model, layer):
    ctx.load(mix_model)
    pos = 77
    ctx.kv_create(4, 256)
    okv = qxo.KV(4, 256)
    k, v, ks, vs = seeded_kv(40 + layer, pos)
    ctx.kv_write(layer, 0, k, v, ks, vs)
    okv.k[layer, :pos], okv.v[layer, :pos], okv.ks[layer, :pos], okv.vs[layer, :pos] = k, v, ks, vs
    x = seeded_normal(50 + layer)
    a, kqv, vcur = ctx.attention_layer(layer, pos, x)
    om = qxo.Model(mix_model)
    oa, okqv, ovcur = qxo.attention_layer(om, layer, pos, okv, x)
    om.close()
    assert rel_l2(vcur, ovcur) <= REL_L2, rel_l2(vcur, ovcur)
    assert rel_l2(kqv, okqv) <= REL_L2, rel_l2(kqv, okqv)
    assert rel_l2(a, oa) <= REL_L2, rel_l2(a, oa)


@pytest.mark.parametrize("layer", [0, 1, 2, 3])
def test_mix_moe_layer(ctx, mix_model, layer):
    ctx.load(mix_model)
    om = qxo.Model(mix_model)
    for seed in (60, 61):
        x = seeded_normal(seed + 10 * layer)
        y, moe, ids, w = ctx.moe_layer(layer, x)
        oy, omoe, oids, ow = om.moe_layer(layer, x)
        assert list(ids) == list(oids)
        assert np.allclose(w, ow, rtol=1e-9, atol=0)
        assert rel_l2(moe, omoe) <= REL_L2, rel_l2(moe, omoe)
        assert rel_l2(y, oy) <= REL_L2
    om.close()


def test_mix_decode_greedy(ctx, mix_model):
    """Embedding + 4 mixed layers + head, 5 greedy steps; then the replayed device loop."""
    ctx.load(mix_model)
    ctx.kv_create(4, 16)
    om = qxo.Model(mix_model)
    okv = qxo.KV(4, 16)
    tok_g = tok_o = 29
    toks = []
    for s in range(5):
        res, lay, lg, ids, tl = ctx.decode_token(tok_g, s, True, 4, want_layers=True, want_logits=True)
        ores, olay, olg, oids, otl = qxo.decode_token(om, tok_o, s, okv, 4, True, 4096, 4)
        assert rel_l2(lay, olay) <= 1e-4, (s, rel_l2(lay, olay))
        assert rel_l2(lg, olg) <= 1e-4
        ok, why = topk_consistent(ids, oids, olg)
        assert ok, why
        tok_g, tok_o = int(ids[0]), int(oids[0])
        toks.append(tok_g)
    om.close()
    for rep in range(2):
        ctx.kv_create(4, 16)
        gen, _ = ctx.generate([29], 5)
        assert list(gen) == toks, rep


@pytest.mark.parametrize("layer", [0, 1, 2, 3])
def test_mix_prefill_layer_replay(ctx, mix_model, layer):
    """The batched prefill GEMMs on every per-layer format combination: Q5_K V and O (the
    dmin term through a pass over an all-ones operand), IQ2_S gate/up, IQ4_XS or IQ3_S down.
    40 tokens through the layer at positions 20..59 (earlier positions hold seeded INT8
    rows), rows 1000x apart in magnitude; each token's attention recomputed by the oracle
    over the GPU's own cache rows (its own row included), the MoE half replayed by the
    oracle on the GPU's own ffn input (1e-5 per row)."""
    ctx.load(mix_model)
    n, p0 = 40, 20
    ctx.kv_create(4, 128)
    okv = qxo.KV(4, 128)
    k, v, ks, vs = seeded_kv(90 + layer, p0)
    ctx.kv_write(layer, 0, k, v, ks, vs)
    okv.k[layer, :p0], okv.v[layer, :p0], okv.ks[layer, :p0], okv.vs[layer, :p0] = k, v, ks, vs
    x = np.random.default_rng(300 + layer).standard_normal((n, 2048)).astype(np.float32)
    x[3] *= 1e-3
    x[5] *= 300.0
    fi, moe, out = ctx.prefill_layer(layer, p0, x)
    gk, gv, gks, gvs = ctx.kv_read(layer, p0, n)
    okv.k[layer, p0:p0 + n], okv.v[layer, p0:p0 + n], okv.ks[layer, p0:p0 + n], okv.vs[layer, p0:p0 + n] = gk, gv, gks, gvs
    om = qxo.Model(mix_model)
    for t in range(n):
        # token t's attention by the oracle over the GPU's own cache rows, its own included;
        # the oracle's row for the token: codes within 1 (inputs within 1e-7), scales 1e-5
        a, _, _, rk, rv, (sk, sv) = qxo.attention_layer_given_row(om, layer, p0 + t, okv, x[t])
        assert rel_l2(fi[t], x[t] + a) <= REL_L2, (layer, t, rel_l2(fi[t], x[t] + a))
        assert np.abs(gk[t].astype(int) - rk.astype(int)).max() <= 1, (layer, t)
        assert np.abs(gv[t].astype(int) - rv.astype(int)).max() <= 1, (layer, t)
        assert abs(gks[t] / sk - 1) < 1e-5 and abs(gvs[t] / sv - 1) < 1e-5, (layer, t)
    for t in range(n):
        y, m, _, _ = om.moe_layer(layer, fi[t])
        assert rel_l2(moe[t], m) <= REL_L2, (layer, t, rel_l2(moe[t], m))
        assert rel_l2(out[t], y) <= REL_L2, (layer, t)
    om.close()


def test_mix_prefill_vs_token_steps(ctx, mix_model):
    """A 29-token prompt batched through the four mixed layers and the head, against the
    oracle's token-by-token steps (residuals and logits 1e-4, top-k by the margin rule)."""
    ctx.load(mix_model)
    prompt = np.random.default_rng(12).integers(0, 4096, size=29).astype(np.uint32)
    n = len(prompt)
    ctx.kv_create(4, 64)
    res, lg, ids, tl, _ = ctx.prefill(prompt, 0, True, 8, want_residual=True, want_logits=True)
    om = qxo.Model(mix_model)
    okv = qxo.KV(4, 64)
    ores = np.zeros((n, 2048), np.float32)
    for t in range(n):
        r, _, olg, oids, _ = qxo.decode_token(om, int(prompt[t]), t, okv, 4, t == n - 1, 4096, 8)
        ores[t] = r
    om.close()
    assert rel_l2(res, ores) <= 1e-4, rel_l2(res, ores)
    assert rel_l2(lg, olg) <= 1e-4, rel_l2(lg, olg)
    ok, why = topk_consistent(ids, oids, olg)
    assert ok, why


def test_mix_prefill_q8k_token_steps(mix_model):
    """In the q8_k_compat mode the prompt still runs as device token steps (the batched GEMMs
    compute in the f32 scheme), bit-identical to stepping it with decode_token."""
    c = qxg.Context(0)
    try:
        c.set_activation("q8_k_compat")
        c.load(mix_model)
        prompt = np.array([29, 4000, 7, 123, 2048], np.uint32)
        c.kv_create(4, 16)
        res, lg, ids, tl, _ = c.prefill(prompt, 0, True, 4, want_residual=True, want_logits=True)
        c.kv_create(4, 16)
        for s, tok in enumerate(prompt):
            r, _, l2, i2, _ = c.decode_token(int(tok), s, s == len(prompt) - 1, 4, want_logits=True)
            assert np.array_equal(res[s], r), s
        assert np.array_equal(lg, l2) and list(ids) == list(i2)
    finally:
        c.close()
