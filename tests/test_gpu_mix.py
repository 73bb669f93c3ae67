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


def test_mix_prefill_token_steps(ctx, mix_model):
    """The batched GEMMs decode the benchmark mix only; this model prefills token by token
    through the decode kernels (as the reference prefills every prompt), so the result
    equals decoding the prompt step by step, bit for bit."""
    ctx.load(mix_model)
    prompt = np.array([29, 4000, 7, 123, 2048], np.uint32)
    ctx.kv_create(4, 16)
    res, lg, ids, tl, _ = ctx.prefill(prompt, 0, True, 4, want_residual=True, want_logits=True)
    ctx.kv_create(4, 16)
    for s, tok in enumerate(prompt):
        r, _, l2, i2, _ = ctx.decode_token(int(tok), s, s == len(prompt) - 1, 4, want_logits=True)
        assert np.array_equal(res[s], r), s
    assert np.array_equal(lg, l2) and list(ids) == list(i2)
    # the same-input layer seam takes the same route: each row's attention and MoE halves
    x = np.random.default_rng(3).standard_normal((3, 2048)).astype(np.float32)
    ctx.kv_create(4, 16)
    fi, moe, out = ctx.prefill_layer(1, 0, x)
    ctx.kv_create(4, 16)
    for t in range(3):
        a, _, _ = ctx.attention_layer(1, t, x[t])
        y, m, _, _ = ctx.moe_layer(1, x[t] + a)
        assert np.array_equal(fi[t], x[t] + a) and np.array_equal(moe[t], m) and np.array_equal(out[t], y), t
