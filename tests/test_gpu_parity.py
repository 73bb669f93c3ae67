"""HIP path vs the oracle on identical seeded inputs (configs 1-3 of the hot path,
plus a small full-token decode).  Runs through the C ABI (include/qxg.h)."""
import numpy as np
import pytest

import qxo
import qxg
from helpers import REL_L2, rel_l2, seeded_kv, seeded_normal, topk_consistent

pytestmark = pytest.mark.gpu

BLOCK_BYTES = {12: 144, 13: 176, 14: 210, 17: 74, 18: 98, 21: 110, 22: 82, 23: 136}
D_OFFSET = {12: 0, 13: 0, 14: 208, 17: 0, 18: 0, 21: 0, 22: 0, 23: 0}


@pytest.fixture(scope="module")
def ctx():
    """The replay seams (dequant, head, MoE, attention) run the per-phase kernels on either
    layer path."""
    c = qxg.Context(0)
    yield c
    c.close()


@pytest.fixture(scope="module", params=[0, 1], ids=["per_phase", "persistent"])
def dctx(request):
    """Decode steps and the greedy loop on both layer paths: one kernel per phase, and the
    persistent decode (every step of a call in one launch)."""
    c = qxg.Context(0)
    c.set_layer_path(request.param)
    c.layer_path = request.param
    yield c
    c.close()


@pytest.mark.parametrize("ggml_type", [12, 13, 14, 17, 18, 21, 22, 23])
def test_dequant_bit_exact(ctx, ggml_type):
    """Random blocks plus every fp16 value of d (including exponent 31 -> 65504)."""
    bb = BLOCK_BYTES[ggml_type]
    rng = np.random.default_rng(100 + ggml_type)
    rand = rng.integers(0, 256, size=(2048, bb), dtype=np.uint8)
    sweep = np.repeat(rng.integers(0, 256, size=(1, bb), dtype=np.uint8), 65536, axis=0)
    d = np.arange(65536, dtype=np.uint16)
    off = D_OFFSET[ggml_type]
    sweep[:, off] = (d & 255).astype(np.uint8)
    sweep[:, off + 1] = (d >> 8).astype(np.uint8)
    blocks = np.concatenate([rand, sweep])
    gpu = ctx.dequant(ggml_type, blocks, len(blocks)).reshape(-1, 256)
    ref = np.stack([qxo.decode_block(ggml_type, b) for b in blocks])
    assert gpu.view(np.uint32).tobytes() == ref.view(np.uint32).tobytes()


@pytest.fixture(scope="module")
def head_model(tmp_path_factory):
    p = tmp_path_factory.mktemp("head") / "head.qxf"
    qxg.generate_model(p, layers=0, vocab=151936, embedding=False, head=True, seed=11)
    return p


def test_final_head_config1(ctx, head_model):
    """Config 1: Q6_K head 2048 -> 151936 on x ~ N(0,1)."""
    ctx.load(head_model)
    x = seeded_normal(1)
    nrm, lg, ids, tl = ctx.final_head(x, top_n=8)
    om = qxo.Model(head_model)
    onrm, olg, oids, otl = om.final_head(x, 151936, top_n=8)
    om.close()
    assert rel_l2(nrm, onrm) <= 1e-7
    assert rel_l2(lg, olg) <= REL_L2, rel_l2(lg, olg)
    ok, why = topk_consistent(ids, oids, olg)
    assert ok, why


@pytest.fixture(scope="module")
def layer_model(tmp_path_factory):
    p = tmp_path_factory.mktemp("layer") / "layer.qxf"
    qxg.generate_model(p, layers=1, vocab=1024, experts=128, embedding=True, head=True, seed=22)
    return p


def test_moe_block_config2(ctx, layer_model):
    """Config 2: one MoE FFN block (128 experts, top-8) on x ~ N(0,1)."""
    ctx.load(layer_model)
    om = qxo.Model(layer_model)
    for seed in (2, 3, 4):
        x = seeded_normal(seed)
        y, moe, ids, w = ctx.moe_layer(0, x)
        oy, omoe, oids, ow = om.moe_layer(0, x)
        assert list(ids) == list(oids)
        assert np.allclose(w, ow, rtol=1e-9, atol=0)
        assert rel_l2(moe, omoe) <= REL_L2, rel_l2(moe, omoe)
        assert rel_l2(y, oy) <= REL_L2
    om.close()


def _tensor_span(path, name):
    """(offset, size) of a tensor in a QXF1 file (header and 208-byte directory entries)."""
    raw = np.fromfile(path, np.uint8)
    n = int(raw[16:20].view(np.uint32)[0])
    d0 = int(raw[24:32].view(np.uint64)[0])
    for i in range(n):
        e = raw[d0 + 208 * i: d0 + 208 * (i + 1)]
        if bytes(e[:96]).split(b"\0")[0].decode() == name:
            return int(e[144:152].view(np.uint64)[0]), int(e[152:160].view(np.uint64)[0])
    raise KeyError(name)


def test_moe_router_ties(ctx, tmp_path):
    """Router rows copied so that experts tie exactly (equal logits: the lower index is
    picked first) or nearly (one weight 1 ulp apart: equal f32 keys, different doubles)."""
    p = tmp_path / "ties.qxf"
    qxg.generate_model(p, layers=1, vocab=1024, experts=128, embedding=True, head=True, seed=22)
    x = seeded_normal(2)
    om = qxo.Model(p)
    _, _, oids, _ = om.moe_layer(0, x)
    om.close()
    a, b = int(oids[0]), int(oids[2])
    off, size = _tensor_span(p, "blk.0.ffn_gate_inp.weight")
    mm = np.memmap(p, np.uint8, mode="r+", offset=off, shape=(size,))
    router = mm.view(np.float32).reshape(128, 2048)
    for dst in sorted({0, 127, (a + 1) % 128, (a + 40) % 128} - {a, b}):
        router[dst] = router[a]                       # exact ties with the top expert
    near = (b + 64) % 128
    if near not in (a, b, 0, 127, (a + 1) % 128, (a + 40) % 128):
        router[near] = router[b]
        router[near, 7] = np.nextafter(router[b, 7], np.float32(np.inf))   # a near tie
    mm.flush()
    del router, mm
    ctx.load(p, verify=False)
    om = qxo.Model(p)
    for seed in (2, 5):
        xs = seeded_normal(seed)
        y, moe, ids, w = ctx.moe_layer(0, xs)
        oy, omoe, oids2, ow = om.moe_layer(0, xs)
        assert list(ids) == list(oids2), (seed, list(ids), list(oids2))
        assert np.allclose(w, ow, rtol=1e-9, atol=0)
        assert rel_l2(moe, omoe) <= REL_L2
    om.close()


@pytest.mark.parametrize("pos,ctx_tokens", [(0, 2048), (5, 2048), (127, 2048), (128, 2048), (130, 2048),
                                            (2047, 2048), (4095, 4096)])
def test_attention_block_config3(ctx, layer_model, pos, ctx_tokens):
    """Config 3: attention at `pos` with positions 0..pos-1 prefilled by seeded INT8 rows
    (one 128-position split up to 127; from 128 on several splits and their merge, up to
    the 32 of the maximum context)."""
    ctx.load(layer_model)
    ctx.kv_create(1, ctx_tokens)
    okv = qxo.KV(1, ctx_tokens)
    if pos:
        k, v, ks, vs = seeded_kv(33, pos)
        ctx.kv_write(0, 0, k, v, ks, vs)
        okv.k[0, :pos], okv.v[0, :pos], okv.ks[0, :pos], okv.vs[0, :pos] = k, v, ks, vs
    x = seeded_normal(7)
    a, kqv, vcur = ctx.attention_layer(0, pos, x)
    om = qxo.Model(layer_model)
    oa, okqv, ovcur = qxo.attention_layer(om, 0, pos, okv, x)
    om.close()
    assert rel_l2(vcur, ovcur) <= REL_L2
    assert rel_l2(kqv, okqv) <= REL_L2, rel_l2(kqv, okqv)
    assert rel_l2(a, oa) <= REL_L2, rel_l2(a, oa)
    gk, gv, gks, gvs = ctx.kv_read(0, pos, 1)
    assert np.abs(gk[0].astype(int) - okv.k[0, pos].astype(int)).max() <= 1
    assert np.abs(gv[0].astype(int) - okv.v[0, pos].astype(int)).max() <= 1
    assert abs(gks[0] / okv.ks[0, pos] - 1) < 1e-5 and abs(gvs[0] / okv.vs[0, pos] - 1) < 1e-5


def test_generate_across_attention_splits(dctx, tmp_path):
    """The recorded step graph launches the attention splits its positions need (two for
    positions 118..138) while eager steps launch the whole cache's (four at 512): the
    context depends only on the position, so both give the same tokens, and the graph
    is recorded again when a later call needs more splits (positions 250..260)."""
    p = tmp_path / "splits.qxf"
    qxg.generate_model(p, layers=2, vocab=4096, experts=32, seed=45)
    dctx.load(p)
    dctx.kv_create(2, 512)
    rng = np.random.default_rng(12)
    pre = rng.integers(0, 4096, size=118).astype(np.uint32)
    dctx.prefill(pre, 0, False, 1)
    toks, t = [], 17
    for s in range(118, 139):
        _, _, _, ids, _ = dctx.decode_token(t, s, True, 1)
        t = int(ids[0])
        toks.append(t)
    for rep in range(2):
        dctx.kv_create(2, 512)
        dctx.prefill(pre, 0, False, 1)
        gen, _ = dctx.generate([17], 21, pos0=118)
        assert list(gen) == toks, rep
    pre2 = rng.integers(0, 4096, size=250).astype(np.uint32)
    dctx.kv_create(2, 512)
    dctx.prefill(pre2, 0, False, 1)
    gen2, _ = dctx.generate([5], 11, pos0=250)
    dctx.kv_create(2, 512)
    dctx.prefill(pre2, 0, False, 1)
    toks2, t = [], 5
    for s in range(250, 261):
        _, _, _, ids, _ = dctx.decode_token(t, s, True, 1)
        t = int(ids[0])
        toks2.append(t)
    assert list(gen2) == toks2


def test_decode_two_layers_greedy(dctx, tmp_path):
    """Embedding + 2 layers + head, 5 greedy steps; per-step residual and tokens."""
    p = tmp_path / "two.qxf"
    qxg.generate_model(p, layers=2, vocab=4096, experts=32, seed=44)
    dctx.load(p)
    dctx.kv_create(2, 16)
    om = qxo.Model(p)
    okv = qxo.KV(2, 16)
    tok_g = tok_o = 17
    for s in range(5):
        res, lay, lg, ids, tl = dctx.decode_token(tok_g, s, True, 4, want_layers=True, want_logits=True)
        ores, olay, olg, oids, otl = qxo.decode_token(om, tok_o, s, okv, 2, True, 4096, 4)
        assert rel_l2(lay, olay) <= 1e-4, (s, rel_l2(lay, olay))
        assert rel_l2(lg, olg) <= 1e-4
        ok, why = topk_consistent(ids, oids, olg)
        assert ok, why
        tok_g, tok_o = int(ids[0]), int(oids[0])
    om.close()
    # the device-resident greedy loop (one recorded step replayed per token) gives the
    # same tokens as the eager step-by-step path, on every replay, interleaved with eager work
    dctx.kv_create(2, 16)
    toks = []
    t = 17
    for s in range(5):
        _, _, _, ids, _ = dctx.decode_token(t, s, True, 1)
        t = int(ids[0])
        toks.append(t)
    for rep in range(3):
        dctx.kv_create(2, 16)
        gen, ms = dctx.generate([17], 5)
        assert list(gen) == toks, rep
        dctx.kv_create(2, 16)
        dctx.decode_token(17, 0, True, 1)             # eager work between replays
        gen2, _ = dctx.generate([toks[0]], 4, pos0=1)  # continue from position 1
        assert list(gen2) == toks[1:], rep
    # eager (per-launch timed) loop agrees with the replayed one
    dctx.kv_create(2, 16)
    dctx.profile_kernel(qxg.KERNELS["layers" if dctx.layer_path else "gate_up"])
    gen3, _ = dctx.generate([17], 5)
    n, _ = dctx.profile_result()
    dctx.profile_kernel(-1)
    # one persistent launch for all steps, or one gate/up launch per layer and step
    assert list(gen3) == toks and n == (1 if dctx.layer_path else 5 * 2)


@pytest.mark.parametrize("p0", [126, 381, 1000])
def test_decode_long_context_vs_oracle(dctx, tmp_path, p0):
    """Greedy steps at positions p0.. over a seeded INT8 cache of p0 positions (both sides
    hold the same rows): the attention's 128-position blocks, their online-softmax merge
    and the split boundaries, against the oracle's single-pass softmax; per-layer outputs
    and logits at the multi-step bar (1e-4), tokens under the margin rule."""
    p = tmp_path / "long.qxf"
    qxg.generate_model(p, layers=2, vocab=4096, experts=32, seed=46)
    dctx.load(p)
    dctx.kv_create(2, p0 + 8)
    om = qxo.Model(p)
    okv = qxo.KV(2, p0 + 8)
    for layer in range(2):
        k, v, ks, vs = seeded_kv(300 + layer, p0)
        dctx.kv_write(layer, 0, k, v, ks, vs)
        okv.k[layer, :p0], okv.v[layer, :p0], okv.ks[layer, :p0], okv.vs[layer, :p0] = k, v, ks, vs
    tok_g = tok_o = 23
    for s in range(p0, p0 + 3):
        res, lay, lg, ids, tl = dctx.decode_token(tok_g, s, True, 4, want_layers=True, want_logits=True)
        ores, olay, olg, oids, otl = qxo.decode_token(om, tok_o, s, okv, 2, True, 4096, 4)
        assert rel_l2(lay, olay) <= 1e-4, (s, rel_l2(lay, olay))
        assert rel_l2(lg, olg) <= 1e-4, (s, rel_l2(lg, olg))
        ok, why = topk_consistent(ids, oids, olg)
        assert ok, why
        tok_g, tok_o = int(ids[0]), int(oids[0])
    om.close()


@pytest.mark.parametrize("layers", [1, 3])
def test_first_launch_of_fresh_context(tmp_path, layers):
    """The persistent decode's exchange buffers start in a state of their own (no layer has
    written them): the very first launch of a fresh context must read only what its own
    layers wrote.  With 3 layers, layer 2 reads x's slot 0 in the first step, which layer
    0 never writes.  Its residuals match the oracle's token steps and a later launch of the
    same steps, bit for bit."""
    p = tmp_path / f"fresh{layers}.qxf"
    qxg.generate_model(p, layers=layers, vocab=1024, experts=16, seed=57 + layers)
    prompt = [11, 500, 77]
    c = qxg.Context(0)
    try:
        c.set_layer_path(1)
        c.load(p)
        c.kv_create(layers, 16)
        first = [c.decode_token(t, s, s == 2, 4, want_layers=True) for s, t in enumerate(prompt)]
        c.kv_create(layers, 16)
        again = [c.decode_token(t, s, s == 2, 4, want_layers=True) for s, t in enumerate(prompt)]
    finally:
        c.close()
    for s in range(3):
        assert np.array_equal(first[s][0], again[s][0]) and np.array_equal(first[s][1], again[s][1]), s
    om = qxo.Model(p)
    okv = qxo.KV(layers, 16)
    for s, t in enumerate(prompt):
        r, lay, _, _, _ = qxo.decode_token(om, t, s, okv, layers, False, 1024, 4)
        assert rel_l2(first[s][0], r) <= 1e-4, (s, rel_l2(first[s][0], r))
        for l in range(layers):
            assert rel_l2(first[s][1][l], lay[l]) <= 1e-4, (s, l)
    om.close()
