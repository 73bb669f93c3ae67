"""The default decode path - the persistent kernel - against the oracle where its own
arithmetic differs from the per-phase kernels: attention over long caches (positions 2047
and 4095, the maximum context; the walk of the 32 q-head workgroups and the chunked stage A
with its merge), and outlier activations reaching its own digit planes (the Q/K/V input,
the context, x', h and the head), its router fold and its top-8.

Every decode step is replayed layer by layer on the device's own inputs (same-input
replay): the attention half (O projection of the context, before the residual add) against
the oracle's attention on the device's layer input and KV rows, the MoE half against the
oracle's MoE on the device's own ffn input, the layer output, the position's INT8 row, the
routed experts (reference router, 1e-4 margin rule) and the logits on the device's final
residual.  The halves are held to 1e-5 each: with outliers the residual stream is ~1e9
while a half can be ~1e3, so the layer output alone would hide an error in a half."""
import numpy as np
import pytest

import qxg
import qxo
from helpers import REL_L2, rel_l2, seeded_kv, topk_consistent
from test_gpu_atsize import router_logits, routing_consistent, row_close

pytestmark = pytest.mark.gpu

LAYERS, VOCAB, EXPERTS = 4, 8192, 128
WALK, CHUNKS = 4097, 1   # qxg_set_attention_chunks: never chunk, chunk every position


def say(msg):
    print(f"[persistent] {msg}", flush=True)


def replay_step(ctx, om, okv, pos, tok, head=True, moe_tol=REL_L2, att_tol=REL_L2):
    """One persistent decode step at `pos`, every layer replayed by the oracle on the
    device's own inputs; returns (worst relative L2 over the halves and layers, top-1).
    moe_tol bounds the MoE half and the layer output (1e-5 but for the stress pattern and
    q8_k_compat), att_tol the attention half (1e-5 but for q8_k_compat)."""
    res, lay, lg, ids, _ = ctx.decode_token(tok, pos, head, 8, want_layers=True, want_logits=head)
    att, moe = ctx.halves()
    r_ids, r_w = ctx.routing()
    for l in range(LAYERS):
        k, v, ks, vs = ctx.kv_read(l, 0, pos + 1)
        okv.k[l, :pos + 1], okv.v[l, :pos + 1], okv.ks[l, :pos + 1], okv.vs[l, :pos + 1] = k, v, ks, vs
    x0 = ctx.embed(tok)
    assert np.array_equal(x0, om.embed(tok))
    inputs = [x0] + [lay[l - 1] for l in range(1, LAYERS)]
    worst = 0.0
    for l in range(LAYERS):
        a_o, _, _, rk, rv, sc = qxo.attention_layer_given_row(om, l, pos, okv, inputs[l])
        ea = rel_l2(att[l], a_o)
        fi = (inputs[l] + att[l]).astype(np.float32)   # the device's own ffn input, bit for bit
        y_o, moe_o, o_ids, o_w = om.moe_layer(l, fi)
        em = rel_l2(moe[l], moe_o)
        ey = rel_l2(lay[l], y_o)
        worst = max(worst, ea, em, ey)
        assert ea <= att_tol, (pos, l, "attention", ea)
        assert em <= moe_tol, (pos, l, "moe", em)
        assert ey <= moe_tol, (pos, l, "layer", ey)
        assert np.array_equal(lay[l], (fi + moe[l]).astype(np.float32)), (pos, l)
        ok, why = routing_consistent(r_ids[l], o_ids, router_logits(om, l, fi))
        assert ok, (pos, l, why)
        if list(r_ids[l]) == list(o_ids):
            # the logits come through the f32-rounded router fold (~1e-7 of the logit's
            # magnitude): with the x1000 norm channels the logits reach ~1e2, and a weight's
            # relative error is the error of its logit difference, ~1e-6; held to the 1e-5 bar
            assert np.allclose(r_w[l], o_w, rtol=REL_L2, atol=1e-9), (pos, l, r_w[l], o_w)
        assert row_close(okv.k[l, pos], okv.v[l, pos], (okv.ks[l, pos], okv.vs[l, pos]), rk, rv, sc), (pos, l)
    if head:
        _, olg, oids, _ = om.final_head(res, VOCAB, 8)
        e = rel_l2(lg, olg)
        worst = max(worst, e)
        assert e <= REL_L2, (pos, "logits", e)
        ok, why = topk_consistent(ids, oids, olg)
        assert ok, (pos, why)
    return worst, int(ids[0]) if head else None


@pytest.fixture(scope="module")
def model():
    m = qxg.MemModel(LAYERS, VOCAB, EXPERTS, seed=81)
    om = qxo.Model(m.path)
    yield m, om
    om.close()
    m.close()


@pytest.fixture(scope="module", params=[1, 2], ids=["single", "stress"])
def outlier_model(request):
    m = qxg.MemModel(LAYERS, VOCAB, EXPERTS, seed=71, outliers=request.param)
    om = qxo.Model(m.path)
    yield m, om, request.param
    om.close()
    m.close()


@pytest.fixture(scope="module")
def sat_model():
    m = qxg.MemModel(LAYERS, VOCAB, EXPERTS, seed=91, outliers=3)
    om = qxo.Model(m.path)
    yield m, om
    om.close()
    m.close()


def open_ctx(path, chunks=None):
    """A persistent-path context; chunks None keeps the library's default threshold."""
    c = qxg.Context(0)
    c.set_layer_path(1)
    if chunks is not None:
        c.set_attention_chunks(chunks)
    c.load(path)
    return c


def seed_cache(ctx, okv, p0, seed):
    for layer in range(LAYERS):
        k, v, ks, vs = seeded_kv(seed + layer, p0)
        ctx.kv_write(layer, 0, k, v, ks, vs)
        okv.k[layer, :p0], okv.v[layer, :p0], okv.ks[layer, :p0], okv.vs[layer, :p0] = k, v, ks, vs


@pytest.mark.parametrize("p0", [0, 1, 31, 32, 33, 63, 64, 65, 127, 300, 1000, 2016, 4032])
def test_chunked_short_positions(model, p0):
    """The chunked stage A at every chunk count boundary it can meet (one chunk, the
    position alone in its chunk, a full last chunk; chunks of 32 positions up to 2048
    positions, of 64 beyond: the switch is met at 2047/2048 below), forced at short
    positions, and at 2016/2017 and 4032/4033, where the last chunk is full and then the
    position opens the 64th."""
    m, om = model
    c = open_ctx(m.path, CHUNKS)
    try:
        c.kv_create(LAYERS, p0 + 2)
        okv = qxo.KV(LAYERS, p0 + 2)
        seed_cache(c, okv, p0, 500 + p0)
        tok = 77
        for pos in (p0, p0 + 1):
            worst, tok = replay_step(c, om, okv, pos, tok)
        say(f"chunked at positions {p0}, {p0 + 1}: worst rel L2 {worst:.2e}")
    finally:
        c.close()


@pytest.mark.parametrize("chunks", [WALK, CHUNKS], ids=["walk", "chunked"])
@pytest.mark.parametrize("p0", [2047, 4095])
def test_long_position_same_input(model, p0, chunks):
    """Config 3's position 2047 and the last position of the 4096 context, over seeded INT8
    caches, on the persistent path with stage A walked by the 32 q-head workgroups and
    chunked over every workgroup (the default from 577 positions on)."""
    m, om = model
    ctx_len = min(p0 + 2, 4096)
    c = open_ctx(m.path, chunks)
    try:
        c.kv_create(LAYERS, ctx_len)
        okv = qxo.KV(LAYERS, ctx_len)
        seed_cache(c, okv, p0, 900 + p0)
        tok = 4242
        for pos in range(p0, ctx_len):
            worst, top = replay_step(c, om, okv, pos, tok)
            say(f"p0 {p0} {'walk' if chunks == WALK else 'chunked'}: position {pos} worst rel L2 {worst:.2e}")
            tok = top
    finally:
        c.close()


def test_generate_long_context_matches_steps(model):
    """The greedy loop of one persistent launch over positions 3968..4095 of a seeded
    4096-long cache (the chunked stage A with the cache rows it stores itself) gives the
    tokens of the step-by-step path, whose steps the same-input tests check."""
    m, om = model
    c = open_ctx(m.path)
    try:
        p0, n = 3968, 128
        c.kv_create(LAYERS, 4096)
        okv = qxo.KV(LAYERS, 4096)
        seed_cache(c, okv, p0, 77)
        gen, _ = c.generate([123], n, pos0=p0)
        seed_cache(c, okv, p0, 77)
        tok, toks = 123, []
        for pos in range(p0, p0 + n):
            _, _, _, ids, _ = c.decode_token(tok, pos, True, 1)
            tok = int(ids[0])
            toks.append(tok)
        assert list(gen) == toks
    finally:
        c.close()


@pytest.mark.parametrize("p0", [0, 571], ids=["start", "across_threshold"])
def test_generate_recorded_matches_steps(model, p0):
    """qxg_generate_recorded (the state loop's one launch) keeps for every step what the
    step-by-step path reads back after each qxg_decode_token: the same tokens, layer outputs,
    attention and MoE halves, routing, head sums, final norms, logits, top tokens and cache
    rows, bit for bit (the same kernels on the same inputs).  From p0 571 the 7 steps cross the
    chunked stage A's default threshold (577 positions), so the call runs as two launches, the
    second writing its records from slot 5 on."""
    m, om = model
    c = open_ctx(m.path)
    try:
        prompt, n_gen = [5, 900, 17], 5
        S = len(prompt) + n_gen - 1
        c.kv_create(LAYERS, p0 + S + 1)
        okv = qxo.KV(LAYERS, p0 + S + 1)
        seed_cache(c, okv, p0, 31)
        r = c.generate_recorded(prompt, n_gen, pos0=p0, top_n=8)
        rows = [c.kv_read(l, p0, S) for l in range(LAYERS)]
        assert list(r["tokens"][:len(prompt)]) == prompt
        seed_cache(c, okv, p0, 31)
        tok = prompt[0]
        for s in range(S):
            head = s + 1 >= len(prompt)
            _, lay, lg, ids, tl = c.decode_token(tok, p0 + s, head, 8, want_layers=True, want_logits=head)
            att, moe = c.halves()
            r_ids, r_w = c.routing()
            assert np.array_equal(r["layer"][s], lay), s
            assert np.array_equal(r["attn"][s], att) and np.array_equal(r["moe"][s], moe), s
            assert np.array_equal(r["ids"][s], r_ids) and np.array_equal(r["weights"][s], r_w), s
            assert np.array_equal(r["head_sums"][s], c.head_sums()), s
            if head:
                assert np.array_equal(r["logits"][s], lg) and np.array_equal(r["norm"][s], c.final_norm()), s
                assert np.array_equal(r["top_ids"][s], ids) and np.array_equal(r["top_logits"][s], tl), s
                tok = int(ids[0])
                assert int(r["tokens"][s + 1]) == tok, s
            else:
                tok = prompt[s + 1]
                assert not r["logits"][s].any() and not r["top_ids"][s].any(), s   # no head: zeros
        for l in range(LAYERS):
            for got, want in zip(rows[l], c.kv_read(l, p0, S)):
                assert np.array_equal(got, want), l
        ms = r["step_ms"]
        assert ms[0] == 0.0 and np.all(np.diff(ms) > 0) and ms[-1] <= r["elapsed_ms"], (ms, r["elapsed_ms"])
        say(f"recorded launch at p0 {p0}: {S} steps in {r['elapsed_ms']:.3f} ms, per step "
            f"{', '.join(f'{d:.3f}' for d in np.diff(ms))} ms")
    finally:
        c.close()


def test_generate_recorded_rejects_bad_arguments(model):
    """qxg_generate_recorded fails with a message, before any launch, on an empty prompt or
    no generated token, a prompt token past the vocabulary, a loop past the KV context, and
    on a context whose decode is not the persistent kernel; the context stays usable."""
    m, om = model
    c = open_ctx(m.path)
    try:
        c.kv_create(LAYERS, 8)
        for prompt, n_gen, pos0, msg in (([], 2, 0, "prompt"), ([5], 0, 0, "generated"),
                                         ([VOCAB], 1, 0, "out of range"), ([5, 6], 8, 0, "KV context"),
                                         ([5], 2, 7, "KV context")):
            with pytest.raises(qxg.QxgError, match=msg):
                c.generate_recorded(prompt, n_gen, pos0=pos0)
        r = c.generate_recorded([5, 6], 3)
        gen, _ = c.generate([5, 6], 3)
        assert list(r["tokens"][2:]) == list(gen)
        c.set_layer_path(0)
        assert not c.persistent_path()
        with pytest.raises(qxg.QxgError, match="persistent"):
            c.generate_recorded([5], 1)
    finally:
        c.close()


@pytest.mark.parametrize("chunks", [WALK, CHUNKS], ids=["walk", "chunked"])
def test_outliers_same_input(outlier_model, chunks):
    """Planted outlier channels through the persistent kernel: a 4-token prompt and 3 greedy
    steps, every step replayed layer by layer.

    single: x1000 channels (one in every fourth 32-group of the attention, ffn and output
    norms, channel 5 of the q/k norms) and x1000 fp16 d in a V row of each kv head (the
    context) and in O row 11 (a x1000 channel of the residual stream): every half at 1e-5.

    stress: as single, plus x1e6 in one channel of the attention and output norms and x1000
    fp16 d in gate row 7 and down row 13 of every expert.  The attention half and the logits
    are held to 1e-5; the MoE half and the layer output to 5e-5.  Reason (measured): here
    32-value groups of x' span ~2.6e3 and of h ~6e4 (max over median), and the expert outputs
    cancel in channel 13, so the decode's 22-bit activation digits (2^-23 of a group's maximum
    per value) move the MoE output by 1.2e-5 (x' digits alone) and 1.8e-5 (h digits alone) in
    a CPU emulation of the digit scheme on the same input (tests/test_digit_precision.py); the
    device measured 2.1e-5.  The per-phase kernels use the same digits."""
    m, om, pattern = outlier_model
    moe_tol = REL_L2 if pattern == 1 else 5e-5
    c = open_ctx(m.path, chunks)
    try:
        c.kv_create(LAYERS, 16)
        okv = qxo.KV(LAYERS, 16)
        prompt = [5, 900, 17, 4000]
        tok = prompt[0]
        for pos in range(len(prompt) + 3):
            head = pos >= len(prompt) - 1
            worst, top = replay_step(c, om, okv, pos, tok, head, moe_tol)
            say(f"outliers {pattern} {'walk' if chunks == WALK else 'chunked'}: position {pos} worst rel L2 {worst:.2e}")
            tok = top if head else prompt[pos + 1]
    finally:
        c.close()


SAT_TOL = 1e-4


@pytest.mark.parametrize("chunks", [WALK, CHUNKS], ids=["walk", "chunked"])
def test_saturated_scales_same_input(sat_model, chunks):
    """Exponent-31 fp16 block scales (+inf, -inf, NaN and NaN with the sign bit, which the
    reference reads as +-65504: src/qx_format.c:1854-1876) in every block of a Q, K, V and O
    row of each layer and of a gate, up and down row of every expert.  The persistent
    decode's packed layouts hold these scales saturated and its dots convert them with the
    plain half conversion, so a scale field the packing missed (an infinity or NaN on the
    device) or a lost sign shows here (an error of 1e-2 or more, or a non-finite value).  A
    4-token prompt and 3 greedy steps, every step replayed layer by layer; the residual
    stream reaches ~1e18.  Halves held to 1e-4: the saturated O row multiplies the context's
    eight ~3.5e9 entries (the saturated V row's, one per q head of kv head 0), and its 4096
    terms cancel ~290-fold (sum 4.6e15 of magnitudes 1.3e18, layer 3, position 1), so the
    f32 sums of the digit dots reach 1.4e-5 of the row; measured: the per-phase kernels,
    which convert the unsaturated scales themselves, give the same 1.445e-5 against the
    oracle and agree with the persistent path to 3e-13."""
    m, om = sat_model
    c = open_ctx(m.path, chunks)
    try:
        c.kv_create(LAYERS, 16)
        okv = qxo.KV(LAYERS, 16)
        prompt = [5, 900, 17, 4000]
        tok = prompt[0]
        for pos in range(len(prompt) + 3):
            head = pos >= len(prompt) - 1
            worst, top = replay_step(c, om, okv, pos, tok, head, SAT_TOL, SAT_TOL)
            say(f"saturated scales {'walk' if chunks == WALK else 'chunked'}: position {pos} worst rel L2 {worst:.2e}")
            tok = top if head else prompt[pos + 1]
    finally:
        c.close()


# q8_k_compat: the O projection re-quantizes the device's own context and the down
# projection its own h, so a code may sit one step from the oracle's where the two inputs
# straddle a rounding boundary.  One such code in h moves this model's MoE half by up to
# ~1e-3 (measured 2.3e-3 worst at position 40 with two); a wrong block scale, sign or
# rounding rule costs 1e-2 or more
REQ_TOL = 5e-3


@pytest.mark.parametrize("chunks", [WALK, CHUNKS], ids=["walk", "chunked"])
def test_q8k_same_input(model, chunks):
    """q8_k_compat on the persistent kernel (its Q8_K instantiation: every matvec input as
    Q8_K blocks, codes in the h digit plane): a 4-token prompt over a 40-position seeded
    cache and 3 greedy steps, every layer replayed by the oracle in the same mode on the
    device's own inputs and rows.  The halves and layer outputs are held to REQ_TOL (they
    re-quantize device intermediates), the head's logits to 1e-5 (its input, the device's
    final residual, reaches the quantizer as the oracle's does)."""
    m, _ = model
    om = qxo.Model(m.path, activation="q8_k_compat")
    c = open_ctx(m.path, chunks)
    c.set_activation("q8_k_compat")
    try:
        assert c.persistent_path()
        p0 = 40
        c.kv_create(LAYERS, p0 + 8)
        okv = qxo.KV(LAYERS, p0 + 8)
        seed_cache(c, okv, p0, 310)
        prompt = [5, 900, 17, 4000]
        tok = prompt[0]
        for i in range(len(prompt) + 3):
            pos = p0 + i
            head = i >= len(prompt) - 1
            worst, top = replay_step(c, om, okv, pos, tok, head, moe_tol=REQ_TOL, att_tol=REQ_TOL)
            say(f"q8k {'walk' if chunks == WALK else 'chunked'}: position {pos} worst rel L2 {worst:.2e}")
            tok = top if head else prompt[i + 1]
    finally:
        c.close()
        om.close()


@pytest.mark.parametrize("chunks", [WALK, CHUNKS], ids=["walk", "chunked"])
def test_q8k_saturated_scales_same_input(sat_model, chunks):
    """The exponent-31 block scales of test_saturated_scales_same_input through the Q8_K
    instantiation (its dots read the same saturated layouts): a 4-token prompt and 3 greedy
    steps replayed layer by layer by the oracle in q8_k_compat, halves at REQ_TOL (the
    q8_k_compat bar, above the f32 test's 1e-4), logits at 1e-5."""
    m, _ = sat_model
    om = qxo.Model(m.path, activation="q8_k_compat")
    c = open_ctx(m.path, chunks)
    c.set_activation("q8_k_compat")
    try:
        assert c.persistent_path()
        c.kv_create(LAYERS, 16)
        okv = qxo.KV(LAYERS, 16)
        prompt = [5, 900, 17, 4000]
        tok = prompt[0]
        for pos in range(len(prompt) + 3):
            head = pos >= len(prompt) - 1
            worst, top = replay_step(c, om, okv, pos, tok, head, moe_tol=REQ_TOL, att_tol=REQ_TOL)
            say(f"q8k saturated scales {'walk' if chunks == WALK else 'chunked'}: position {pos} worst rel L2 {worst:.2e}")
            tok = top if head else prompt[pos + 1]
    finally:
        c.close()
        om.close()


def test_q8k_generate_matches_steps(model):
    """q8_k_compat: one persistent launch over a prompt and 6 greedy tokens gives the
    tokens of the step-by-step calls (the same kernel, step by step)."""
    m, _ = model
    c = open_ctx(m.path)
    c.set_activation("q8_k_compat")
    try:
        c.kv_create(LAYERS, 16)
        gen, _ = c.generate([31, 7, 2048], 6)
        c.kv_create(LAYERS, 16)
        for pos, t in enumerate([31, 7, 2048]):
            _, _, _, ids, _ = c.decode_token(t, pos, pos == 2, 1)
        tok = int(ids[0])
        toks = [tok]
        for pos in range(3, 8):
            _, _, _, ids, _ = c.decode_token(tok, pos, True, 1)
            tok = int(ids[0])
            toks.append(tok)
        assert list(gen) == toks
    finally:
        c.close()


def test_q8k_nonfinite_fails_and_clears(model):
    """q8_k_compat on the persistent kernel: a NaN V scale in the cache makes the context,
    the O projection's Q8_K input, non-finite, and the call fails with the reference's
    message (src/qx_format.c:3906); f32 mode zeroes that projection instead.  After the row
    is rewritten the next call succeeds."""
    m, _ = model
    c = open_ctx(m.path)
    try:
        c.kv_create(LAYERS, 8)
        for layer in range(1, LAYERS):
            c.kv_write(layer, 0, *seeded_kv(56 + layer, 1))
        k, v, ks, vs = seeded_kv(55, 1)
        vs_bad = vs.copy()
        vs_bad[0] = np.nan
        c.kv_write(0, 0, k, v, ks, vs_bad)
        res, _, _, _, _ = c.decode_token(9, 1, True, 1)   # f32: the projection of a NaN context is 0
        assert np.isfinite(res).all()
        c.set_activation("q8_k_compat")
        c.kv_write(0, 0, k, v, ks, vs_bad)
        with pytest.raises(qxg.QxgError, match="Q8_K activation contains NaN or Inf"):
            c.decode_token(9, 1, True, 1)
        c.kv_write(0, 0, k, v, ks, vs)
        res, _, _, ids, _ = c.decode_token(9, 1, True, 1)
        assert np.isfinite(res).all()
    finally:
        c.close()


def test_q8k_prefill_one_launch_matches_steps(model):
    """q8_k_compat: qxg_prefill (the reference's token steps) runs as one persistent launch
    when no per-token residual is asked for; its head outputs and the cache rows it leaves
    equal the persistent decode_token steps over the same prompt, bit for bit (the same
    kernel on the same inputs)."""
    m, _ = model
    c = open_ctx(m.path)
    c.set_activation("q8_k_compat")
    try:
        prompt = np.array([31, 7, 2048, 900, 5], np.uint32)
        c.kv_create(LAYERS, 16)
        _, lg, ids, tl, _ = c.prefill(prompt, 0, True, 8, want_logits=True)
        rows = [c.kv_read(l, 0, len(prompt)) for l in range(LAYERS)]
        c.kv_create(LAYERS, 16)
        for pos, t in enumerate(prompt):
            _, _, lg2, ids2, tl2 = c.decode_token(int(t), pos, pos == len(prompt) - 1, 8, want_logits=pos == len(prompt) - 1)
        assert np.array_equal(lg, lg2)
        assert list(ids) == list(ids2) and np.array_equal(tl, tl2)
        for l in range(LAYERS):
            for a, b in zip(rows[l], c.kv_read(l, 0, len(prompt))):
                assert np.array_equal(a, b), l
    finally:
        c.close()
