"""QXKVSNP1 KV snapshots (reference src/qx_format.c:5860-5968) on the host side of the
C ABI: the files the reference's own CLI wrote for the golden state loops
(tests/golden/kvsnap_*.bin) are read back, and rewritten byte for byte from the
oracle's cache after the same steps; SHA-256 digest and fail-closed checks."""
import hashlib
import json
import os

import numpy as np
import pytest

import qxo
import qxg

GOLDEN_DIR = os.path.join(os.path.dirname(__file__), "golden")
GOLDEN = json.load(open(os.path.join(GOLDEN_DIR, "golden.json")))


def oracle_cache(tmp_path, k):
    """The oracle's INT8 cache after the golden state loop of model k (the golden test
    pins those steps bit-for-bit to the reference)."""
    spec = GOLDEN["models"][k]
    p = tmp_path / f"{k}.qxf"
    qxg.generate_model(p, **spec)
    m = qxo.Model(p)
    g = GOLDEN["state_loop"][k]
    kv = qxo.KV(spec["layers"], g["ctx"])
    for s, tok in enumerate(g["input_tokens"]):
        x = m.embed(tok)
        for layer in range(spec["layers"]):
            a, _, _ = qxo.attention_layer(m, layer, s, kv, x)
            x = x + a
            x, _, _, _ = m.moe_layer(layer, x)
    m.close()
    return kv


@pytest.mark.parametrize("k", ["A", "B", "C"])
def test_snapshot_bytes_match_reference(tmp_path, k):
    snap = GOLDEN["kv_snapshot"][k]
    ref = np.fromfile(os.path.join(GOLDEN_DIR, snap["file"]), np.uint8)
    kv = oracle_cache(tmp_path, k)
    out = tmp_path / "mine.bin"
    qxg.kvsnap_write(out, snap["final_token"], snap["seed"], kv.k, kv.v, kv.ks, kv.vs, snap["positions"])
    assert np.fromfile(out, np.uint8).tobytes() == ref.tobytes()
    # and the reference's file reads back into the same cache
    layers, ctx = kv.ks.shape
    rk, rv, rks, rvs, pos, nt = qxg.kvsnap_read(os.path.join(GOLDEN_DIR, snap["file"]), layers, ctx, snap["seed"])
    assert (pos, nt) == (snap["positions"], snap["final_token"])
    n = snap["positions"]
    assert np.array_equal(rk[:, :n], kv.k[:, :n]) and np.array_equal(rv[:, :n], kv.v[:, :n])
    assert np.array_equal(rks[:, :n].view(np.uint32), kv.ks[:, :n].view(np.uint32))
    assert np.array_equal(rvs[:, :n].view(np.uint32), kv.vs[:, :n].view(np.uint32))


def test_digest_is_sha256_of_the_body(tmp_path):
    rng = np.random.default_rng(3)
    layers, ctx, n = 3, 40, 37   # 37 positions: the body is not a multiple of the 64-byte block
    k = rng.integers(-127, 128, (layers, ctx, 512), dtype=np.int8)
    v = rng.integers(-127, 128, (layers, ctx, 512), dtype=np.int8)
    ks = rng.uniform(1e-3, 1.0, (layers, ctx)).astype(np.float32)
    vs = rng.uniform(1e-3, 1.0, (layers, ctx)).astype(np.float32)
    p = tmp_path / "s.bin"
    qxg.kvsnap_write(p, 99, 7, k, v, ks, vs, n)
    raw = p.read_bytes()
    assert len(raw) == 48 + layers * n * 1032 + 32
    assert raw[:8] == b"QXKVSNP1"
    assert list(np.frombuffer(raw[8:48], np.uint32)) == [2, layers, n, ctx, 4, 128, 1, 512, 99, 7]
    assert hashlib.sha256(raw[:-32]).digest() == raw[-32:]
    # layout: layer-major, then position: K row, V row, K scale, V scale
    off = 48 + (1 * n + 5) * 1032
    assert raw[off:off + 512] == k[1, 5].tobytes() and raw[off + 512:off + 1024] == v[1, 5].tobytes()
    assert raw[off + 1024:off + 1032] == np.array([ks[1, 5], vs[1, 5]], np.float32).tobytes()
    rk, rv, rks, rvs, pos, nt = qxg.kvsnap_read(p, layers, ctx, 7)
    assert (pos, nt) == (n, 99)
    assert np.array_equal(rk[:, :n], k[:, :n]) and np.array_equal(rvs[:, :n], vs[:, :n])


def test_snapshot_fails_closed(tmp_path):
    src = os.path.join(GOLDEN_DIR, GOLDEN["kv_snapshot"]["B"]["file"])
    raw = bytearray(open(src, "rb").read())
    seed = GOLDEN["kv_snapshot"]["B"]["seed"]
    cases = {"payload": (500, "payload mismatch"), "digest": (len(raw) - 1, "payload mismatch"),
             "layers": (12, "header mismatch"), "magic": (0, "header mismatch")}
    for name, (off, msg) in cases.items():
        bad = bytearray(raw)
        bad[off] ^= 1
        p = tmp_path / f"{name}.bin"
        p.write_bytes(bytes(bad))
        with pytest.raises(qxg.QxgError, match=msg):
            qxg.kvsnap_read(p, 2, 8, seed)
    p = tmp_path / "tail.bin"
    p.write_bytes(bytes(raw) + b"\0")
    with pytest.raises(qxg.QxgError, match="payload mismatch"):
        qxg.kvsnap_read(p, 2, 8, seed)
    with pytest.raises(qxg.QxgError, match="header mismatch"):
        qxg.kvsnap_read(src, 2, 8, seed + 1)
    with pytest.raises(qxg.QxgError, match="header mismatch"):
        qxg.kvsnap_read(src, 2, 16, seed)
