"""Host side without a GPU: the QXF1 loader's fail-closed validation (reference
src/qx_format.c:438-460, 712-841), the generator's determinism, the C-ABI
library's exports, and the CLI's usage/failure exit codes."""
import ctypes
import os
import re
import shutil
import subprocess

import numpy as np
import pytest

import qxg

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "qx-mini-c_amd")


class QxfFile(ctypes.Structure):
    _fields_ = [("fd", ctypes.c_int), ("header", ctypes.c_uint8 * 272), ("dir", ctypes.c_void_p), ("map", ctypes.c_void_p)]


_h = qxg._h
_h.qxf_open.argtypes = [ctypes.c_char_p, ctypes.POINTER(QxfFile), ctypes.c_char_p, ctypes.c_uint64]
_h.qxf_close.argtypes = [ctypes.POINTER(QxfFile)]


def open_err(path):
    f = QxfFile()
    err = ctypes.create_string_buffer(256)
    ok = _h.qxf_open(str(path).encode(), ctypes.byref(f), err, 256)
    if ok:
        _h.qxf_close(ctypes.byref(f))
        return None
    return err.value.decode()


@pytest.fixture(scope="module")
def small(tmp_path_factory):
    p = tmp_path_factory.mktemp("host") / "m.qxf"
    qxg.generate_model(p, layers=1, vocab=512, experts=8, seed=9)
    return p


def test_generated_file_opens_and_has_reference_tensor_set(small):
    assert open_err(small) is None
    data = open(small, "rb").read()
    assert data[:4] == b"QXF1" and int.from_bytes(data[16:20], "little") == 3 + 12


def test_generator_is_deterministic(tmp_path):
    a, b, c = tmp_path / "a.qxf", tmp_path / "b.qxf", tmp_path / "c.qxf"
    qxg.generate_model(a, layers=1, vocab=256, experts=8, seed=3, threads=1)
    qxg.generate_model(b, layers=1, vocab=256, experts=8, seed=3, threads=8)
    qxg.generate_model(c, layers=1, vocab=256, experts=8, seed=4)
    assert open(a, "rb").read() == open(b, "rb").read()
    assert open(a, "rb").read() != open(c, "rb").read()


def _corrupt(src, dst, off, data):
    shutil.copy(src, dst)
    with open(dst, "r+b") as f:
        f.seek(off)
        f.write(data)


@pytest.mark.parametrize("off,data,msg", [
    (0, b"QXF2", "bad QXF magic"),
    (4, (2).to_bytes(4, "little"), "unsupported QXF version"),
    (56 + 8, (7).to_bytes(4, "little"), "manifest checksum mismatch"),
    (24, (4096 + 8).to_bytes(8, "little"), "invalid QXF layout"),
])
def test_header_corruption_fails_closed(small, tmp_path, off, data, msg):
    p = tmp_path / "bad.qxf"
    _corrupt(small, p, off, data)
    assert open_err(p) == msg


def test_directory_corruption_fails_closed(small, tmp_path):
    raw = open(small, "rb").read()
    dir_off = int.from_bytes(raw[24:32], "little")
    e0, e1 = dir_off, dir_off + 208
    cases = [
        (e1, raw[e0:e0 + 96], "duplicate tensor name"),                            # name clash
        (e0 + 164, (99).to_bytes(4, "little"), "invalid tensor metadata"),          # unknown ggml type
        (e0 + 152, (12345).to_bytes(8, "little"), "tensor byte size inconsistent with dimensions"),
        (e1 + 144, raw[e0 + 144:e0 + 152], "overlapping tensor ranges"),             # same offset
        (e0 + 144, (5).to_bytes(8, "little"), "invalid tensor placement"),           # misaligned
    ]
    for off, data, msg in cases:
        p = tmp_path / "bad.qxf"
        _corrupt(small, p, off, data)
        assert open_err(p) == msg, msg
    p = tmp_path / "short.qxf"
    shutil.copy(small, p)
    with open(p, "r+b") as f:
        f.truncate(len(raw) - 4096)
    assert open_err(p) == "declared QXF file size does not match file"


def test_abi_library_exports_every_declared_symbol():
    for header, lib in (("qxg.h", qxg._g), ("qx_host.h", qxg._h)):
        src = open(os.path.join(ROOT, "include", header)).read()
        names = set(re.findall(r"^\s*(?:int|void|uint64_t)\s+\**(q\w+)\s*\(", src, re.M))
        assert len(names) >= 8
        for n in sorted(names):
            assert hasattr(lib, n), f"{n} declared in {header} but not exported"


def test_reference_prototypes_compile_and_link(tmp_path):
    """A C caller written against the reference's declarations of the replaced entry points
    (tests/abi/reference_prototypes.c holds them verbatim beside include/qx_host.h) compiles
    without conflicting types, links against libqxhost.so by those names, and runs (it only
    takes their addresses)."""
    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("no C compiler")
    lib = os.path.join(ROOT, "qx-mini-c_amd", "lib")
    exe = tmp_path / "abi_check"
    r = subprocess.run([gcc, "-std=c17", "-Wall", "-Wextra", "-Werror", "-I" + os.path.join(ROOT, "include"),
                        os.path.join(ROOT, "tests", "abi", "reference_prototypes.c"), "-o", str(exe), "-L" + lib,
                        "-lqxhost", "-lqxg", "-Wl,-rpath," + lib], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0 and r.stdout.strip() == "7", (r.returncode, r.stdout, r.stderr)


def _have_gpu():
    try:
        c = qxg.Context(0)
        c.close()
        return True
    except qxg.QxgError:
        return False


@pytest.mark.skipif(_have_gpu(), reason="checks the no-device error path")
def test_open_without_device_reports_an_error():
    with pytest.raises(qxg.QxgError):
        qxg.Context(0)


def test_cli_usage_and_failures(small, tmp_path):
    exe = os.path.join(PKG, "bin", "qxqxf")
    assert subprocess.run([exe], capture_output=True).returncode == 2
    assert subprocess.run([exe, "final-head-probe", "--in", str(small)], capture_output=True).returncode == 2
    r = subprocess.run([exe, "generate-model", "--out", str(tmp_path / "g.qxf"), "--layers", "1", "--vocab", "256",
                        "--experts", "8", "--seed", "9"], capture_output=True, text=True)
    assert r.returncode == 0 and '"file_size"' in r.stdout
    # non-finite sidecar is rejected before any device work (reference src/qx_format.c:5340-5342)
    x = np.zeros(2048, np.float32)
    x[5] = np.nan
    x.tofile(tmp_path / "r.f32")
    r = subprocess.run([exe, "final-head-probe", "--in", str(small), "--residual", str(tmp_path / "r.f32"),
                        "--out-dir", str(tmp_path)], capture_output=True, text=True)
    assert r.returncode == 1 and "non-finite" in r.stderr
    assert not os.path.exists(tmp_path / "logits.f32")


def test_cli_q8k_probe_argument_errors():
    """q8-k-activation-probe rejects bad arguments before any device work, with the
    reference's messages and exit codes (src/qx_qxf_main.c:235-258, qx_format.c:4304-4314)."""
    exe = os.path.join(PKG, "bin", "qxqxf")
    r = subprocess.run([exe, "q8-k-activation-probe"], capture_output=True, text=True)
    assert r.returncode == 2 and "invalid --values" in r.stderr
    r = subprocess.run([exe, "q8-k-activation-probe", "--values", "x"], capture_output=True, text=True)
    assert r.returncode == 2
    r = subprocess.run([exe, "q8-k-activation-probe", "--values", "256", "--inject", "bogus"], capture_output=True, text=True)
    assert r.returncode == 1 and "invalid Q8_K activation injection" in r.stderr
    r = subprocess.run([exe, "q8-k-activation-probe", "--values", "8192"], capture_output=True, text=True)
    assert r.returncode == 1 and "workspace is too small" in r.stderr


def test_cli_state_loop_and_stage_refusals(small, tmp_path):
    """The state-loop and stage probes refuse before any device work: the reference's
    usage errors (exit 2: --start-layer without --residual-in, both snapshot flags,
    src/qx_qxf_main.c:1803) and argument checks (exit 1, src/qx_format.c:5971-6041,
    5482-5486, 5590-5593), and this build's own limits (the --full-moe path, INT8 KV, no
    tokenizer)."""
    exe = os.path.join(PKG, "bin", "qxqxf")

    def run(*args):
        return subprocess.run([exe, *map(str, args)], capture_output=True, text=True)

    base = ["state-loop-probe", "--in", small, "--prompt-token", "1"]
    assert run(*base, "--full-moe", "--start-layer", "1").returncode == 2
    assert run(*base, "--full-moe", "--kv-snapshot-in", "a", "--kv-snapshot-out", "b").returncode == 2
    assert run(*base, "--full-moe", "--bogus").returncode == 2
    r = run(*base)
    assert r.returncode == 1 and r.stderr.strip() == "state-loop-probe failed: the GPU state loop implements the --full-moe path only"
    r = run(*base, "--full-moe", "--kv", "f16")
    assert r.returncode == 1 and "supports INT8 KV only" in r.stderr
    r = run(*base, "--full-moe", "--activation", "bf16")
    assert r.returncode == 1 and r.stderr.strip() == "state-loop-probe failed: unsupported activation format"
    r = run(*base, "--full-moe", "--norm", "x")
    assert r.returncode == 1 and "--norm cannot be combined with --full-moe" in r.stderr
    r = run(*base, "--full-moe", "--steps", "2", "--start-layer", "0", "--residual-in", tmp_path / "r.f32")
    assert r.returncode == 1 and "residual replay requires" in r.stderr
    r = run("prompt-state-loop-probe", "--in", small, "--tokenizer", "t.qxt", "--text-file", "p.txt", "--full-moe", "--final-head")
    assert r.returncode == 2 and "--prompt-ids" in r.stderr
    r = run("prompt-state-loop-probe", "--in", small, "--prompt-ids", "1,2", "--generate", "1", "--full-moe", "--final-head",
            "--thread-policy", "serial", "--threads", "4")
    assert r.returncode == 1 and "serial thread policy requires --threads 1" in r.stderr
    r = run("attention-stage-probe", "--in", small, "--layer", "0", "--layer-in", "x", "--out-dir", tmp_path, "--kv", "int8")
    assert r.returncode == 1 and "invalid attention stage probe argument, activation mode, or KV format" in r.stderr
    r = run("moe-stage-probe", "--in", small, "--layer", "0", "--ffn-inp", "x", "--out-dir", tmp_path, "--activation", "f16")
    assert r.returncode == 1 and "invalid MoE stage probe argument or activation mode" in r.stderr
    assert run("moe-stage-probe", "--in", small, "--layer", "0").returncode == 2
