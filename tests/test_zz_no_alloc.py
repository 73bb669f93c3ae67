"""qxg_dequant_blocks_static (the allocation-free entry point: static device workspace,
caller-owned device input and output) against qxg_dequant_blocks on the same blocks,
bit for bit, on two calls in a row - the second with fewer blocks and another type -
plus its size limit and the device's free memory left unchanged by its calls.

The caller's device buffers come from the HIP runtime libqxg.so itself uses
(/opt/rocm/lib/libamdhip64.so.7, already loaded with it), not from torch, whose wheel
carries a HIP runtime of its own."""
import ctypes

import numpy as np
import pytest

import qxg
import qxo

pytestmark = pytest.mark.gpu

BLOCK_BYTES = {12: 144, 13: 176, 14: 210, 17: 74, 18: 98, 21: 110, 22: 82, 23: 136}
H2D, D2H = 1, 2


class Hip:
    def __init__(self):
        self.lib = ctypes.CDLL("/opt/rocm/lib/libamdhip64.so.7")
        for name, args in (("hipMalloc", [ctypes.POINTER(ctypes.c_void_p), ctypes.c_size_t]),
                           ("hipFree", [ctypes.c_void_p]),
                           ("hipMemcpy", [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]),
                           ("hipMemGetInfo", [ctypes.POINTER(ctypes.c_size_t), ctypes.POINTER(ctypes.c_size_t)])):
            getattr(self.lib, name).argtypes = args
            getattr(self.lib, name).restype = ctypes.c_int
        self.held = []

    def malloc(self, n):
        p = ctypes.c_void_p()
        assert self.lib.hipMalloc(ctypes.byref(p), n) == 0
        self.held.append(p.value)
        return p.value

    def put(self, arr):
        arr = np.ascontiguousarray(arr)
        p = self.malloc(arr.nbytes)
        assert self.lib.hipMemcpy(p, arr.ctypes.data, arr.nbytes, H2D) == 0
        return p

    def get(self, p, dtype, count):
        out = np.empty(count, dtype)
        assert self.lib.hipMemcpy(out.ctypes.data, p, out.nbytes, D2H) == 0
        return out

    def free_bytes(self):
        f, t = ctypes.c_size_t(), ctypes.c_size_t()
        assert self.lib.hipMemGetInfo(ctypes.byref(f), ctypes.byref(t)) == 0
        return f.value

    def release(self):
        for p in self.held:
            self.lib.hipFree(p)
        self.held = []


def test_static_dequant_matches_dequant_blocks(tmp_path):
    p = tmp_path / "m.qxf"
    qxg.generate_model(p, layers=2, vocab=4096, experts=16, seed=11, mix=1)
    m = qxo.Model(p)
    cases = [("output.weight", 4096), ("blk.1.ffn_down_exps.weight", 700), ("token_embd.weight", 33)]
    with qxg.Context(0) as c:      # opening the context makes device 0 current on this thread
        c.load(p, verify=False)
        hip = Hip()
        try:
            for name, nb in cases:
                t, _, raw = m.tensor(name)
                r = np.ascontiguousarray(raw[:nb * BLOCK_BYTES[t]])
                want = c.dequant(t, r, nb)                   # the existing entry point
                draw = hip.put(r)
                dout = hip.put(np.full(nb * 256, np.nan, np.float32))
                c.dequant_static(t, draw, nb, dout)
                got = hip.get(dout, np.float32, nb * 256)
                assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (name, nb)
            small = hip.malloc(256)
            with pytest.raises(qxg.QxgError, match="at most 4096"):
                c.dequant_static(14, small, 4097, small)
        finally:
            hip.release()
    m.close()


def test_static_dequant_allocates_nothing(tmp_path):
    """Calls after a first one (which brings the kernels' code in): the device's free
    memory is the same before and after them."""
    p = tmp_path / "m.qxf"
    qxg.generate_model(p, layers=1, vocab=4096, experts=16, seed=12)
    m = qxo.Model(p)
    t, _, raw = m.tensor("output.weight")
    r = np.ascontiguousarray(raw[:4096 * BLOCK_BYTES[t]])
    with qxg.Context(0) as c:
        hip = Hip()
        try:
            draw = hip.put(r)
            dout = hip.malloc(4096 * 256 * 4)
            c.dequant_static(t, draw, 4096, dout)
            first = hip.get(dout, np.float32, 4096 * 256)
            free0 = hip.free_bytes()
            c.dequant_static(t, draw, 4096, dout)
            c.dequant_static(t, draw, 100, dout)
            assert hip.free_bytes() == free0
            again = hip.get(dout, np.float32, 4096 * 256)
            assert np.array_equal(again.view(np.uint32), first.view(np.uint32))
        finally:
            hip.release()
    m.close()
