"""ORACLE — test infrastructure only.  ctypes binding of liboracle.so (qxo.h), the
scalar CPU restatement of the reference's f32 path.  Imported by tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg only, as the checker."""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
_path = os.path.join(HERE, "liboracle.so")
if not os.path.exists(_path):
    raise RuntimeError(f"{_path} is not built: run `make -C {HERE} oracle`")
_o = ctypes.CDLL(_path)
vp, u32, u64, c_int = ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint64, ctypes.c_int


def _sig(name, args, res=c_int):
    f = getattr(_o, name)
    f.argtypes = args
    f.restype = res


_sig("qxo_open", [ctypes.c_char_p], vp)
_sig("qxo_close", [vp], None)
_sig("qxo_fp16_to_f32", [ctypes.c_uint16], ctypes.c_float)
_sig("qxo_decode_block", [u32, vp, vp])
_sig("qxo_fnv1a64", [vp, u64], u64)
_sig("qxo_tensor", [vp, ctypes.c_char_p, ctypes.POINTER(u32), vp, ctypes.POINTER(u64)], vp)
_sig("qxo_final_head", [vp, vp, vp, vp, u32, vp, vp])
_sig("qxo_moe_layer", [vp, u32, vp, vp, vp, vp, vp])
_sig("qxo_attention_layer", [vp, u32, u32, u32, vp, vp, vp, vp, vp, vp, vp, vp])
_sig("qxo_attention_layer_ex", [vp, u32, u32, u32, vp, vp, vp, vp, vp, vp, vp, vp, c_int, vp, vp, vp])
_sig("qxo_decode_token", [vp, u32, u32, u32, u32, vp, vp, vp, vp, vp, vp, c_int, vp, u32, vp, vp])
_sig("qxo_embed", [vp, u32, vp])
_sig("qxo_matvec", [u32, vp, u32, u32, vp, vp], None)
_sig("qxo_quantize_q8k", [vp, u32, vp])
_sig("qxo_matvec_q8k", [u32, vp, u32, u32, vp, vp, c_int])
_sig("qxo_set_activation", [vp, c_int], None)
_sig("qxo_f32_to_fp16", [ctypes.c_float], ctypes.c_uint16)
_sig("qxo_attention_stage", [vp, u32, vp, c_int, vp, vp, vp, vp, vp, vp])
_sig("qxo_moe_stage", [vp, u32, vp, vp, vp])
_sig("qxo_quantize_int8", [vp, vp, u32], ctypes.c_float)

Q8K_BYTES = 292   # ggml block_q8_K: f32 d, int8 qs[256], int16 bsums[16]


def _p(a):
    return None if a is None else a.ctypes.data_as(vp)


def fnv1a64(a):
    a = np.ascontiguousarray(a)
    return int(_o.qxo_fnv1a64(_p(a), a.nbytes))


def fp16_to_f32(h):
    return float(_o.qxo_fp16_to_f32(h))


def decode_block(ggml_type, raw):
    raw = np.ascontiguousarray(raw, np.uint8)
    out = np.zeros(256, np.float32)
    if not _o.qxo_decode_block(ggml_type, _p(raw), _p(out)):
        raise ValueError("unsupported type")
    return out


def quantize_int8(x):
    """reference qx_quantize_int8_vector (src/qx_format.c:4449-4463): (codes, scale)"""
    x = np.ascontiguousarray(x, np.float32)
    codes = np.zeros(len(x), np.int8)
    sc = _o.qxo_quantize_int8(_p(x), _p(codes), len(x))
    return codes, np.float32(sc)


def f32_to_fp16(v):
    return int(_o.qxo_f32_to_fp16(float(v)))


def moe_stage_floats(experts):
    return 2048 + 2 * experts + 25 + 3 * 8 * 768 + 2 * 8 * 2048


def split_moe_stage(block, experts):
    """The named vectors of a MoE-stage output block (qxo.h / qxg.h layout)."""
    names = [("ffn_norm", 2048), ("ffn_moe_logits", experts), ("ffn_moe_probs", experts), ("ffn_moe_topk", 8),
             ("ffn_moe_weights", 8), ("ffn_moe_weights_sum", 1), ("ffn_moe_weights_norm", 8),
             ("ffn_moe_gate", 8 * 768), ("ffn_moe_up", 8 * 768), ("ffn_moe_swiglu", 8 * 768),
             ("ffn_moe_down", 8 * 2048), ("ffn_moe_weighted", 8 * 2048)]
    out, o = {}, 0
    for n, c in names:
        out[n] = block[o:o + c]
        o += c
    assert o == len(block)
    return out


def quantize_q8k(x):
    """Q8_K blocks of x (length a multiple of 256) as raw bytes, or None when the
    reference would fail (a non-finite value)."""
    x = np.ascontiguousarray(x, np.float32)
    out = np.zeros(Q8K_BYTES * (len(x) // 256), np.uint8)
    return out if _o.qxo_quantize_q8k(_p(x), len(x), _p(out)) else None


def matvec(ggml_type, w, rows, in_dims, x):
    """rows of raw weight bytes w against f32 x (double accumulation, f32 results)."""
    w = np.ascontiguousarray(w, np.uint8)
    x = np.ascontiguousarray(x, np.float32)
    y = np.zeros(rows, np.float32)
    _o.qxo_matvec(ggml_type, _p(w), rows, in_dims, _p(x), _p(y))
    return y


def matvec_q8k(ggml_type, w, rows, in_dims, x, expert=False):
    """rows of raw weight bytes w against x in q8_k_compat mode; None on failure."""
    w = np.ascontiguousarray(w, np.uint8)
    x = np.ascontiguousarray(x, np.float32)
    y = np.zeros(rows, np.float32)
    return y if _o.qxo_matvec_q8k(ggml_type, _p(w), rows, in_dims, _p(x), _p(y), int(expert)) else None


class Model:
    """A QXF1 file opened by the oracle (mmap).  activation: "f32" or "q8_k_compat"."""

    def __init__(self, path, activation="f32"):
        if activation not in ("f32", "q8_k_compat"):
            raise ValueError(activation)
        self._m = _o.qxo_open(str(path).encode())
        if not self._m:
            raise RuntimeError(f"oracle cannot open {path}")
        _o.qxo_set_activation(self._m, int(activation == "q8_k_compat"))

    def close(self):
        if self._m:
            _o.qxo_close(self._m)
            self._m = None

    def tensor(self, name):
        t = u32(); n = u64(); dims = np.zeros(4, np.uint64)
        p = _o.qxo_tensor(self._m, name.encode(), ctypes.byref(t), _p(dims), ctypes.byref(n))
        if not p:
            raise KeyError(name)
        buf = (ctypes.c_uint8 * n.value).from_address(p)
        return t.value, dims, np.frombuffer(buf, np.uint8)

    def final_head(self, residual, vocab, top_n=8):
        r = np.ascontiguousarray(residual, np.float32)
        nrm = np.zeros(2048, np.float32); lg = np.zeros(vocab, np.float32)
        ids = np.zeros(top_n, np.uint32); tl = np.zeros(top_n)
        if not _o.qxo_final_head(self._m, _p(r), _p(nrm), _p(lg), top_n, _p(ids), _p(tl)):
            raise RuntimeError("oracle final head failed (non-finite logit?)")
        return nrm, lg, ids, tl

    def moe_layer(self, layer, x):
        x = np.ascontiguousarray(x, np.float32)
        y = np.zeros(2048, np.float32); moe = np.zeros(2048, np.float32)
        ids = np.zeros(8, np.uint32); w = np.zeros(8)
        if not _o.qxo_moe_layer(self._m, layer, _p(x), _p(y), _p(moe), _p(ids), _p(w)):
            raise RuntimeError("oracle MoE failed")
        return y, moe, ids, w

    def attention_stage(self, layer, x, f16_kv=False):
        """(attn_norm, Vcur, kqv_out, attn_out, ffn_inp, (v_probe, output_probe)); None when
        the reference fails the probe (a non-finite output)."""
        x = np.ascontiguousarray(x, np.float32)
        nrm = np.zeros(2048, np.float32); vc = np.zeros(512, np.float32); kqv = np.zeros(4096, np.float32)
        ao = np.zeros(2048, np.float32); fi = np.zeros(2048, np.float32); pr = np.zeros(2)
        if not _o.qxo_attention_stage(self._m, layer, _p(x), int(f16_kv), _p(nrm), _p(vc), _p(kqv), _p(ao), _p(fi), _p(pr)):
            return None
        return nrm, vc, kqv, ao, fi, (float(pr[0]), float(pr[1]))

    def moe_stage(self, layer, x, experts):
        """(dict of the stage's named vectors, ids[8]); None when the reference fails."""
        x = np.ascontiguousarray(x, np.float32)
        blk = np.zeros(moe_stage_floats(experts), np.float32); ids = np.zeros(8, np.uint32)
        if not _o.qxo_moe_stage(self._m, layer, _p(x), _p(blk), _p(ids)):
            return None
        return split_moe_stage(blk, experts), ids

    def embed(self, token):
        x = np.zeros(2048, np.float32)
        if not _o.qxo_embed(self._m, token, _p(x)):
            raise RuntimeError("oracle embed failed")
        return x


class KV:
    """Host INT8 KV cache in the reference layout [layers][ctx][512]."""

    def __init__(self, layers, ctx):
        self.layers, self.ctx = layers, ctx
        self.k = np.zeros((layers, ctx, 512), np.int8)
        self.v = np.zeros((layers, ctx, 512), np.int8)
        self.ks = np.zeros((layers, ctx), np.float32)
        self.vs = np.zeros((layers, ctx), np.float32)


def attention_layer(model, layer, pos, kv, x):
    x = np.ascontiguousarray(x, np.float32)
    a = np.zeros(2048, np.float32); kqv = np.zeros(4096, np.float32); vcur = np.zeros(512, np.float32)
    if not _o.qxo_attention_layer(model._m, layer, pos, kv.ctx, _p(x), _p(kv.k), _p(kv.v), _p(kv.ks), _p(kv.vs),
                                  _p(a), _p(kqv), _p(vcur)):
        raise RuntimeError("oracle attention failed")
    return a, kqv, vcur


def attention_layer_given_row(model, layer, pos, kv, x):
    """Attention on the cache as given, including the row at [layer][pos] (not
    overwritten); also returns the oracle's own INT8 row for that position:
    (attn_out, kqv, vcur, k_row, v_row, (k_scale, v_scale))."""
    x = np.ascontiguousarray(x, np.float32)
    a = np.zeros(2048, np.float32); kqv = np.zeros(4096, np.float32); vcur = np.zeros(512, np.float32)
    rk = np.zeros(512, np.int8); rv = np.zeros(512, np.int8); sc = np.zeros(2, np.float32)
    if not _o.qxo_attention_layer_ex(model._m, layer, pos, kv.ctx, _p(x), _p(kv.k), _p(kv.v), _p(kv.ks), _p(kv.vs),
                                     _p(a), _p(kqv), _p(vcur), 1, _p(rk), _p(rv), _p(sc)):
        raise RuntimeError("oracle attention failed")
    return a, kqv, vcur, rk, rv, (float(sc[0]), float(sc[1]))


def decode_token(model, token, pos, kv, layers, run_head, vocab, top_n=8):
    res = np.zeros(2048, np.float32); lay = np.zeros((layers, 2048), np.float32)
    lg = np.zeros(vocab, np.float32) if run_head else None
    ids = np.zeros(top_n, np.uint32); tl = np.zeros(top_n)
    if not _o.qxo_decode_token(model._m, token, pos, kv.ctx, layers, _p(kv.k), _p(kv.v), _p(kv.ks), _p(kv.vs),
                               _p(res), _p(lay), int(run_head), _p(lg), top_n, _p(ids), _p(tl)):
        raise RuntimeError("oracle decode failed")
    return res, lay, lg, ids, tl
