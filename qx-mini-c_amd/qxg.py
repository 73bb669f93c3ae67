"""ctypes binding of the C ABI in include/qxg.h and include/qx_host.h.

Loads lib/libqxg.so and lib/libqxhost.so built in-tree by the Makefile next to
this file; raises if they are missing (there is no fallback path)."""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_DIR = os.path.join(HERE, "lib")


def _load(name):
    path = os.path.join(LIB_DIR, name)
    if not os.path.exists(path):
        raise RuntimeError(f"{path} is not built: run `make -C {HERE}` (or __graft_entry__.build())")
    return ctypes.CDLL(path)


_g = _load("libqxg.so")
_h = _load("libqxhost.so")

u32, u64, c_int, c_float, c_double, vp, cp = (ctypes.c_uint32, ctypes.c_uint64, ctypes.c_int, ctypes.c_float,
                                               ctypes.c_double, ctypes.c_void_p, ctypes.c_char_p)
ERR = (cp, u64)


MOE_STAGE_NAMES = ["ffn_norm", "ffn_moe_logits", "ffn_moe_probs", "ffn_moe_topk", "ffn_moe_weights",
                   "ffn_moe_weights_sum", "ffn_moe_weights_norm", "ffn_moe_gate", "ffn_moe_up", "ffn_moe_swiglu",
                   "ffn_moe_down", "ffn_moe_weighted"]


def moe_stage_floats(experts):
    """QXG_MOE_STAGE_FLOATS of include/qxg.h"""
    return 2048 + 2 * experts + 25 + 3 * 8 * 768 + 2 * 8 * 2048


def split_moe_stage(block, experts):
    sizes = [2048, experts, experts, 8, 8, 1, 8, 8 * 768, 8 * 768, 8 * 768, 8 * 2048, 8 * 2048]
    out, o = {}, 0
    for n, c in zip(MOE_STAGE_NAMES, sizes):
        out[n] = block[o:o + c]
        o += c
    return out


def _sig(lib, name, args, res=c_int):
    f = getattr(lib, name)
    f.argtypes = list(args)
    f.restype = res
    return f


class GenSpec(ctypes.Structure):
    _fields_ = [("layers", u32), ("vocab", u32), ("experts", u32), ("with_embedding", u32), ("with_head", u32),
                ("seed", u64), ("threads", u32), ("mix", u32), ("outliers", u32)]


class ModelInfo(ctypes.Structure):
    _fields_ = [("layers", u32), ("vocab", u32), ("experts", u32), ("has_embedding", c_int), ("has_head", c_int),
                ("tensor_bytes", u64), ("tensors", u32)]


_sig(_g, "qxg_open", [c_int, ctypes.POINTER(vp), *ERR])
_sig(_g, "qxg_close", [vp], None)
_sig(_g, "qxg_upload_tensor", [vp, cp, u32, ctypes.POINTER(u64), vp, u64, *ERR])
_sig(_g, "qxg_bind_model", [vp, u32, c_int, c_int, *ERR])
_sig(_g, "qxg_kv_create", [vp, u32, u32, u32, *ERR])
_sig(_g, "qxg_kv_write", [vp, u32, u32, u32, vp, vp, vp, vp, *ERR])
_sig(_g, "qxg_kv_read", [vp, u32, u32, u32, vp, vp, vp, vp, *ERR])
_sig(_g, "qxg_decode_token", [vp, u32, u32, c_int, vp, vp, vp, u32, vp, vp, *ERR])
_sig(_g, "qxg_generate", [vp, vp, u32, u32, u32, vp, ctypes.POINTER(c_float), *ERR])
_sig(_g, "qxg_persistent_path", [vp])
_sig(_g, "qxg_generate_recorded", [vp, vp, u32, u32, u32, u32] + [vp] * 12 + [ctypes.POINTER(c_float), *ERR])
_sig(_g, "qxg_embed_token", [vp, u32, vp, *ERR])
_sig(_g, "qxg_dequant_blocks", [vp, u32, vp, u64, vp, *ERR])
_sig(_g, "qxg_dequant_blocks_static", [vp, u32, vp, u64, vp, *ERR])
_sig(_g, "qxg_int8_quantize", [vp, vp, u32, vp, vp, *ERR])
_sig(_g, "qxg_attention_layer", [vp, u32, u32, vp, vp, vp, vp, *ERR])
_sig(_g, "qxg_moe_layer", [vp, u32, vp, vp, vp, vp, vp, *ERR])
_sig(_g, "qxg_attention_layer_ex", [vp, u32, u32, vp, vp, vp, vp, vp, *ERR])
_sig(_g, "qxg_attention_stage", [vp, u32, c_int, vp, vp, vp, vp, vp, vp, *ERR])
_sig(_g, "qxg_moe_stage", [vp, u32, vp, vp, vp, *ERR])
_sig(_g, "qxg_final_head", [vp, vp, vp, vp, u32, vp, vp, *ERR])
_sig(_g, "qxg_set_layer_path", [vp, c_int])
_sig(_g, "qxg_set_activation", [vp, u32, vp, u64])
_sig(_g, "qxg_q8k_quantize", [vp, vp, u32, vp, vp, u64])
_sig(_g, "qxg_kv_export", [vp, cp, u32, u32, u32, u32, u32, *ERR])
_sig(_g, "qxg_kv_import", [vp, cp, u32, u32, u32, ctypes.POINTER(u32), ctypes.POINTER(u32), *ERR])
_sig(_g, "qxg_kvsnap_write", [cp, u32, u32, u32, u32, u32, vp, vp, vp, vp, *ERR])
_sig(_g, "qxg_kvsnap_read", [cp, u32, u32, u32, vp, vp, vp, vp, ctypes.POINTER(u32), ctypes.POINTER(u32), *ERR])
_sig(_g, "qxg_prefill", [vp, vp, u32, u32, c_int, vp, vp, u32, vp, vp, ctypes.POINTER(c_float), *ERR])
_sig(_g, "qxg_prefill_layer", [vp, u32, u32, u32, vp, vp, vp, vp, *ERR])
_sig(_g, "qxg_time_kernel", [vp, c_int, u32, u32, ctypes.POINTER(c_float), *ERR])
_sig(_g, "qxg_decode_routing", [vp, u32, vp, vp, *ERR])
_sig(_g, "qxg_decode_halves", [vp, u32, vp, vp, *ERR])
_sig(_g, "qxg_set_attention_chunks", [vp, u32])
_sig(_g, "qxg_decode_head_sums", [vp, u32, vp, *ERR])
_sig(_g, "qxg_decode_final_norm", [vp, vp, *ERR])
_sig(_g, "qxg_kv_read_position", [vp, u32, u32, vp, vp, vp, vp, *ERR])
_sig(_g, "qxg_device_bytes", [vp], u64)
_sig(_g, "qxg_profile_kernel", [vp, c_int])
_sig(_g, "qxg_profile_result", [vp, ctypes.POINTER(u32), ctypes.POINTER(c_double)])
_sig(_h, "qxgen_write", [cp, ctypes.POINTER(GenSpec), ctypes.POINTER(u64), *ERR])
_sig(_h, "qxgen_memfd", [ctypes.POINTER(GenSpec), cp, u64, ctypes.POINTER(c_int), *ERR])
_sig(_h, "qxgen_memfd_close", [c_int], None)
_sig(_h, "qx_gpu_load", [vp, cp, c_int, ctypes.POINTER(ModelInfo), *ERR])
_sig(_h, "qxf_fnv1a64", [vp, u64], u64)


class QxgError(RuntimeError):
    pass


def _p(a):
    return None if a is None else a.ctypes.data_as(vp)


def fnv1a64(a):
    a = np.ascontiguousarray(a)
    return int(_h.qxf_fnv1a64(_p(a), a.nbytes))


def generate_model(path, layers=1, vocab=4096, experts=128, embedding=True, head=True, seed=1, threads=0, mix=0,
                   outliers=0):
    """Writes the seeded random-init QXF1 model (mix=1: the real checkpoint's per-layer
    quant types; outliers=1: planted outlier channels, see qx_host.h); returns its size in
    bytes."""
    sp = GenSpec(layers, vocab, experts, int(embedding), int(head), seed, threads, mix, outliers)
    err = ctypes.create_string_buffer(512)
    size = u64()
    if not _h.qxgen_write(str(path).encode(), ctypes.byref(sp), ctypes.byref(size), err, 512):
        raise QxgError(err.value.decode())
    return size.value


def kvsnap_write(path, next_token, seed, k, v, ks, vs, positions):
    """QXKVSNP1 file from host caches k, v [layers, ctx, 512] int8 and ks, vs [layers, ctx] f32."""
    k, v = np.ascontiguousarray(k, np.int8), np.ascontiguousarray(v, np.int8)
    ks, vs = np.ascontiguousarray(ks, np.float32), np.ascontiguousarray(vs, np.float32)
    layers, ctx = ks.shape
    err = ctypes.create_string_buffer(512)
    if not _g.qxg_kvsnap_write(str(path).encode(), layers, positions, ctx, next_token, seed, _p(k), _p(v), _p(ks),
                               _p(vs), err, 512):
        raise QxgError(err.value.decode())


def kvsnap_read(path, layers, ctx, seed):
    """(k, v, ks, vs, positions, next_token) of a QXKVSNP1 file; rows past `positions` are zero."""
    k = np.zeros((layers, ctx, 512), np.int8); v = np.zeros_like(k)
    ks = np.zeros((layers, ctx), np.float32); vs = np.zeros_like(ks)
    pos, nt = u32(), u32()
    err = ctypes.create_string_buffer(512)
    if not _g.qxg_kvsnap_read(str(path).encode(), layers, ctx, seed, _p(k), _p(v), _p(ks), _p(vs), ctypes.byref(pos),
                              ctypes.byref(nt), err, 512):
        raise QxgError(err.value.decode())
    return k, v, ks, vs, pos.value, nt.value


class MemModel:
    """Seeded QXF1 model in an anonymous in-memory file (path /proc/self/fd/N)."""

    def __init__(self, layers=48, vocab=151936, experts=128, embedding=True, head=True, seed=1, threads=0, mix=0,
                 outliers=0):
        sp = GenSpec(layers, vocab, experts, int(embedding), int(head), seed, threads, mix, outliers)
        err = ctypes.create_string_buffer(512)
        path = ctypes.create_string_buffer(128)
        fd = c_int()
        if not _h.qxgen_memfd(ctypes.byref(sp), path, 128, ctypes.byref(fd), err, 512):
            raise QxgError(err.value.decode())
        self.path = path.value.decode()
        self.fd = fd.value

    def close(self):
        if self.fd >= 0:
            _h.qxgen_memfd_close(self.fd)
            self.fd = -1


class Context:
    """One qxg_ctx (one HIP stream) on `device`."""

    def __init__(self, device=0):
        self._c = vp()
        self._err = ctypes.create_string_buffer(1024)
        self._check(_g.qxg_open(device, ctypes.byref(self._c), self._err, 1024))
        self.info = None

    def _check(self, ok):
        if not ok:
            raise QxgError(self._err.value.decode())

    def close(self):
        if self._c:
            _g.qxg_close(self._c)
            self._c = vp()

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def load(self, path, verify=True):
        info = ModelInfo()
        self._check(_h.qx_gpu_load(self._c, str(path).encode(), int(verify), ctypes.byref(info), self._err, 1024))
        self.info = info
        return info

    def kv_create(self, layers, ctx_tokens):
        self._check(_g.qxg_kv_create(self._c, layers, ctx_tokens, 1, self._err, 1024))

    def kv_write(self, layer, pos0, k, v, ks, vs):
        k, v = np.ascontiguousarray(k, np.int8), np.ascontiguousarray(v, np.int8)
        ks, vs = np.ascontiguousarray(ks, np.float32), np.ascontiguousarray(vs, np.float32)
        self._check(_g.qxg_kv_write(self._c, layer, pos0, len(ks), _p(k), _p(v), _p(ks), _p(vs), self._err, 1024))

    def kv_read(self, layer, pos0, count):
        k = np.zeros((count, 512), np.int8); v = np.zeros((count, 512), np.int8)
        ks = np.zeros(count, np.float32); vs = np.zeros(count, np.float32)
        self._check(_g.qxg_kv_read(self._c, layer, pos0, count, _p(k), _p(v), _p(ks), _p(vs), self._err, 1024))
        return k, v, ks, vs

    def kv_export(self, path, layers, positions, ctx_tokens, next_token, seed):
        self._check(_g.qxg_kv_export(self._c, str(path).encode(), layers, positions, ctx_tokens, next_token, seed,
                                     self._err, 1024))

    def kv_import(self, path, layers, ctx_tokens, seed):
        """Returns (positions, next_token) of the snapshot written into the device cache."""
        pos, nt = u32(), u32()
        self._check(_g.qxg_kv_import(self._c, str(path).encode(), layers, ctx_tokens, seed, ctypes.byref(pos),
                                     ctypes.byref(nt), self._err, 1024))
        return pos.value, nt.value

    def dequant(self, ggml_type, raw, nblocks):
        raw = np.ascontiguousarray(raw, np.uint8)
        out = np.zeros(nblocks * 256, np.float32)
        self._check(_g.qxg_dequant_blocks(self._c, ggml_type, _p(raw), nblocks, _p(out), self._err, 1024))
        return out

    def int8_quantize(self, x):
        """The device KV quantizer on one row: (int8 codes, f32 scale)."""
        x = np.ascontiguousarray(x, np.float32)
        codes = np.zeros(len(x), np.int8)
        sc = np.zeros(1, np.float32)
        self._check(_g.qxg_int8_quantize(self._c, _p(x), len(x), _p(codes), _p(sc), self._err, 1024))
        return codes, sc[0]

    def dequant_static(self, ggml_type, raw_dev, nblocks, out_dev):
        """qxg_dequant_blocks_static on device addresses (ints) the caller owns."""
        self._check(_g.qxg_dequant_blocks_static(self._c, ggml_type, vp(raw_dev), nblocks, vp(out_dev), self._err, 1024))

    def embed(self, token):
        x = np.zeros(2048, np.float32)
        self._check(_g.qxg_embed_token(self._c, token, _p(x), self._err, 1024))
        return x

    def attention_layer(self, layer, pos, x):
        x = np.ascontiguousarray(x, np.float32)
        a = np.zeros(2048, np.float32); kqv = np.zeros(4096, np.float32); vcur = np.zeros(512, np.float32)
        self._check(_g.qxg_attention_layer(self._c, layer, pos, _p(x), _p(a), _p(kqv), _p(vcur), self._err, 1024))
        return a, kqv, vcur

    def attention_layer_sums(self, layer, pos, x):
        """attention_layer plus each q head's sum of normalised softmax weights (32)."""
        x = np.ascontiguousarray(x, np.float32)
        a = np.zeros(2048, np.float32); kqv = np.zeros(4096, np.float32); vcur = np.zeros(512, np.float32)
        hs = np.zeros(32, np.float64)
        self._check(_g.qxg_attention_layer_ex(self._c, layer, pos, _p(x), _p(a), _p(kqv), _p(vcur), _p(hs), self._err, 1024))
        return a, kqv, vcur, hs

    def attention_stage(self, layer, x, f16_kv=False):
        """(attn_norm, Vcur, kqv_out, attn_out, ffn_inp) of the single-token attention stage."""
        x = np.ascontiguousarray(x, np.float32)
        nrm = np.zeros(2048, np.float32); vc = np.zeros(512, np.float32); kqv = np.zeros(4096, np.float32)
        ao = np.zeros(2048, np.float32); fi = np.zeros(2048, np.float32)
        self._check(_g.qxg_attention_stage(self._c, layer, int(f16_kv), _p(x), _p(nrm), _p(vc), _p(kqv), _p(ao), _p(fi),
                                           self._err, 1024))
        return nrm, vc, kqv, ao, fi

    def moe_stage(self, layer, x):
        """(dict of the MoE stage's named vectors, ids[8]); names as the reference's sidecars."""
        x = np.ascontiguousarray(x, np.float32)
        E = self.info.experts
        blk = np.zeros(moe_stage_floats(E), np.float32); ids = np.zeros(8, np.uint32)
        self._check(_g.qxg_moe_stage(self._c, layer, _p(x), _p(blk), _p(ids), self._err, 1024))
        return split_moe_stage(blk, E), ids

    def moe_layer(self, layer, x):
        x = np.ascontiguousarray(x, np.float32)
        y = np.zeros(2048, np.float32); moe = np.zeros(2048, np.float32)
        ids = np.zeros(8, np.uint32); w = np.zeros(8, np.float64)
        self._check(_g.qxg_moe_layer(self._c, layer, _p(x), _p(y), _p(moe), _p(ids), _p(w), self._err, 1024))
        return y, moe, ids, w

    def final_head(self, residual, top_n=8):
        r = np.ascontiguousarray(residual, np.float32)
        nrm = np.zeros(2048, np.float32); lg = np.zeros(self.info.vocab, np.float32)
        ids = np.zeros(top_n, np.uint32); tl = np.zeros(top_n, np.float64)
        self._check(_g.qxg_final_head(self._c, _p(r), _p(nrm), _p(lg), top_n, _p(ids), _p(tl), self._err, 1024))
        return nrm, lg, ids, tl

    def decode_token(self, token, pos, run_head=True, top_n=8, want_layers=False, want_logits=False):
        res = np.zeros(2048, np.float32)
        lay = np.zeros((self.info.layers, 2048), np.float32) if want_layers else None
        lg = np.zeros(self.info.vocab, np.float32) if want_logits else None
        ids = np.zeros(top_n, np.uint32); tl = np.zeros(top_n, np.float64)
        self._check(_g.qxg_decode_token(self._c, token, pos, int(run_head), _p(res), _p(lay), _p(lg), top_n, _p(ids),
                                        _p(tl), self._err, 1024))
        return res, lay, lg, ids, tl

    def routing(self, layers=None):
        """(ids [layers, 8], weights [layers, 8]) of every layer in the last decode step."""
        n = self.info.layers if layers is None else layers
        ids = np.zeros((n, 8), np.uint32); w = np.zeros((n, 8), np.float64)
        self._check(_g.qxg_decode_routing(self._c, n, _p(ids), _p(w), self._err, 1024))
        return ids, w

    def generate(self, prompt, n_gen, pos0=0):
        prompt = np.ascontiguousarray(prompt, np.uint32)
        out = np.zeros(n_gen, np.uint32)
        ms = c_float()
        self._check(_g.qxg_generate(self._c, _p(prompt), len(prompt), n_gen, pos0, _p(out), ctypes.byref(ms),
                                    self._err, 1024))
        return out, ms.value

    def persistent_path(self):
        return bool(_g.qxg_persistent_path(self._c))

    def generate_recorded(self, prompt, n_gen, pos0=0, top_n=8):
        """qxg_generate with every step's records (one persistent launch): a dict of tokens
        [S+1], layer/attn/moe [S, layers, 2048], ids/weights [S, layers, 8], head_sums
        [S, layers, 32], norm [S, 2048], logits [S, vocab], top_ids/top_logits [S, top_n],
        step_ms [S+1] and elapsed_ms, with S = len(prompt) + n_gen - 1."""
        prompt = np.ascontiguousarray(prompt, np.uint32)
        S, L = len(prompt) + n_gen - 1, self.info.layers
        r = {"tokens": np.zeros(S + 1, np.uint32), "layer": np.zeros((S, L, 2048), np.float32),
             "attn": np.zeros((S, L, 2048), np.float32), "moe": np.zeros((S, L, 2048), np.float32),
             "ids": np.zeros((S, L, 8), np.uint32), "weights": np.zeros((S, L, 8), np.float64),
             "head_sums": np.zeros((S, L, 32), np.float64), "norm": np.zeros((S, 2048), np.float32),
             "logits": np.zeros((S, self.info.vocab), np.float32), "top_ids": np.zeros((S, top_n), np.uint32),
             "top_logits": np.zeros((S, top_n), np.float64), "step_ms": np.zeros(S + 1, np.float64)}
        ms = c_float()
        self._check(_g.qxg_generate_recorded(
            self._c, _p(prompt), len(prompt), n_gen, pos0, top_n, _p(r["tokens"]), _p(r["layer"]), _p(r["attn"]),
            _p(r["moe"]), _p(r["ids"]), _p(r["weights"]), _p(r["head_sums"]), _p(r["norm"]), _p(r["logits"]),
            _p(r["top_ids"]), _p(r["top_logits"]), _p(r["step_ms"]), ctypes.byref(ms), self._err, 1024))
        r["elapsed_ms"] = ms.value
        return r

    def prefill(self, tokens, pos0=0, run_head=True, top_n=8, want_residual=False, want_logits=False):
        """Batched prefill of `tokens` at positions pos0..; returns (residual [n, 2048] or
        None, logits of the last token or None, top ids, top logits, device ms)."""
        tokens = np.ascontiguousarray(tokens, np.uint32)
        n = len(tokens)
        res = np.zeros((n, 2048), np.float32) if want_residual else None
        lg = np.zeros(self.info.vocab, np.float32) if want_logits and run_head else None
        ids = np.zeros(top_n, np.uint32); tl = np.zeros(top_n, np.float64)
        ms = c_float()
        self._check(_g.qxg_prefill(self._c, _p(tokens), n, pos0, int(run_head), _p(res), _p(lg), top_n, _p(ids),
                                   _p(tl), ctypes.byref(ms), self._err, 1024))
        return res, lg, ids, tl, ms.value

    def prefill_layer(self, layer, pos0, x):
        """One prefill layer on the rows of x [n, 2048]: (ffn_inp, moe, out), each [n, 2048]."""
        x = np.ascontiguousarray(x, np.float32)
        n = x.shape[0]
        fi = np.zeros((n, 2048), np.float32); moe = np.zeros((n, 2048), np.float32); out = np.zeros((n, 2048), np.float32)
        self._check(_g.qxg_prefill_layer(self._c, layer, n, pos0, _p(x), _p(fi), _p(moe), _p(out), self._err, 1024))
        return fi, moe, out

    def halves(self, layers=None):
        """(attention outputs, MoE outputs) [layers, 2048] of the last decode_token step,
        each before its residual add."""
        n = self.info.layers if layers is None else layers
        a = np.zeros((n, 2048), np.float32)
        m = np.zeros((n, 2048), np.float32)
        self._check(_g.qxg_decode_halves(self._c, n, _p(a), _p(m), self._err, 1024))
        return a, m

    def head_sums(self, layers=None):
        """[layers, 32] each q head's sum of normalised attention weights, last decode_token step."""
        n = self.info.layers if layers is None else layers
        out = np.zeros((n, 32), np.float64)
        self._check(_g.qxg_decode_head_sums(self._c, n, _p(out), self._err, 1024))
        return out

    def final_norm(self):
        """The output-RMSNorm vector of the last decode_token head step."""
        out = np.zeros(2048, np.float32)
        self._check(_g.qxg_decode_final_norm(self._c, _p(out), self._err, 1024))
        return out

    def kv_read_position(self, pos, layers):
        """(k [layers, 512], v, ks [layers], vs) of one position."""
        k = np.zeros((layers, 512), np.int8); v = np.zeros_like(k)
        ks = np.zeros(layers, np.float32); vs = np.zeros_like(ks)
        self._check(_g.qxg_kv_read_position(self._c, pos, layers, _p(k), _p(v), _p(ks), _p(vs), self._err, 1024))
        return k, v, ks, vs

    def set_attention_chunks(self, min_positions):
        """Persistent decode: stage A by kv head and chunk from n = pos + 1 >= min_positions."""
        _g.qxg_set_attention_chunks(self._c, int(min_positions))

    def set_layer_path(self, persistent):
        """1: the persistent layer kernel (the default); 0: one kernel per phase."""
        self._check(_g.qxg_set_layer_path(self._c, int(persistent)))

    def set_activation(self, fmt):
        """"f32" (default) or "q8_k_compat" (Q8_K activations, integer dots)."""
        modes = {"f32": 0, "q8_k_compat": 1}
        if fmt not in modes:
            raise ValueError(f"unsupported activation format {fmt!r}")
        self._check(_g.qxg_set_activation(self._c, modes[fmt], self._err, 1024))

    def q8k_quantize(self, x):
        """Q8_K blocks (292 bytes each) of x on the device, as raw bytes."""
        x = np.ascontiguousarray(x, np.float32)
        out = np.zeros(292 * (len(x) // 256), np.uint8)
        self._check(_g.qxg_q8k_quantize(self._c, x.ctypes.data_as(vp), len(x), out.ctypes.data_as(vp), self._err, 1024))
        return out

    def time_kernel(self, which, layer=0, iters=20):
        ms = c_float()
        self._check(_g.qxg_time_kernel(self._c, which, layer, iters, ctypes.byref(ms), self._err, 1024))
        return ms.value

    def profile_kernel(self, which):
        _g.qxg_profile_kernel(self._c, which)

    def profile_result(self):
        n = u32(); ms = c_double()
        _g.qxg_profile_result(self._c, ctypes.byref(n), ctypes.byref(ms))
        return n.value, ms.value

    def device_bytes(self):
        return int(_g.qxg_device_bytes(self._c))


KERNELS = {"gate_up": 0, "down": 1, "qkv": 2, "oproj": 3, "head": 4, "attention": 5, "router": 6, "layers": 7,
           "pf_qkv": 8, "pf_oproj": 9, "pf_gate_up": 10, "pf_down": 11, "pf_router": 12, "pf_attn": 13}
