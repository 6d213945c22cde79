"""CPU oracle bindings — TEST INFRASTRUCTURE.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this package. It binds two libraries built by oracle/Makefile:

  liboracle.so       this repo's C restatement of the reference path
                     (nut_oracle.c)
  _ref/libnutref.so  the reference's own sources compiled in place with
                     ref_harness.cpp (present only where it was built)

The product (nutllm_amd) never imports it.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_PATH = os.path.join(_HERE, "liboracle.so")
REF_PATH = os.path.join(_HERE, "_ref", "libnutref.so")

PROJECTIONS = ("query", "key", "value", "output", "gate", "up", "down")


class OrcConfig(C.Structure):
    _fields_ = [(n, C.c_size_t) for n in (
        "layers", "heads", "dim", "head_dim", "ffn_dim", "vocab_size",
        "max_seq", "eos_token", "kv_heads")]


class OrcQMat(C.Structure):
    _fields_ = [("data", C.c_void_p), ("scales", C.c_void_p),
                ("rows", C.c_size_t), ("cols", C.c_size_t),
                ("block_size", C.c_size_t), ("type", C.c_int)]


class OrcLayer(C.Structure):
    _fields_ = [(n, OrcQMat) for n in PROJECTIONS] + [
        ("attention_norm", C.c_void_p), ("ffn_norm", C.c_void_p)]


class OrcModel(C.Structure):
    _fields_ = [("config", OrcConfig), ("embeddings", C.c_void_p),
                ("final_norm", C.c_void_p), ("output_weights", C.c_void_p),
                ("layers", C.c_void_p)]


_P, _SZ = C.c_void_p, C.c_size_t
_ORC = {
    "orc_float_to_half": (C.c_int, [C.c_float, _P]),
    "orc_half_to_float": (C.c_float, [C.c_uint16]),
    "orc_quantize": (C.c_int, [_P, _SZ, _SZ, C.c_int, _SZ, _P, _P]),
    "orc_storage_bytes": (_SZ, [_SZ, _SZ, C.c_int, _SZ]),
    "orc_error_bound": (C.c_float, [_P, _SZ, _SZ]),
    "orc_dequantize": (None, [_P, _P]),
    "orc_matvec_q": (C.c_int, [_P, _P, _P]),
    "orc_matvec_f32": (C.c_int, [_P, _SZ, _SZ, _P, _P]),
    "orc_matmul": (C.c_int, [_P, _P, _P, _SZ, _SZ, _SZ]),
    "orc_rmsnorm": (C.c_int, [_P, _P, _P, _SZ, C.c_float]),
    "orc_silu": (C.c_float, [C.c_float]),
    "orc_rotate": (None, [_P, _SZ, _SZ]),
    "orc_config_valid": (C.c_int, [_P]),
    "orc_kv_elements": (_SZ, [_P]),
    "orc_decode": (C.c_int, [_P, _P, _P, _P, C.c_int, _P]),
    "orc_prefill": (C.c_int, [_P, _P, _P, _P, _P, _SZ, _P]),
    "orc_logits": (C.c_int, [_P, _P, _P]),
    "orc_argmax": (_SZ, [_P, _SZ]),
    "orc_generate": (C.c_int, [_P, _P, _SZ, _SZ, _P, _P, _P, _P]),
    "orc_set_threads": (None, [C.c_int]),
    "orc_get_threads": (C.c_int, []),
}
_REF = {
    "ref_quantize": (C.c_int, [_P, _SZ, _SZ, C.c_int, _SZ, _P, _P, _P, _P]),
    "ref_matvec_q": (C.c_int, [_P, _SZ, _SZ, C.c_int, _SZ, _P, _P, _SZ]),
    "ref_matvec_f32": (C.c_int, [_P, _SZ, _SZ, _P, _P, _SZ]),
    "ref_matmul": (C.c_int, [_P, _P, _P, _SZ, _SZ, _SZ, _SZ]),
    "ref_matmul_time": (C.c_int, [_P, _P, _SZ, _SZ, _SZ, _SZ, _SZ, _P]),
    "ref_rmsnorm": (C.c_int, [_P, _P, _P, _SZ, C.c_float]),
    "ref_silu": (C.c_float, [C.c_float]),
    "ref_model_create": (C.c_int, [_P, C.c_int, C.c_int, _P, _P, _P, _P]),
    "ref_model_add_layer": (C.c_int, [_P] * 10),
    "ref_model_add_layer_quantized": (C.c_int, [_P] * 5),
    "ref_model_free": (None, [_P]),
    "ref_model_storage_bytes": (_SZ, [_P]),
    "ref_decode_trace": (C.c_int, [_P, _P, _SZ, _SZ, _P, _P, _P]),
    "ref_logits": (C.c_int, [_P, _P, _P, _SZ]),
    "ref_generate": (C.c_int, [_P, _P, _SZ, _SZ, _SZ, _P, _P, _P, _P]),
    "ref_fmodel_create": (C.c_int, [_P, C.c_int, _P, _P, _P, _P]),
    "ref_fmodel_add_layer": (C.c_int, [_P] * 10),
    "ref_fmodel_free": (None, [_P]),
    "ref_fmodel_run": (C.c_int, [_P, _P, _SZ, _P, _SZ, _SZ, _P, _P, _P, _P]),
    "ref_matvec_q_time": (C.c_int, [_P, _SZ, _SZ, C.c_int, _P, _SZ, _SZ, _P]),
    "ref_decode_time": (C.c_int, [_P, _SZ, _P, _SZ, _SZ, _P]),
    "ref_generate_sampled": (C.c_int, [_P, _P, _SZ, _SZ, _SZ, C.c_float, C.c_float,
                                       C.c_uint, _P, _P]),
}

_orc = None
_ref = None


def _bind(path, sigs):
    h = C.CDLL(path)
    for name, (res, args) in sigs.items():
        fn = getattr(h, name)
        fn.restype = res
        fn.argtypes = args
    return h


def orc():
    global _orc
    if _orc is None:
        if not os.path.exists(ORACLE_PATH):
            raise RuntimeError(f"{ORACLE_PATH} not built (make -C oracle)")
        _orc = _bind(ORACLE_PATH, _ORC)
    return _orc


def ref_available():
    return os.path.exists(REF_PATH)


def ref():
    global _ref
    if _ref is None:
        if not ref_available():
            raise RuntimeError(f"{REF_PATH} not built (make -C oracle ref)")
        _ref = _bind(REF_PATH, _REF)
    return _ref


def ptr(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def check(status, what="oracle"):
    if status != 0:
        raise RuntimeError(f"{what}: status {status}")


# ------------------------------------------------------- oracle helpers --

def quantize(w, qtype, block_size=32):
    w = np.ascontiguousarray(w, np.float32)
    rows, cols = w.shape
    n = rows * cols
    data = np.zeros(n if qtype == 0 else (n + 1) // 2, np.uint8)
    scales = np.zeros(max(1, -(-n // block_size)) if block_size else 1,
                      np.uint16)
    st = orc().orc_quantize(ptr(w), rows, cols, qtype, block_size, ptr(data),
                            ptr(scales))
    return st, data, scales


def qmat(data, scales, rows, cols, qtype, block_size=32):
    return OrcQMat(data.ctypes.data, scales.ctypes.data, rows, cols,
                   block_size, qtype)


def matvec_q(data, scales, rows, cols, qtype, x, block_size=32):
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty(rows, np.float32)
    q = qmat(data, scales, rows, cols, qtype, block_size)
    check(orc().orc_matvec_q(C.byref(q), ptr(x), ptr(y)))
    return y


def dequantize(data, scales, rows, cols, qtype, block_size=32):
    out = np.empty((rows, cols), np.float32)
    q = qmat(data, scales, rows, cols, qtype, block_size)
    orc().orc_dequantize(C.byref(q), ptr(out))
    return out


class OracleModel:
    """orc_model over host arrays of a synthetic model (keeps them alive)."""

    def __init__(self, cfg_dict, qtype, embeddings, final_norm, output_weights,
                 layers, norms=None):
        self.cfg = OrcConfig(**cfg_dict)
        self.keep = [embeddings, final_norm, output_weights]
        n = cfg_dict["layers"]
        arr = (OrcLayer * n)()
        for i, mats in enumerate(layers):
            fields = {}
            for name in PROJECTIONS:
                data, scales, rows, cols, *bs = mats[name]
                self.keep += [data, scales]
                fields[name] = qmat(data, scales, rows, cols, qtype,
                                    bs[0] if bs else 32)
            an, fn = (norms[i] if norms else
                      (np.ones(cfg_dict["dim"], np.float32),) * 2)
            self.keep += [an, fn]
            arr[i] = OrcLayer(**fields, attention_norm=an.ctypes.data,
                              ffn_norm=fn.ctypes.data)
        self.layers = arr
        self.model = OrcModel(self.cfg, embeddings.ctypes.data,
                              final_norm.ctypes.data,
                              output_weights.ctypes.data,
                              C.cast(arr, C.c_void_p))
        kv = orc().orc_kv_elements(C.byref(self.cfg))
        self.keys = np.zeros(kv, np.float32)
        self.values = np.zeros(kv, np.float32)
        self.length = C.c_size_t(0)

    def reset(self):
        self.length.value = 0

    def decode(self, token):
        h = np.empty(self.cfg.dim, np.float32)
        check(orc().orc_decode(C.byref(self.model), ptr(self.keys),
                               ptr(self.values), C.byref(self.length),
                               int(token), ptr(h)), "orc_decode")
        return h

    def prefill(self, tokens):
        t = np.ascontiguousarray(tokens, np.int32)
        h = np.empty(self.cfg.dim, np.float32)
        check(orc().orc_prefill(C.byref(self.model), ptr(self.keys),
                                ptr(self.values), C.byref(self.length),
                                ptr(t), t.size, ptr(h)), "orc_prefill")
        return h

    def logits(self, hidden):
        h = np.ascontiguousarray(hidden, np.float32)
        out = np.empty(self.cfg.vocab_size, np.float32)
        check(orc().orc_logits(C.byref(self.model), ptr(h), ptr(out)))
        return out

    def generate(self, prompt, max_tokens):
        p = np.ascontiguousarray(prompt, np.int32)
        out = np.empty(max(1, max_tokens), np.int32)
        count = C.c_size_t()
        pre, dec = C.c_double(), C.c_double()
        check(orc().orc_generate(C.byref(self.model), ptr(p), p.size,
                                 max_tokens, ptr(out), C.byref(count),
                                 C.byref(pre), C.byref(dec)), "orc_generate")
        return out[:count.value].tolist(), pre.value, dec.value

    def kv_row(self, layer, head, position):
        c = self.cfg
        kvh = c.kv_heads or c.heads
        o = ((layer * kvh + head) * c.max_seq + position) * c.head_dim
        return (self.keys[o:o + c.head_dim].copy(),
                self.values[o:o + c.head_dim].copy())


def oracle_model(synth):
    """OracleModel over a nutllm_amd.workloads.SynthModel's arrays."""
    cfg = {n: getattr(synth.config, n) for n, _ in OrcConfig._fields_}
    return OracleModel(cfg, synth.qtype, synth.embeddings, synth.final_norm,
                       synth.lm_head, synth.layers,
                       getattr(synth, "norms", None))


class RefModel:
    """The compiled reference's QuantizedModelWeights (quantises fp32)."""

    def __init__(self, cfg_dict, qtype, embeddings, final_norm, lm_head,
                 fp32_layers, norms=None):
        cfg = (C.c_size_t * 9)(*[cfg_dict[n] for n, _ in OrcConfig._fields_])
        h = C.c_void_p()
        check(ref().ref_model_create(cfg, qtype, 0, ptr(embeddings),
                                     ptr(final_norm), ptr(lm_head),
                                     C.byref(h)), "ref_model_create")
        self.handle = h
        self.dim = cfg_dict["dim"]
        self.vocab = cfg_dict["vocab_size"]
        ones = np.ones(self.dim, np.float32)
        for i, w in enumerate(fp32_layers):
            an, fn = norms[i] if norms else (ones, ones)
            check(ref().ref_model_add_layer(
                self.handle, *[ptr(np.ascontiguousarray(w[n], np.float32))
                               for n in PROJECTIONS], ptr(an), ptr(fn)),
                "ref_model_add_layer")

    @classmethod
    def from_quantized(cls, synth):
        """Reference model over a SynthModel's quantised storage (its
        quantiser is bit-identical to the reference's)."""
        self = cls.__new__(cls)
        c = synth.config
        cfg_dict = {n: getattr(c, n) for n, _ in OrcConfig._fields_}
        cfg = (C.c_size_t * 9)(*[cfg_dict[n] for n, _ in OrcConfig._fields_])
        h = C.c_void_p()
        check(ref().ref_model_create(cfg, synth.qtype, 0,
                                     ptr(synth.embeddings),
                                     ptr(synth.final_norm),
                                     ptr(synth.lm_head), C.byref(h)),
              "ref_model_create")
        self.handle = h
        self.dim = c.dim
        self.vocab = c.vocab_size
        ones = np.ones(c.dim, np.float32)
        norms = getattr(synth, "norms", None)
        for i, mats in enumerate(synth.layers):
            data = (C.c_void_p * 7)(*[mats[n][0].ctypes.data
                                      for n in PROJECTIONS])
            scales = (C.c_void_p * 7)(*[mats[n][1].ctypes.data
                                        for n in PROJECTIONS])
            an, fn = norms[i] if norms else (ones, ones)
            check(ref().ref_model_add_layer_quantized(self.handle, data,
                                                      scales, ptr(an),
                                                      ptr(fn)),
                  "ref_model_add_layer_quantized")
        return self

    def decode_trace(self, tokens, threads=1, kv_elements=None):
        t = np.ascontiguousarray(tokens, np.int32)
        hidden = np.empty((t.size, self.dim), np.float32)
        keys = values = None
        if kv_elements:
            keys = np.zeros(kv_elements, np.float32)
            values = np.zeros(kv_elements, np.float32)
        check(ref().ref_decode_trace(self.handle, ptr(t), t.size, threads,
                                     ptr(hidden), ptr(keys), ptr(values)),
              "ref_decode_trace")
        return hidden, keys, values

    def logits(self, hidden, threads=1):
        out = np.empty(self.vocab, np.float32)
        check(ref().ref_logits(self.handle, ptr(np.ascontiguousarray(
            hidden, np.float32)), ptr(out), threads), "ref_logits")
        return out

    def generate(self, prompt, max_tokens, threads=1):
        p = np.ascontiguousarray(prompt, np.int32)
        out = np.empty(max(1, max_tokens), np.int32)
        count = C.c_size_t()
        pre, dec = C.c_double(), C.c_double()
        check(ref().ref_generate(self.handle, ptr(p), p.size, max_tokens,
                                 threads, ptr(out), C.byref(count),
                                 C.byref(pre), C.byref(dec)), "ref_generate")
        return out[:count.value].tolist(), pre.value, dec.value

    def generate_sampled(self, prompt, max_tokens, temperature, top_p, seed,
                         threads=1):
        p = np.ascontiguousarray(prompt, np.int32)
        out = np.empty(max(1, max_tokens), np.int32)
        count = C.c_size_t()
        check(ref().ref_generate_sampled(self.handle, ptr(p), p.size, max_tokens,
                                         threads, temperature, top_p, seed,
                                         ptr(out), C.byref(count)),
              "ref_generate_sampled")
        return out[:count.value].tolist()

    def decode_time(self, start_length, tokens, threads):
        """Seconds of len(tokens) decode-loop steps from start_length."""
        t = np.ascontiguousarray(tokens, np.int32)
        sec = C.c_double()
        check(ref().ref_decode_time(self.handle, start_length, ptr(t), t.size,
                                    threads, C.byref(sec)), "ref_decode_time")
        return sec.value

    def storage_bytes(self):
        return ref().ref_model_storage_bytes(self.handle)

    def close(self):
        if self.handle:
            ref().ref_model_free(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
