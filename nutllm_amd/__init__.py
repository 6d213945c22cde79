"""nutllm_amd — MI355X (gfx950) token loop of nutllm behind a C ABI.

This module binds ``lib/libnutllm_hip.so`` (declared in
``include/nutllm_hip.h``) with ctypes and mirrors the reference's C++ entry
points for Python callers: ``QuantizedMatrix.quantize`` (src/quant.cpp:154),
``matvec_quantized`` (src/quant.cpp:262), ``decode_quantized_token`` /
``prefill_quantized`` (src/quant_model.cpp:158-220), ``KVCache``
(include/kvcache.hpp:8-31) and ``generate_tokens_cached``
(src/generate.cpp:174-216). Errors raise the Python counterpart of the C++
exception the reference throws, with the same message.

There is no CPU fallback: if the library is missing or no gfx950 device is
present, calls that need the GPU raise ``DeviceError``.
"""
from __future__ import annotations

import ctypes as C
import os
from dataclasses import dataclass

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "lib", "libnutllm_hip.so")

INT8, INT4 = 0, 1
PATH_AUTO, PATH_STEPS, PATH_TOKEN = 0, 1, 2


class NutError(Exception):
    """Base of the errors raised through the C ABI."""


class InvalidArgument(NutError, ValueError):
    """std::invalid_argument."""


class OutOfRange(NutError, IndexError):
    """std::out_of_range."""


class LengthError(NutError, ValueError):
    """std::length_error."""


class RangeError(NutError, ArithmeticError):
    """std::range_error."""


class DeviceError(NutError, RuntimeError):
    """HIP runtime error or no gfx950 device."""


_ERRORS = {1: InvalidArgument, 2: OutOfRange, 3: LengthError, 4: RangeError,
           5: NutError, 6: DeviceError}


class Config(C.Structure):
    """ModelConfig (include/model.hpp:8-24)."""

    _fields_ = [(n, C.c_size_t) for n in (
        "layers", "heads", "dim", "head_dim", "ffn_dim", "vocab_size",
        "max_seq", "eos_token", "kv_heads")]

    def as_dict(self):
        return {n: getattr(self, n) for n, _ in self._fields_}

    @property
    def kv_dim(self):
        return (self.kv_heads or self.heads) * self.head_dim


class QMatrix(C.Structure):
    _fields_ = [("data", C.c_void_p), ("scales", C.c_void_p),
                ("rows", C.c_size_t), ("cols", C.c_size_t),
                ("block_size", C.c_size_t), ("type", C.c_int)]


class GenerationStats(C.Structure):
    """GenerationStats (include/generate.hpp:19-24)."""

    _fields_ = [("prefill_tokens", C.c_size_t),
                ("generated_tokens", C.c_size_t),
                ("prefill_seconds", C.c_double),
                ("decode_seconds", C.c_double)]


_lib = None

_P = C.c_void_p
_SZ = C.c_size_t
_SIGS = {
    "nut_last_error": (C.c_char_p, []),
    "nut_quantize": (C.c_int, [_P, _SZ, _SZ, C.c_int, _SZ, _P, _P]),
    "nut_quant_data_bytes": (_SZ, [_SZ, _SZ, C.c_int]),
    "nut_quant_scale_count": (_SZ, [_SZ, _SZ, _SZ]),
    "nut_quant_storage_bytes": (_SZ, [_SZ, _SZ, C.c_int, _SZ]),
    "nut_float_to_half": (C.c_int, [C.c_float, _P]),
    "nut_half_to_float": (C.c_float, [C.c_uint16]),
    "nut_config_valid": (C.c_int, [_P]),
    "nut_synth_normal": (C.c_int, [C.c_uint64, C.c_uint64, C.c_float, _P, _SZ]),
    "nut_synth_tokens": (C.c_int, [C.c_uint64, _SZ, _P, _SZ]),
    "nut_device_count": (C.c_int, [_P]),
    "nut_set_device": (C.c_int, [C.c_int]),
    "nut_malloc": (C.c_int, [_P, _SZ]),
    "nut_free": (C.c_int, [_P]),
    "nut_device_allocations": (C.c_int, [_P]),
    "nut_memcpy_h2d": (C.c_int, [_P, _P, _SZ]),
    "nut_memcpy_d2h": (C.c_int, [_P, _P, _SZ]),
    "nut_memcpy_d2d": (C.c_int, [_P, _P, _SZ]),
    "nut_memset": (C.c_int, [_P, C.c_int, _SZ]),
    "nut_synchronize": (C.c_int, []),
    "nut_qweight_create": (C.c_int, [_P, _P]),
    "nut_qweight_destroy": (C.c_int, [_P]),
    "nut_qweight_device_bytes": (_SZ, [_P]),
    "nut_matvec_q": (C.c_int, [_P, _P, _P, _P]),
    "nut_matvec_f32": (C.c_int, [_P, _SZ, _SZ, _P, _P, _P]),
    "nut_matmul_f32": (C.c_int, [_P, _P, _P, _SZ, _SZ, _SZ, _P]),
    "nut_timer_begin": (C.c_int, [_P]),
    "nut_timer_end": (C.c_int, [_P, _P]),
    "nut_model_create": (C.c_int, [_P, C.c_int, C.c_int, _P]),
    "nut_model_set_globals": (C.c_int, [_P, _P, _P, _P]),
    "nut_model_set_layer": (C.c_int, [_P, _SZ] + [_P] * 9),
    "nut_model_storage_bytes": (_SZ, [_P]),
    "nut_model_last_decode_ms": (C.c_int, [_P, _P]),
    "nut_model_set_path": (C.c_int, [_P, C.c_int]),
    "nut_model_record_timeline": (C.c_int, [_P, C.c_int]),
    "nut_model_timeline": (C.c_int, [_P, _P, _SZ, _P]),
    "nut_model_destroy": (C.c_int, [_P]),
    "nut_token_tag_base": (C.c_int, [_P, _P, _P]),
    "nut_model_load_llama2c": (C.c_int, [C.c_char_p, C.c_int, _P, _P]),
    "nut_model_config": (C.c_int, [_P, _P, _P, _P]),
    "nut_model_set_launch_count": (C.c_int, [_P, C.c_uint]),
    "nut_model_inject_fault": (C.c_int, [_P, C.c_int]),
    "nut_kv_create": (C.c_int, [_P, _P]),
    "nut_kv_destroy": (C.c_int, [_P]),
    "nut_kv_length": (_SZ, [_P]),
    "nut_kv_capacity": (_SZ, [_P]),
    "nut_kv_memory_bytes": (_SZ, [_P]),
    "nut_kv_compatible": (C.c_int, [_P, _P]),
    "nut_kv_reset": (C.c_int, [_P]),
    "nut_kv_set_length": (C.c_int, [_P, _SZ]),
    "nut_kv_read": (C.c_int, [_P, _SZ, _SZ, _SZ, _P, _P]),
    "nut_kv_store": (C.c_int, [_P, _SZ, _SZ, _P, _P]),
    "nut_decode": (C.c_int, [_P, _P, C.c_int, _P]),
    "nut_decode_noalloc": (C.c_int, [_P, _P, C.c_int, _P]),
    "nut_prefill": (C.c_int, [_P, _P, _P, _SZ, _P]),
    "nut_logits": (C.c_int, [_P, _P, _P]),
    "nut_generate_greedy": (C.c_int, [_P, _P, _SZ, _SZ, _P, _P, _P]),
    "nut_fmodel_create": (C.c_int, [_P, C.c_int, _P]),
    "nut_fmodel_set_globals": (C.c_int, [_P, _P, _P, _P]),
    "nut_fmodel_set_layer": (C.c_int, [_P, _SZ] + [_P] * 9),
    "nut_fmodel_destroy": (C.c_int, [_P]),
    "nut_decode_token": (C.c_int, [_P, _P, C.c_int, _P]),
    "nut_prefill_tokens": (C.c_int, [_P, _P, _P, _SZ, _P]),
    "nut_generate_sampled": (C.c_int, [_P, _P, _SZ, _SZ, C.c_float, C.c_float,
                                       C.c_uint32, _P, _P, _P]),
    "nut_kv_read_positions": (C.c_int, [_P, _SZ, _SZ, _P, _P]),
    "nut_kv_write_positions": (C.c_int, [_P, _SZ, _SZ, _P, _P]),
}


def exported_symbols():
    """Every C entry point this binding expects the library to export."""
    return sorted(_SIGS)


def lib():
    """Load the C-ABI library (raises DeviceError when it is not built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise DeviceError(
                f"{LIB_PATH} is not built; run __graft_entry__.build()")
        handle = C.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def check(status):
    if status != 0:
        msg = lib().nut_last_error().decode()
        raise _ERRORS.get(status, NutError)(msg)


def _ptr(a):
    return a.ctypes.data_as(C.c_void_p) if a is not None else None


# ------------------------------------------------------------- host utils --

def quantize(weights, qtype, block_size=32):
    """QuantizedMatrix::quantize: returns (data uint8, scales uint16)."""
    w = np.ascontiguousarray(weights, dtype=np.float32)
    rows, cols = w.shape
    L = lib()
    data = np.zeros(L.nut_quant_data_bytes(rows, cols, qtype), np.uint8)
    scales = np.zeros(L.nut_quant_scale_count(rows, cols, block_size),
                      np.uint16)
    check(L.nut_quantize(_ptr(w), rows, cols, qtype, block_size, _ptr(data),
                         _ptr(scales)))
    return data, scales


def float_to_half(value):
    bits = C.c_uint16()
    check(lib().nut_float_to_half(C.c_float(value), C.byref(bits)))
    return bits.value


def half_to_float(bits):
    return lib().nut_half_to_float(bits)


def synth_normal(seed, stream, count, sigma=0.02):
    out = np.empty(count, np.float32)
    check(lib().nut_synth_normal(seed, stream, sigma, _ptr(out), count))
    return out


def synth_tokens(seed, vocab, count):
    out = np.empty(count, np.int32)
    check(lib().nut_synth_tokens(seed, vocab, _ptr(out), count))
    return out


def token_tag_base(launch_count):
    """Next exchange-tag base after launch_count: (base, new count, clear)."""
    count = C.c_uint(launch_count)
    base = C.c_uint()
    clear = C.c_int()
    check(lib().nut_token_tag_base(C.byref(count), C.byref(base),
                                   C.byref(clear)))
    return base.value, count.value, bool(clear.value)


# ---------------------------------------------------------------- device --

def device_allocations():
    """hipMalloc calls the library has made since it was loaded."""
    n = C.c_ulonglong(0)
    check(lib().nut_device_allocations(C.byref(n)))
    return n.value


def device_count():
    n = C.c_int(0)
    check(lib().nut_device_count(C.byref(n)))
    return n.value


class DeviceArray:
    """A device buffer holding a numpy array's bytes (freed on close)."""

    def __init__(self, nbytes=None, like=None):
        if like is not None:
            like = np.ascontiguousarray(like)
            nbytes = like.nbytes
        self.nbytes = int(nbytes)
        p = C.c_void_p()
        check(lib().nut_malloc(C.byref(p), self.nbytes))
        self.ptr = p
        if like is not None:
            self.upload(like)

    def upload(self, array):
        a = np.ascontiguousarray(array)
        assert a.nbytes <= self.nbytes
        check(lib().nut_memcpy_h2d(self.ptr, _ptr(a), a.nbytes))

    def download(self, dtype, count):
        out = np.empty(count, dtype)
        assert out.nbytes <= self.nbytes
        check(lib().nut_memcpy_d2h(_ptr(out), self.ptr, out.nbytes))
        return out

    def close(self):
        if self.ptr:
            check(lib().nut_free(self.ptr))
            self.ptr = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def synchronize():
    check(lib().nut_synchronize())


def _qmatrix(data, scales, rows, cols, qtype, block_size=32):
    return QMatrix(data.ctypes.data, scales.ctypes.data, rows, cols,
                   block_size, qtype)


class QWeight:
    """A QuantizedMatrix resident in HBM for the standalone matvec."""

    def __init__(self, data, scales, rows, cols, qtype, block_size=32):
        self._keep = (np.ascontiguousarray(data), np.ascontiguousarray(scales))
        q = _qmatrix(self._keep[0], self._keep[1], rows, cols, qtype,
                     block_size)
        h = C.c_void_p()
        check(lib().nut_qweight_create(C.byref(q), C.byref(h)))
        self.handle = h
        self.rows, self.cols, self.qtype = rows, cols, qtype
        self.device_bytes = lib().nut_qweight_device_bytes(h)
        self._keep = None

    def matvec(self, d_x, d_y, stream=None):
        check(lib().nut_matvec_q(self.handle, d_x.ptr, d_y.ptr, stream))

    def close(self):
        if self.handle:
            check(lib().nut_qweight_destroy(self.handle))
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def matvec_quantized(data, scales, rows, cols, qtype, x, block_size=32):
    """matvec_quantized (src/quant.cpp:257-321) on the GPU; host in/out."""
    w = QWeight(data, scales, rows, cols, qtype, block_size)
    dx = DeviceArray(like=np.asarray(x, np.float32))
    dy = DeviceArray(4 * rows)
    w.matvec(dx, dy)
    y = dy.download(np.float32, rows)
    w.close(), dx.close(), dy.close()
    return y


def matvec_f32(weights, x):
    """matvec_threaded (src/threading.cpp:183-198) on the GPU."""
    w = np.ascontiguousarray(weights, np.float32)
    rows, cols = w.shape
    dw, dx, dy = DeviceArray(like=w), DeviceArray(like=np.asarray(x, np.float32)), DeviceArray(4 * rows)
    check(lib().nut_matvec_f32(dw.ptr, rows, cols, dx.ptr, dy.ptr, None))
    y = dy.download(np.float32, rows)
    dw.close(), dx.close(), dy.close()
    return y


def matmul_f32(a, b):
    """matmul_threaded (src/threading.cpp:163-181) on the GPU."""
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    m, k = a.shape
    k2, n = b.shape
    assert k == k2
    da, db, dc = DeviceArray(like=a), DeviceArray(like=b), DeviceArray(4 * m * n)
    check(lib().nut_matmul_f32(da.ptr, db.ptr, dc.ptr, m, k, n, None))
    c = dc.download(np.float32, m * n).reshape(m, n)
    da.close(), db.close(), dc.close()
    return c


class Timer:
    """HIP-event timer on a stream (None = null stream)."""

    def __init__(self, stream=None):
        self.stream = stream

    def begin(self):
        check(lib().nut_timer_begin(self.stream))

    def end(self):
        ms = C.c_double()
        check(lib().nut_timer_end(self.stream, C.byref(ms)))
        return ms.value


# ----------------------------------------------------------------- model --

PROJECTIONS = ("query", "key", "value", "output", "gate", "up", "down")


def projection_shapes(cfg):
    """[out x in] shapes of a layer's projections (src/llama2.cpp:374-396)."""
    d, f, kv = cfg.dim, cfg.ffn_dim, cfg.kv_dim
    return {"query": (d, d), "key": (kv, d), "value": (kv, d),
            "output": (d, d), "gate": (f, d), "up": (f, d), "down": (d, f)}


class KVCache:
    """KVCache (include/kvcache.hpp:8-31) resident in HBM."""

    def __init__(self, config):
        self.config = config
        h = C.c_void_p()
        check(lib().nut_kv_create(C.byref(config), C.byref(h)))
        self.handle = h

    def length(self):
        return lib().nut_kv_length(self.handle)

    def capacity(self):
        return lib().nut_kv_capacity(self.handle)

    def memory_bytes(self):
        return lib().nut_kv_memory_bytes(self.handle)

    def compatible(self, config):
        return bool(lib().nut_kv_compatible(self.handle, C.byref(config)))

    def reset(self):
        check(lib().nut_kv_reset(self.handle))

    def set_length(self, n):
        check(lib().nut_kv_set_length(self.handle, n))

    def key_value(self, layer, head, position):
        hd = self.config.head_dim
        k = np.empty(hd, np.float32)
        v = np.empty(hd, np.float32)
        check(lib().nut_kv_read(self.handle, layer, head, position, _ptr(k),
                                _ptr(v)))
        return k, v

    def read_positions(self, begin, end):
        """K and V rows of positions [begin, end): [layer][kv_head][n][hd]."""
        c = self.config
        shape = (c.layers, c.kv_heads or c.heads, end - begin, c.head_dim)
        k = np.empty(shape, np.float32)
        v = np.empty(shape, np.float32)
        check(lib().nut_kv_read_positions(self.handle, begin, end, _ptr(k), _ptr(v)))
        return k, v

    def write_positions(self, begin, keys, values):
        k = np.ascontiguousarray(keys, np.float32)
        v = np.ascontiguousarray(values, np.float32)
        check(lib().nut_kv_write_positions(self.handle, begin, begin + k.shape[2],
                                           _ptr(k), _ptr(v)))

    def store(self, layer, position, key, value):
        k = np.ascontiguousarray(key, np.float32)
        v = np.ascontiguousarray(value, np.float32)
        check(lib().nut_kv_store(self.handle, layer, position, _ptr(k),
                                 _ptr(v)))

    def close(self):
        if self.handle:
            check(lib().nut_kv_destroy(self.handle))
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class DeviceModel:
    """QuantizedModelWeights resident in HBM plus its token loop."""

    def __init__(self, config, qtype, tied=False, _handle=None):
        self.config = config
        self.qtype = qtype
        if _handle is not None:
            self.handle = _handle
            return
        h = C.c_void_p()
        check(lib().nut_model_create(C.byref(config), qtype, int(tied),
                                     C.byref(h)))
        self.handle = h

    @classmethod
    def load_llama2c(cls, path, qtype):
        """load_llama2c_quantized_model into HBM: (model, load seconds)."""
        h = C.c_void_p()
        seconds = C.c_double()
        check(lib().nut_model_load_llama2c(os.fsencode(path), qtype,
                                           C.byref(h), C.byref(seconds)))
        cfg = Config()
        check(lib().nut_model_config(h, C.byref(cfg), None, None))
        return cls(cfg, qtype, _handle=h), seconds.value

    def set_globals(self, embeddings, final_norm, lm_head=None):
        e = np.ascontiguousarray(embeddings, np.float32)
        n = np.ascontiguousarray(final_norm, np.float32)
        l = None if lm_head is None else np.ascontiguousarray(lm_head,
                                                              np.float32)
        check(lib().nut_model_set_globals(self.handle, _ptr(e), _ptr(n),
                                          _ptr(l)))

    def set_layer(self, index, mats, attention_norm, ffn_norm):
        """mats: name -> (data, scales, rows, cols[, block_size])."""
        qs = []
        for name in PROJECTIONS:
            data, scales, rows, cols, *bs = mats[name]
            qs.append(_qmatrix(np.ascontiguousarray(data),
                               np.ascontiguousarray(scales), rows, cols,
                               self.qtype, bs[0] if bs else 32))
        an = np.ascontiguousarray(attention_norm, np.float32)
        fn = np.ascontiguousarray(ffn_norm, np.float32)
        check(lib().nut_model_set_layer(self.handle, index,
                                        *[C.byref(q) for q in qs], _ptr(an),
                                        _ptr(fn)))

    def storage_bytes(self):
        return lib().nut_model_storage_bytes(self.handle)

    def set_path(self, path):
        """0 auto, 1 per-phase step kernels, 2 cooperative token kernel."""
        check(lib().nut_model_set_path(self.handle, path))

    def record_timeline(self, mode=1):
        """0 off, 1 workgroup 0 (True), 2 every workgroup."""
        check(lib().nut_model_record_timeline(self.handle, int(mode)))
        self._timeline_wgs = {0: 0, 1: 1, 2: 256}[int(mode)]

    def timeline(self, iterations):
        """Phase timeline of the last token-kernel launch, in microseconds
        from workgroup 0's first mark: array [iterations, 4 + 13 * layers],
        or [workgroups, iterations, marks] when every workgroup records."""
        marks = 4 + 13 * self.config.layers
        wgs = getattr(self, "_timeline_wgs", 1)
        per = self.config.max_seq * marks
        out = np.zeros(max(wgs, 1) * per, np.uint64)
        n = C.c_size_t()
        check(lib().nut_model_timeline(self.handle, _ptr(out), out.size,
                                       C.byref(n)))
        t = out[:n.value].astype(np.float64).reshape(-1, self.config.max_seq, marks)
        t = t[:, :iterations]
        t = (t - t[0, 0, 0]) / 100.0  # 100 MHz ticks -> us
        return t[0] if wgs == 1 else t

    def set_launch_count(self, count):
        """Preset the token kernel's launch counter (test hook)."""
        check(lib().nut_model_set_launch_count(self.handle, count))

    def inject_fault(self, fault):
        """nut_model_inject_fault: 1 makes the token kernel's waits for one
        workgroup's words run into their spin limit (test hook)."""
        check(lib().nut_model_inject_fault(self.handle, int(fault)))

    def last_decode_ms(self):
        """Device time of the last generate() decode loop (HIP events)."""
        ms = C.c_double()
        check(lib().nut_model_last_decode_ms(self.handle, C.byref(ms)))
        return ms.value

    def decode(self, cache, token, want_hidden=True):
        hidden = np.empty(self.config.dim, np.float32) if want_hidden else None
        check(lib().nut_decode(self.handle, cache.handle, int(token),
                               _ptr(hidden)))
        return hidden

    def decode_noalloc(self, cache, token, out):
        """nut_decode_noalloc: the hidden state lands in the DeviceArray
        `out` (dim floats, or None)."""
        check(lib().nut_decode_noalloc(self.handle, cache.handle, int(token),
                                       None if out is None else out.ptr))

    def prefill(self, cache, tokens):
        t = np.ascontiguousarray(tokens, np.int32)
        hidden = np.empty(self.config.dim, np.float32)
        check(lib().nut_prefill(self.handle, cache.handle, _ptr(t), t.size,
                                _ptr(hidden)))
        return hidden

    def logits(self, hidden):
        h = np.ascontiguousarray(hidden, np.float32)
        out = np.empty(self.config.vocab_size, np.float32)
        check(lib().nut_logits(self.handle, _ptr(h), _ptr(out)))
        return out

    def generate(self, prompt, max_tokens):
        """Greedy generate_tokens_cached; returns (ids, GenerationStats)."""
        p = np.ascontiguousarray(prompt, np.int32)
        out = np.empty(max(1, max_tokens), np.int32)
        count = C.c_size_t()
        stats = GenerationStats()
        check(lib().nut_generate_greedy(self.handle, _ptr(p), p.size,
                                        max_tokens, _ptr(out),
                                        C.byref(count), C.byref(stats)))
        return out[:count.value].tolist(), stats

    def generate_sampled(self, prompt, max_tokens, temperature, top_p, seed):
        """generate_tokens_cached with temperature / top-p sampling."""
        p = np.ascontiguousarray(prompt, np.int32)
        out = np.empty(max(1, max_tokens), np.int32)
        count = C.c_size_t()
        stats = GenerationStats()
        check(lib().nut_generate_sampled(self.handle, _ptr(p), p.size, max_tokens,
                                         float(temperature), float(top_p), int(seed),
                                         _ptr(out), C.byref(count), C.byref(stats)))
        return out[:count.value].tolist(), stats

    def close(self):
        if self.handle:
            check(lib().nut_model_destroy(self.handle))
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class DeviceFModel:
    """fp32 ModelWeights resident in HBM: decode_token / prefill_tokens
    (src/kvcache.cpp:237-284). Projections in the reference's [in x out]
    layout."""

    def __init__(self, config, tied=False):
        self.config = config
        self.tied = tied
        h = C.c_void_p()
        check(lib().nut_fmodel_create(C.byref(config), int(tied), C.byref(h)))
        self.handle = h

    def set_globals(self, embeddings, final_norm, lm_head=None):
        e = np.ascontiguousarray(embeddings, np.float32)
        n = np.ascontiguousarray(final_norm, np.float32)
        l = None if lm_head is None else np.ascontiguousarray(lm_head, np.float32)
        check(lib().nut_fmodel_set_globals(self.handle, _ptr(e), _ptr(n), _ptr(l)))

    def set_layer(self, index, weights, attention_norm, ffn_norm):
        ws = [np.ascontiguousarray(weights[n], np.float32) for n in PROJECTIONS]
        an = np.ascontiguousarray(attention_norm, np.float32)
        fn = np.ascontiguousarray(ffn_norm, np.float32)
        check(lib().nut_fmodel_set_layer(self.handle, index, *[_ptr(w) for w in ws],
                                         _ptr(an), _ptr(fn)))

    def decode(self, cache, token):
        hidden = np.empty(self.config.dim, np.float32)
        check(lib().nut_decode_token(self.handle, cache.handle, int(token), _ptr(hidden)))
        return hidden

    def prefill(self, cache, tokens):
        t = np.ascontiguousarray(tokens, np.int32)
        rows = np.empty((t.size, self.config.dim), np.float32)
        check(lib().nut_prefill_tokens(self.handle, cache.handle, _ptr(t), t.size,
                                       _ptr(rows)))
        return rows

    def close(self):
        if self.handle:
            check(lib().nut_fmodel_destroy(self.handle))
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


__all__ = [n for n in dir() if not n.startswith("_")]
