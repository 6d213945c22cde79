"""The C-ABI library on a host without a GPU.

* libnutllm_hip.so loads and exports every entry point include/nutllm_hip.h
  declares (and the Python binding binds only declared ones);
* host-side entry points work without a device: the quantiser, fp16
  helpers, config validation and the synthetic generator, with the
  reference's exception kinds and messages (src/quant.cpp:24-27,61,138-139,
  158-168);
* nothing falls back to the CPU: device entry points fail with
  NUT_EDEVICE / DeviceError when no gfx950 device is visible.
"""
from __future__ import annotations

import ctypes as C
import os
import re

import numpy as np
import pytest

import nutllm_amd as nut

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "nutllm_hip.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(nut_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_boundary():
    names = declared_functions()
    for must in ("nut_quantize", "nut_matvec_q", "nut_matvec_f32",
                 "nut_matmul_f32", "nut_model_create", "nut_decode",
                 "nut_prefill", "nut_logits", "nut_generate_greedy",
                 "nut_kv_create", "nut_kv_read", "nut_kv_set_length"):
        assert must in names


def test_library_exports_every_declared_symbol():
    handle = C.CDLL(nut.LIB_PATH)
    missing = [n for n in declared_functions() if not hasattr(handle, n)]
    assert not missing, missing


def test_binding_only_binds_declared_symbols():
    assert set(nut.exported_symbols()) <= set(declared_functions())


def _no_gpu():
    try:
        return nut.device_count() == 0
    except nut.DeviceError:
        return True


def test_quantize_messages_match_reference():
    w = np.ones((2, 32), np.float32)
    with pytest.raises(nut.InvalidArgument, match="^quantize: zero block size$"):
        nut.quantize(w, 0, block_size=0)
    bad = w.copy()
    bad[1, 3] = np.inf
    with pytest.raises(nut.InvalidArgument,
                       match="^quantize: non-finite source weight$"):
        nut.quantize(bad, 1)
    big = w.copy()
    big[0, 0] = 1e9
    with pytest.raises(nut.RangeError, match="^quantize: scale exceeds fp16$"):
        nut.quantize(big, 0)
    L = nut.lib()
    data = np.zeros(64, np.uint8)
    scales = np.zeros(2, np.uint16)
    st = L.nut_quantize(None, 2, 32, 0, 32, data.ctypes.data,
                        scales.ctypes.data)
    assert st == 1 and L.nut_last_error().decode() == "quantize: null source"
    st = L.nut_quantize(w.ctypes.data, 0, 32, 0, 32, data.ctypes.data,
                        scales.ctypes.data)
    assert st == 1
    assert L.nut_last_error().decode() == "quantize: invalid dimensions"


def test_quantize_first_failing_block_wins():
    """A matrix with a non-finite weight in a late block and an oversized
    scale in an early one reports the early block's error, as the
    reference's block loop does (src/quant.cpp:161-175), also when the
    host quantiser splits blocks over threads."""
    w = np.ones((512, 1024), np.float32) * 0.01
    w[3, 0] = 1e9     # block of row 3: range_error
    w[500, 7] = np.nan  # later block: invalid_argument
    with pytest.raises(nut.RangeError):
        nut.quantize(w, 0)
    w[3, 0] = 0.01
    with pytest.raises(nut.InvalidArgument):
        nut.quantize(w, 0)


def test_synthetic_generator_is_deterministic_and_normal():
    a = nut.synth_normal(3, 16, 1 << 16, 0.02)
    b = nut.synth_normal(3, 16, 1 << 16, 0.02)
    c = nut.synth_normal(3, 17, 1 << 16, 0.02)
    assert np.array_equal(a, b) and not np.array_equal(a, c)
    # element i depends only on (seed, stream, i)
    assert np.array_equal(nut.synth_normal(3, 16, 100, 0.02), a[:100])
    assert abs(a.mean()) < 3 * 0.02 / 256
    assert abs(a.std() - 0.02) < 0.02 * 0.02
    t = nut.synth_tokens(5, 32000, 4096)
    assert t.min() >= 0 and t.max() < 32000
    assert np.array_equal(t, nut.synth_tokens(5, 32000, 4096))


@pytest.mark.skipif(not _no_gpu(), reason="a GPU is visible")
def test_device_calls_fail_loudly_without_gpu():
    assert nut.device_count() == 0
    cfg = nut.Config(layers=2, heads=4, dim=64, head_dim=16, ffn_dim=172,
                     vocab_size=256, max_seq=64, eos_token=1, kv_heads=2)
    with pytest.raises(nut.DeviceError):
        nut.DeviceModel(cfg, 0)
    with pytest.raises(nut.DeviceError):
        nut.DeviceArray(1024)
    data, scales = nut.quantize(np.ones((4, 32), np.float32), 0)
    with pytest.raises(nut.DeviceError):
        nut.QWeight(data, scales, 4, 32, 0)


def test_token_tag_schedule_never_reuses_a_live_base():
    """The token kernel's exchange words carry (tag << 32) | value and each
    launch polls for tags of its own base. Over three restarts of the
    32-bit tag range (every launch kind uses the same counter): no base is
    0 (the tag of zeroed words), no base repeats since the last zeroing,
    and a zeroing is asked for exactly when the counter restarts, so a word
    left by an earlier launch can never already hold the tag a consumer of
    a later launch waits for."""
    count = 0
    live = set()  # bases launched since the buffer was last zeroed
    clears = 0
    for _ in range(3 * 4095 + 10):
        base, count, clear = nut.token_tag_base(count)
        if clear:
            clears += 1
            live.clear()
        assert base != 0 and base % (1 << 20) == 0
        assert base not in live
        live.add(base)
    assert clears == 3
    # a preset counter (the GPU test hook) restarts on its next launch
    assert nut.token_tag_base(4095) == (1 << 20, 1, True)
    assert nut.token_tag_base(4094) == (4095 << 20, 4095, False)
