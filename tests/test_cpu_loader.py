"""The llama2.c product loader's checks without a GPU: the reference's
header and size errors (src/llama2.cpp:199-296, its messages) come before
the device is touched, and a valid file then fails with DeviceError (no
CPU fallback)."""
import os

import numpy as np
import pytest

import nutllm_amd as nut

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
FIXTURE = os.path.join(ROOT, "tests", "golden", "tiny-llama2.bin")


def write_bytes(tmp_path, name, data):
    p = tmp_path / name
    p.write_bytes(data)
    return str(p)


def header(dim=64, ffn=172, layers=2, heads=4, kv=2, vocab=-256, seq=64):
    return np.array([dim, ffn, layers, heads, kv, vocab, seq], np.int32).tobytes()


@pytest.mark.parametrize("data,message", [
    (b"\x01\x02", "llama2 checkpoint: truncated header"),
    (header(dim=0), "llama2 checkpoint: invalid dimension"),
    (header(kv=-1), "llama2 checkpoint: invalid kv head count"),
    (header(vocab=0), "llama2 checkpoint: invalid vocabulary"),
    (header(vocab=-2**31), "llama2 checkpoint: invalid vocabulary"),
    (header(dim=66, heads=4), "llama2 checkpoint: heads do not divide dimension"),
    (header() + b"\0" * 64, "llama2 checkpoint: size does not match configuration"),
], ids=["short", "dim", "kv", "vocab0", "vocabmin", "heads", "size"])
def test_header_errors_match_reference(tmp_path, data, message):
    path = write_bytes(tmp_path, "bad.bin", data)
    with pytest.raises(nut.NutError) as e:
        nut.DeviceModel.load_llama2c(path, nut.INT8)
    assert str(e.value) == message


def test_missing_and_empty_files(tmp_path):
    with pytest.raises(nut.NutError, match="^llama2 checkpoint: cannot open "):
        nut.DeviceModel.load_llama2c(str(tmp_path / "none.bin"), nut.INT4)
    with pytest.raises(nut.NutError, match="^llama2 checkpoint: empty file$"):
        nut.DeviceModel.load_llama2c(write_bytes(tmp_path, "e.bin", b""), nut.INT4)


def test_invalid_config_is_the_models_error(tmp_path):
    # head_dim 63 is odd: ModelConfig::validate rejects it
    with pytest.raises(nut.InvalidArgument, match="^model config: invalid dimensions$"):
        nut.DeviceModel.load_llama2c(
            write_bytes(tmp_path, "odd.bin", header(dim=126, heads=2, kv=2)), nut.INT8)


def _no_gpu():
    try:
        return nut.device_count() == 0
    except nut.DeviceError:
        return True


@pytest.mark.skipif(not _no_gpu(), reason="a GPU is visible")
def test_valid_file_needs_the_device():
    with pytest.raises(nut.DeviceError):
        nut.DeviceModel.load_llama2c(FIXTURE, nut.INT8)
