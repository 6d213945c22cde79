"""The llama2.c product loader on the GPU (load_llama2c_quantized_model,
src/llama2.cpp:339-412, straight into HBM).

* The reference's fixtures: [1, 0, 3] generates [4, 5] (INT8 and INT4,
  src/loader_selftest.cpp, file lines 96-116); the shared-classifier file
  loads tied.
* A checkpoint written from a seeded model (two layers, dim 256, non-unit
  norms, unshared classifier): the loaded model equals the one uploaded
  from the same weights through the quantiser (storage_bytes, the
  post-prompt hidden state bit for bit, greedy ids), and its greedy ids
  equal the oracle's; load_s is reported.
"""
import os

import numpy as np
import pytest

import llama2c
import nutllm_amd as nut
import oracle as O
from nutllm_amd import workloads as W

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.mark.parametrize("qtype", [0, 1], ids=["int8", "int4"])
def test_fixture_says_hi(gpu, qtype):
    dev, seconds = gpu.DeviceModel.load_llama2c(
        os.path.join(GOLDEN, "tiny-llama2.bin"), qtype)
    try:
        assert dev.config.eos_token == 1 and seconds > 0
        ids, stats = dev.generate(np.array([1, 0, 3], np.int32), 8)
        assert ids == [4, 5]
        assert stats.prefill_tokens == 3 and stats.generated_tokens == 2
    finally:
        dev.close()
    shared, _ = gpu.DeviceModel.load_llama2c(
        os.path.join(GOLDEN, "tiny-llama2-shared.bin"), qtype)
    try:
        tied = np.zeros(1, np.int32)
        cfg = nut.Config()
        nut.check(nut.lib().nut_model_config(shared.handle, nut.C.byref(cfg),
                                             None, tied.ctypes.data))
        assert tied[0] == 1
        cfg_file, w, is_shared = llama2c.load(os.path.join(GOLDEN, "tiny-llama2-shared.bin"))
        assert is_shared
        ids, _ = shared.generate(np.array([1, 0, 3], np.int32), 8)
        # oracle over the file's weights, the classifier being the embeddings
        mats = []
        for l in range(cfg_file["layers"]):
            layer = {}
            for name in O.PROJECTIONS:
                m = np.ascontiguousarray(w[name][l])
                data, scales = gpu.quantize(m, qtype)
                layer[name] = (data, scales, m.shape[0], m.shape[1])
            mats.append(layer)
        norms = [(np.ascontiguousarray(w["attention_norm"][l]),
                  np.ascontiguousarray(w["ffn_norm"][l])) for l in range(cfg_file["layers"])]
        emb = np.ascontiguousarray(w["embeddings"])
        om = O.OracleModel(cfg_file, qtype, emb, np.ascontiguousarray(w["final_norm"]), emb,
                           mats, norms)
        ref, _, _ = om.generate(np.array([1, 0, 3], np.int32), 8)
        assert ids == ref
    finally:
        shared.close()


@pytest.mark.parametrize("qtype", [0, 1], ids=["int8", "int4"])
def test_written_checkpoint_equals_direct_upload(gpu, tmp_path, qtype):
    O.orc().orc_set_threads(16)
    model = W.build("step_gqa2", qtype, 9, 300, keep_fp32=True, norm_seed=17)
    c = model.config
    w = {"embeddings": model.embeddings, "classifier": model.lm_head,
         "final_norm": model.final_norm,
         "attention_norm": np.stack([a for a, _ in model.norms]),
         "ffn_norm": np.stack([f for _, f in model.norms])}
    for name in O.PROJECTIONS:
        w[name] = np.stack([model.fp32_layers[l][name] for l in range(c.layers)])
    path = str(tmp_path / "model.bin")
    llama2c.write(path, c.as_dict(), w, shared=False)
    loaded, seconds = gpu.DeviceModel.load_llama2c(path, qtype)
    direct = model.to_device()
    prompt = gpu.synth_tokens(4, c.vocab_size, 12)
    try:
        print(f"load_s {seconds:.3f}", flush=True)
        assert seconds > 0
        assert loaded.storage_bytes() == direct.storage_bytes()
        ca, cb = gpu.KVCache(c), gpu.KVCache(c)
        assert np.array_equal(loaded.prefill(ca, prompt), direct.prefill(cb, prompt))
        ids, _ = loaded.generate(prompt, 10)
        assert ids == direct.generate(prompt, 10)[0]
        ref, _, _ = O.oracle_model(model).generate(prompt, 10)
        assert ids == ref
    finally:
        loaded.close()
        direct.close()
