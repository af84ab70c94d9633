"""GPU parity of a model loaded from disk by the library's own GGUF loader
(cohx_load_gguf: the engine's parser and graph checks, gguf.rs:304-496,
compat.rs:54-221) against the CPU oracle over the same file."""
import os

import numpy as np
import pytest

import cohx
import gguf
import orc
import synth

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype,hidden,intermediate", [("q8_0", 128, 256), ("f16", 128, 256),
                                                       ("q4_k_m", 256, 512)])
def test_loaded_file_steps_match_oracle(tmp_path, dtype, hidden, intermediate):
    print(f"case: load {dtype} from disk", flush=True)
    cfg = synth.config(layers=2, hidden=hidden, intermediate=intermediate, heads=4, kv_heads=2,
                       vocabulary=300, context=512)
    path = synth.write_model(os.path.join(tmp_path, f"{dtype}.gguf"), cfg, dtype, seed=21)
    m = cohx.Model.load(path, max_lanes=4, max_rows=32, max_seqs=4, max_context=128)
    assert m.desc.weight_dtype == (cohx.MIXED if dtype == "q4_k_m" else cohx.DTYPE[dtype])
    meta, tensors = gguf.read(path)
    o = orc.Model(gguf.qwen2_config(meta), tensors, threads=8)
    rng = np.random.default_rng(22)
    seqs = [m.seq_alloc() for _ in range(2)]
    sess = [o.session(128) for _ in range(2)]
    for step, spec in enumerate([{0: 6, 1: 2}, {0: 1, 1: 1}, {1: 3, 0: 1}]):
        lanes, toks = [], {}
        for i, n in spec.items():
            toks[i] = [int(v) for v in rng.integers(0, 300, n)]
            lanes.append(dict(seq=seqs[i], tokens=toks[i], logits=True))
        res = m.step(lanes)
        for (i, _), r in zip(spec.items(), res):
            assert r["status"] == 0
            for tok in toks[i]:
                assert o.forward_batch([sess[i]], [tok])[0] == 0
            want = sess[i].logits()
            bad = int((r["logits"].view(np.uint32) != want.view(np.uint32)).sum())
            print(f"step {step} lane {i}: {bad} logits differ in bits", flush=True)
            assert bad == 0
            assert r["argmax"] == orc.Sampler().sample(want)[1]
    for i in range(2):
        for layer in range(cfg["layers"]):
            assert np.array_equal(m.seq_read_kv(seqs[i], layer), sess[i].kv(layer))
    m.close()


def test_load_refuses_what_the_step_does_not_run(tmp_path):
    """F32 matrices: the engine runs them; this library refuses the file at
    load with COHX_UNSUPPORTED instead of computing them another way."""
    cfg = synth.config(layers=1, hidden=128, intermediate=256, heads=4, kv_heads=2,
                       vocabulary=64, context=64)
    path = synth.write_model(os.path.join(tmp_path, "f32.gguf"), cfg, "f32", seed=1)
    with pytest.raises(cohx.CohxError) as e:
        cohx.Model.load(path, max_lanes=2, max_context=32)
    assert e.value.code == cohx.UNSUPPORTED
