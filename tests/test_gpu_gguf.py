"""A GGUF checkpoint loaded into HBM decodes exactly like the same weights
produced on the device: the file is written from the CPU restatement's copy
of the synthetic weights (the GPU tests pin every tensor kind to the device
generator), loaded with cq35_model_load_gguf (Model::load_gguf,
src/model.rs:43, 81-153), and its greedy tokens, BF16 logits and session
state are compared bit for bit with Model.synthetic over a prompt and decode
steps."""
import numpy as np
import pytest

import cq35
import cq35.config as cc
import gguf_writer as gw

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)


@pytest.mark.parametrize("name,tied", [("tiny-moe", 0), ("mini-moe", 0), ("mini", 0), ("mini", 1)])
def test_gguf_model_decodes_like_synthetic(tmp_path, oracle, name, tied):
    cfg = dict(cc.preset(name), tied=tied)
    seed = 21
    say("gguf", name, "tied", tied)
    arrays = oracle.synthetic_weights(cfg, seed)
    path = str(tmp_path / "model.gguf")
    gw.write(path, gw.metadata(cfg), gw.tensors_for(cfg, arrays))
    loaded = cq35.Model.load_gguf(path)
    for k, v in cfg.items():
        assert loaded.cfg[k] == pytest.approx(v) if isinstance(v, float) else loaded.cfg[k] == v, k
    synth = cq35.Model.synthetic(cfg, seed=seed)
    prompt = np.random.default_rng(3).integers(0, cfg["vocab"], 9).tolist()
    sa, sb = loaded.session(32), synth.session(32)
    la, ta = sa.step_raw(prompt)
    lb, tb = sb.step_raw(prompt)
    assert ta == tb and np.array_equal(la, lb), f"{name}: prompt differs"
    for i in range(12):
        la, ta = sa.step_raw([ta])
        lb, tb = sb.step_raw([tb])
        assert ta == tb and np.array_equal(la, lb), f"{name}: decode step {i} differs"
    assert np.array_equal(sa.export_state(0), sb.export_state(0))
