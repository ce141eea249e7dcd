"""The CPU restatement of the model pipeline (tests/toy_models.py) against the reference's own
end-to-end assertions (tests/toy_models.rs:247-445) on checkpoints shaped to the reference's
Hessian fixtures. The GPU pipeline is then compared with this restatement byte for byte
(tests/test_gpu_pipeline.py)."""
import os

import pytest

import toy_models as T


@pytest.mark.parametrize("mi", range(len(T.MODELS)))
def test_oracle_pipeline_passes_the_reference_checks(tmp_path, mi):
    m = T.MODELS[mi]
    ck = T.make_checkpoint(m, str(tmp_path / m["dir"] / "model.safetensors"), seed=mi)
    cfg = T.cfg_kw(m)
    outs, reports = T.oracle_quantize_model([ck], [os.path.join(T.GOLDEN, m["fixture"])], cfg)
    orig, _ = T.read_st(ck)
    deq = outs["dequant"]["model.safetensors"]
    pk, meta = outs["packed"]["model.safetensors"]
    assert meta["orig_dtype"] == m["dtype"]
    T.reference_checks(m, orig, deq, pk, meta, reports, cfg)


def test_checkpoint_layout_matches_the_fixture_hessians(tmp_path):
    m = T.MODELS[1]
    ck = T.make_checkpoint(m, str(tmp_path / "model.safetensors"))
    t, meta = T.read_st(ck)
    store = T.HessStore([os.path.join(T.GOLDEN, m["fixture"])])
    q = t["model.layers.0.self_attn.q_proj.weight"]
    assert q[0] == "BF16" and q[1] == [512, store.tensor(store.resolve("model.layers.0.self_attn.q_proj"), "H").shape[0]]
    assert t["model.layers.0.self_attn.o_proj.weight"][1] == [8, 512]
    assert meta == {"format": "pt"}
