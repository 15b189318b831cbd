"""The transformers-layout mapping (transform_hf_state_dict) on the
reference test's one-layer checkpoint (test/zoo/privacy-filter/
stateDictHooks.test.ts:14-120: its names, values and expected results), and
a float network built from a mapped checkpoint on the GPU."""
import numpy as np
import pytest

from runntime_amd import privacy_filter as pf
from runntime_amd.errors import RunntimeError

RENAMED = {
    "model.layers.0.input_layernorm.weight": "block.0.attn.norm.weight",
    "model.layers.0.post_attention_layernorm.weight": "block.0.mlp.norm.weight",
    "model.layers.0.self_attn.o_proj.weight": "block.0.attn.out.weight",
    "model.layers.0.self_attn.o_proj.bias": "block.0.attn.out.bias",
    "model.layers.0.mlp.router.weight": "block.0.mlp.gate.weight",
    "model.layers.0.mlp.router.bias": "block.0.mlp.gate.bias",
    "model.layers.0.self_attn.sinks": "block.0.attn.sinks",
    "model.layers.0.mlp.experts.down_proj_bias": "block.0.mlp.outBias",
    "model.embed_tokens.weight": "embedding.weight",
    "model.norm.weight": "norm.weight",
    "score.weight": "unembedding.weight",
}


def checkpoint(dtype):
    a = lambda v, s: np.array(v, dtype).reshape(s)
    ck = {n: a([0, 0], [2]) for n in RENAMED}
    ck["score.bias"] = a([0, 0], [2])
    ck.update({
        "model.layers.0.self_attn.q_proj.weight": a([1, 2, 3, 4], [2, 2]),
        "model.layers.0.self_attn.k_proj.weight": a([5, 6], [1, 2]),
        "model.layers.0.self_attn.v_proj.weight": a([7, 8], [1, 2]),
        "model.layers.0.self_attn.q_proj.bias": a([1, 2], [2]),
        "model.layers.0.self_attn.k_proj.bias": a([3], [1]),
        "model.layers.0.self_attn.v_proj.bias": a([4], [1]),
        "model.layers.0.mlp.experts.gate_up_proj": a([1, 2, 3, 4, 5, 6, 7, 8], [2, 1, 4]),
        "model.layers.0.mlp.experts.gate_up_proj_bias": a([10, 11, 12, 13, 14, 15, 16, 17], [2, 4]),
        "model.layers.0.mlp.experts.down_proj": a([1, 2, 3, 4], [2, 2, 1]),
    })
    return ck


@pytest.mark.parametrize("dtype", [np.float32, np.float16])
def test_maps_the_reference_checkpoint(dtype):
    ck = checkpoint(dtype)
    sd = pf.transform_hf_state_dict(ck)
    mapped = ["block.0.attn.qkv.weight", "block.0.attn.qkv.bias", "block.0.mlp.gluWeight",
              "block.0.mlp.linWeight", "block.0.mlp.gluBias", "block.0.mlp.linBias",
              "block.0.mlp.outWeight"]
    assert sorted(sd) == sorted(list(RENAMED.values()) + mapped)   # score.bias dropped
    for hf, ours in RENAMED.items():
        assert sd[ours] is ck[hf]
    qkv = sd["block.0.attn.qkv.weight"]
    assert qkv.shape == (4, 2) and qkv.dtype == dtype
    assert qkv.reshape(-1).tolist() == [1, 2, 3, 4, 5, 6, 7, 8]
    assert sd["block.0.attn.qkv.bias"].tolist() == [1, 2, 3, 4]
    for name, shape, values in [("block.0.mlp.gluWeight", (2, 2), [1, 2, 5, 6]),
                                ("block.0.mlp.linWeight", (2, 2), [3, 4, 7, 8]),
                                ("block.0.mlp.gluBias", (2, 2), [10, 11, 14, 15]),
                                ("block.0.mlp.linBias", (2, 2), [12, 13, 16, 17])]:
        assert sd[name].shape == shape and sd[name].dtype == dtype
        assert sd[name].reshape(-1).tolist() == values
    ow = sd["block.0.mlp.outWeight"]
    assert ow.shape == (4, 1) and ow.reshape(-1).tolist() == [1, 2, 3, 4]
    # the only bytes lost are score.bias's
    assert (sum(v.nbytes for v in sd.values()) ==
            sum(v.nbytes for v in ck.values()) - ck["score.bias"].nbytes)


def test_missing_tensor_is_a_checkpoint_mismatch():
    ck = checkpoint(np.float32)
    del ck["model.layers.0.self_attn.k_proj.weight"]
    with pytest.raises(RunntimeError, match="missing tensor 'model.layers.0.self_attn.k_proj.weight'"):
        pf.transform_hf_state_dict(ck)


@pytest.mark.gpu
def test_float_network_from_a_mapped_checkpoint(tmp_path):
    import torch
    from runntime_amd.safetensors import write
    rng = np.random.default_rng(2)
    E, d, I, vocab = 8, 640, 640, 40
    r = lambda *s, sc=1.0: (rng.standard_normal(s) * sc).astype(np.float32)
    t = {}
    for n in range(2):
        h = f"model.layers.{n}"
        t[f"{h}.input_layernorm.weight"] = r(d, sc=0.1) + 1
        t[f"{h}.post_attention_layernorm.weight"] = r(d, sc=0.1) + 1
        for p_, rows in (("q", 896), ("k", 128), ("v", 128)):
            t[f"{h}.self_attn.{p_}_proj.weight"] = r(rows, d, sc=d ** -0.5)
            t[f"{h}.self_attn.{p_}_proj.bias"] = r(rows, sc=0.1)
        t[f"{h}.self_attn.o_proj.weight"] = r(d, 896, sc=896 ** -0.5)
        t[f"{h}.self_attn.o_proj.bias"] = r(d, sc=0.1)
        t[f"{h}.self_attn.sinks"] = r(14)
        t[f"{h}.mlp.router.weight"] = r(E, d, sc=0.02)
        t[f"{h}.mlp.router.bias"] = r(E, sc=0.1)
        t[f"{h}.mlp.experts.gate_up_proj"] = r(E, d, 2 * I, sc=d ** -0.5)
        t[f"{h}.mlp.experts.gate_up_proj_bias"] = r(E, 2 * I, sc=0.1)
        t[f"{h}.mlp.experts.down_proj"] = r(E, I, d, sc=I ** -0.5)
        t[f"{h}.mlp.experts.down_proj_bias"] = r(E, d, sc=0.1)
    t["model.embed_tokens.weight"] = r(vocab, d)
    t["model.norm.weight"] = np.ones(d, np.float32)
    t["score.weight"] = r(36, d, sc=d ** -0.5)
    t["score.bias"] = np.zeros(36, np.float32)
    path = tmp_path / "hf.safetensors"
    write(str(path), {n: ("F32", list(a.shape), a) for n, a in t.items()})
    model = pf.load_privacy_filter_hf(str(path), "cuda")
    ids = rng.integers(0, vocab, size=33)
    logits = model.forward(ids)
    torch.cuda.synchronize()
    assert logits.shape == (33, 36) and torch.isfinite(logits).all()
    # the same tensors mapped and built directly give the same logits
    direct = pf.model_from_float_state_dict(pf.transform_hf_state_dict(t), "cuda")
    assert torch.equal(direct.forward(ids), logits)
