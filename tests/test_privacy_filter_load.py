"""load_privacy_filter on a small model written in the exported layout
(runntime.quant I8 + F16 `_scale` attention Linears, U32 quantW MoE words):
the loader's checks on the CPU, and on the GPU the loaded model's logits
equal those of the same weights built directly."""
import json

import numpy as np
import pytest

from runntime_amd import privacy_filter as pf
from runntime_amd.errors import RunntimeError
from runntime_amd.quantw import pack_expert_weights
from runntime_amd.safetensors import write

E, I, VOCAB, CLASSES = 8, 64, 50, 36
QUANT = json.dumps({"version": 1, "bits": 8, "scheme": "symmetric"})


def _qlin(rng, out_f, in_f, g):
    ints = rng.integers(-127, 128, size=(out_f, in_f)).astype(np.int8)
    sc = (rng.uniform(0.5, 1.5, size=(out_f, in_f // g)) / (127 * np.sqrt(in_f))).astype(np.float16)
    return ints, sc


def make_file(path, blocks=2, seed=0, drop=None, model="privacy-filter"):
    rng = np.random.default_rng(seed)
    t = {}
    raw = {"blocks": []}
    for b in range(blocks):
        p = f"block.{b}."
        qi, qs = _qlin(rng, 1152, 640, 640)
        oi, os_ = _qlin(rng, 640, 896, 128)
        qb = rng.standard_normal(1152).astype(np.float32) * 0.1
        ob = rng.standard_normal(640).astype(np.float32) * 0.1
        sinks = rng.standard_normal(14).astype(np.float32)
        an = rng.uniform(0.5, 1.5, 640).astype(np.float32)
        t[p + "attn.norm.scale"] = ("F32", [640], an)
        t[p + "attn.qkv.weight"] = ("I8", [1152, 640], qi)
        t[p + "attn.qkv.weight_scale"] = ("F16", list(qs.shape), qs)
        t[p + "attn.qkv.bias"] = ("F32", [1152], qb)
        t[p + "attn.out.weight"] = ("I8", [640, 896], oi)
        t[p + "attn.out.weight_scale"] = ("F16", list(os_.shape), os_)
        t[p + "attn.out.bias"] = ("F32", [640], ob)
        t[p + "attn.sinks"] = ("F32", [14], sinks)
        t[p + "mlp.norm.scale"] = ("F32", [640], rng.uniform(0.5, 1.5, 640).astype(np.float32))
        t[p + "mlp.gate.weight"] = ("F32", [E, 640], (rng.standard_normal((E, 640)) * 0.02).astype(np.float32))
        for stem, K, N in (("glu", 640, I), ("lin", 640, I), ("out", I, 640)):
            q = rng.integers(-127, 128, size=(E, K, N)).astype(np.int8)
            words = pack_expert_weights(q, 8)
            t[p + f"mlp.{stem}Weight"] = ("U32", [words.size], words)
            t[p + f"mlp.{stem}Scales"] = ("F32", [E, N], rng.uniform(0.5e-3, 2e-3, (E, N)).astype(np.float32))
            t[p + f"mlp.{stem}Bias"] = ("F32", [E, N], (rng.standard_normal((E, N)) * 0.01).astype(np.float32))
        raw["blocks"].append((qi, qs, qb, oi, os_, ob, sinks, an))
    t["embedding.weight"] = ("F32", [VOCAB, 640], rng.standard_normal((VOCAB, 640)).astype(np.float32))
    t["norm.scale"] = ("F32", [640], np.ones(640, np.float32))
    ui, us = _qlin(rng, CLASSES, 640, 640)
    t["unembedding.weight"] = ("I8", [CLASSES, 640], ui)
    t["unembedding.weight_scale"] = ("F16", list(us.shape), us)
    if drop:
        t.pop(drop)
    write(str(path), t, {"model": model, "runntime.quant": QUANT})
    return raw


def test_loader_checks(tmp_path):
    p = tmp_path / "m.safetensors"
    make_file(p, drop="block.1.attn.sinks")
    with pytest.raises(RunntimeError, match="missing tensor 'block.1.attn.sinks'"):
        pf.load_privacy_filter(str(p), device="cpu")
    make_file(p, model="yolo26")
    with pytest.raises(RunntimeError, match="file is for model 'yolo26', expected 'privacy-filter'"):
        pf.load_privacy_filter(str(p), device="cpu")
    make_file(p, drop="embedding.weight")
    with pytest.raises(RunntimeError, match="missing 'embedding.weight' tensor"):
        pf.load_privacy_filter(str(p), device="cpu")
    make_file(p)
    with pytest.raises(RunntimeError, match="2 blocks in the file, expected 8"):
        pf.load_privacy_filter(str(p), device="cpu", blocks=8)


def test_loader_reads_the_layout(tmp_path):
    p = tmp_path / "m.safetensors"
    make_file(p)
    m = pf.load_privacy_filter(str(p), device="cpu", blocks=2, experts=E)
    assert len(m.blocks) == 2 and m.embedding.shape == (VOCAB, 640)
    a = m.blocks[0].attn
    assert (a.qkv.in_features, a.qkv.out_features, a.qkv.group_size) == (640, 1152, 640)
    assert (a.out.in_features, a.out.out_features, a.out.group_size) == (896, 640, 128)
    assert m.unembed.out_features == CLASSES and m.blocks[1].mlp.E == E


@pytest.mark.gpu
def test_loaded_model_matches_the_built_one(tmp_path):
    import torch
    from runntime_amd.checkpoint import load_moe_block
    from runntime_amd.linear import Linear
    p = tmp_path / "m.safetensors"
    raw = make_file(p)
    m = pf.load_privacy_filter(str(p), device="cuda")
    blocks = []
    for b, (qi, qs, qb, oi, os_, ob, sinks, an) in enumerate(raw["blocks"]):
        attn = pf.AttnBlock(torch.from_numpy(an).cuda(),
                            Linear.from_quant(qi, qs.astype(np.float32), 8, qb, "cuda"),
                            Linear.from_quant(oi, os_.astype(np.float32), 8, ob, "cuda"),
                            torch.from_numpy(sinks).cuda())
        blocks.append(pf.Block(attn, load_moe_block(str(p), b, "cuda")))
    built = pf.PrivacyFilterModel(m.embedding, blocks, m.norm_w, m.unembed)
    ids = np.random.default_rng(3).integers(0, VOCAB, size=64)
    a, b = m.forward(ids), built.forward(ids)
    torch.cuda.synchronize()
    assert torch.equal(a, b) and torch.isfinite(a).all()
