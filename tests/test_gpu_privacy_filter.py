"""The privacy-filter attention block (attnBlock.ts:28-57) on the GPU
against an f64 composition of the pinned pieces (rmsNorm, dequantized
Linears, oracle rope_f64 and sdpa_f64, + x), with int8 group-quantized qkv
and out projections; the whole model forward (model.ts:62-75) against an
f64 composition of the pinned pieces, and equal to its own chain of block
calls; graph replays equal to eager forwards."""
import numpy as np
import pytest
import torch

from oracle import ref
from runntime_amd import privacy_filter as pf
from runntime_amd.checkpoint import MoeBlock
from runntime_amd.linear import Linear
from runntime_amd.quantw import QuantExpertWeight, QuantW, pack_expert_weights

pytestmark = pytest.mark.gpu
DEV = "cuda"


def say(msg):
    print(msg, flush=True)


def qlinear(rng, out_f, in_f, g, bias=True):
    ints = rng.integers(-127, 128, size=(out_f, in_f)).astype(np.int8)
    scales = rng.uniform(0.5, 1.5, size=(out_f, in_f // g)).astype(np.float32) / (127 * np.sqrt(in_f))
    b = rng.standard_normal(out_f).astype(np.float32) * 0.1 if bias else None
    lin = Linear.from_quant(ints, scales, 8, b, DEV)
    deq = (ints.astype(np.float64).reshape(out_f, in_f // g, g) * scales[..., None]).reshape(out_f, in_f)
    return lin, deq, (b.astype(np.float64) if b is not None else 0.0)


def attn_f64(x, norm_w, wqkv, bqkv, wout, bout, sinks, cos, sin):
    x = x.astype(np.float64)
    xn = x / np.sqrt((x * x).mean(1, keepdims=True) + pf.RMS_EPS) * norm_w
    qkv = xn @ wqkv.T + bqkv
    q = ref.rope_f64(qkv, cos, sin, 64, 0, 896)
    k = ref.rope_f64(qkv, cos, sin, 64, 896, 128)
    v = qkv[:, 1024:1152]
    a = ref.sdpa_f64(q, k, v, 14, 2, 64, 128, 128, 0, sinks)
    return x + a @ wout.T + bout


def make_attn(rng):
    qkv, wqkv, bqkv = qlinear(rng, 1152, 640, 640)
    out, wout, bout = qlinear(rng, 640, 896, 128)
    norm_w = rng.uniform(0.5, 1.5, 640).astype(np.float32)
    sinks = rng.standard_normal(14).astype(np.float32)
    blk = pf.AttnBlock(torch.from_numpy(norm_w).to(DEV), qkv, out, torch.from_numpy(sinks).to(DEV))
    return blk, (norm_w.astype(np.float64), wqkv, bqkv, wout, bout, sinks)


@pytest.mark.parametrize("T", [1, 37, 300, 700])
def test_attention_block_against_f64(T):
    say(f"attn block T={T}")
    rng = np.random.default_rng(T)
    blk, ref_args = make_attn(rng)
    x = rng.standard_normal((T, 640)).astype(np.float32)
    cos, sin = pf.rope_constants(T)
    got = blk.forward(torch.from_numpy(x).to(DEV), torch.from_numpy(cos).to(DEV),
                      torch.from_numpy(sin).to(DEV))
    torch.cuda.synchronize()
    want = attn_f64(x, *ref_args, cos, sin)
    np.testing.assert_allclose(got.cpu().numpy(), want, atol=2e-4, rtol=1e-3)


def moe_block(rng, E=8, k=4, I=640, with_ref=False):
    refs = {}

    def expert(name, K, N):
        q = rng.integers(-127, 128, size=(E, K, N)).astype(np.int8)
        sc = rng.uniform(0.5e-3, 2e-3, size=(E, N)).astype(np.float32)
        b = rng.standard_normal((E, N)).astype(np.float32) * 0.01
        refs[name] = (q.astype(np.float64) * sc[:, None, :].astype(np.float64), b.astype(np.float64))
        words = pack_expert_weights(q, 8)
        d = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(DEV)
        return QuantExpertWeight(QuantW(d(words.view(np.int32)), (E * K, N)), d(sc), d(b))
    norm_w = rng.uniform(0.5, 1.5, 640).astype(np.float32)
    router_w = rng.standard_normal((640, E)).astype(np.float32) * 0.02
    blk = MoeBlock(norm_w=torch.from_numpy(norm_w).to(DEV), router_w=torch.from_numpy(router_w).to(DEV),
                   router_b=None, glu=expert("glu", 640, I), lin=expert("lin", 640, I),
                   down=expert("down", I, 640), E=E, d=640, I=I, bits=8, group_up=640,
                   group_down=I, k=k)
    if not with_ref:
        return blk
    refs.update(norm_w=norm_w.astype(np.float64), router_w=router_w.astype(np.float64), k=k)
    return blk, refs


_swiglu_f64 = np.vectorize(ref.swiglu, otypes=[np.float64])


def moe_block_f64(x, r):
    """EagerMoeMlp.forward (moeMlp.ts:79-121) in f64 from the pinned pieces:
    rmsNorm, router = xn·W, topk (lowest id on ties, softmax over the picked
    logits), dequantized expert products with the oracle's SwiGLU, + x.
    Returns the output and the smallest gap between the k-th and (k+1)-th
    logit over the tokens (the route is stable against rounding when it is
    well above the f32 error of the logits)."""
    k = r["k"]
    xn = x / np.sqrt((x * x).mean(1, keepdims=True) + pf.RMS_EPS) * r["norm_w"]
    logits = xn @ r["router_w"]
    ids = np.argsort(-logits, axis=1, kind="stable")[:, :k]
    top = np.take_along_axis(logits, ids, 1)
    gap = (top[:, k - 1] - np.sort(logits, axis=1)[:, -k - 1]).min()
    gates = np.exp(top - top[:, :1])
    gates /= gates.sum(1, keepdims=True)
    out = x.copy()
    (wg, bg), (wl, bl), (wd, bd) = r["glu"], r["lin"], r["down"]
    for t in range(x.shape[0]):
        for s in range(k):
            e = ids[t, s]
            act = _swiglu_f64(xn[t] @ wg[e] + bg[e], xn[t] @ wl[e] + bl[e])
            out[t] += gates[t, s] * (act @ wd[e] + bd[e])
    return out, gap


def test_model_forward_is_its_block_chain_and_decodes():
    rng = np.random.default_rng(11)
    blocks = []
    for _ in range(2):
        attn, _ = make_attn(rng)
        blocks.append(pf.Block(attn, moe_block(rng)))
    unembed, uw, _ = qlinear(rng, 36, 640, 640, bias=False)  # 33 classes, padded to 36
    emb = rng.standard_normal((50, 640)).astype(np.float32)
    model = pf.PrivacyFilterModel(emb, blocks, torch.ones(640, device=DEV), unembed)
    ids = rng.integers(0, 50, size=90)
    say("model forward T=90")
    logits = model.forward(ids)
    torch.cuda.synchronize()
    cos, sin = pf.rope_constants(90)
    x = torch.from_numpy(emb[ids]).to(DEV)
    cos_t, sin_t = torch.from_numpy(cos).to(DEV), torch.from_numpy(sin).to(DEV)
    for b in blocks:
        x = b.forward(x, cos_t, sin_t)
    from runntime_amd.core import rmsNorm
    want = unembed.forward(rmsNorm(x, torch.ones(640, device=DEV), pf.RMS_EPS))
    assert torch.equal(logits, want)
    assert torch.isfinite(logits).all()
    # unembed against f64 from the GPU's own last hidden state
    h = x.cpu().numpy().astype(np.float64)
    hn = h / np.sqrt((h * h).mean(1, keepdims=True) + pf.RMS_EPS)
    np.testing.assert_allclose(logits.cpu().numpy(), hn @ uw.T, atol=1e-4, rtol=1e-3)
    info = pf.build_label_info(pf.V2_NER_CLASS_NAMES)
    labels = pf.ViterbiDecoder(info).decode(pf.log_softmax_rows(logits[:, :33].cpu().numpy()))
    assert len(labels) == 90 and all(0 <= l < 33 for l in labels)
    assert np.isfinite(hn).all()


def test_model_forward_against_f64_composition():
    """The whole 2-block network (model.ts:62-75: attention block, MoE
    block, final rmsNorm, unembed) against an f64 composition of the pinned
    pieces: attn_f64 (rope_f64, sdpa_f64, dequantized Linears) and the f64
    MoE block. Logits within the layer bar, Viterbi labels equal."""
    rng = np.random.default_rng(35)  # route gaps 1.7e-3 and 4.8e-3
    blocks, refs = [], []
    for _ in range(2):
        attn, aref = make_attn(rng)
        mlp, mref = moe_block(rng, with_ref=True)
        blocks.append(pf.Block(attn, mlp))
        refs.append((aref, mref))
    unembed, uw, _ = qlinear(rng, 36, 640, 640, bias=False)
    emb = rng.standard_normal((50, 640)).astype(np.float32)
    model = pf.PrivacyFilterModel(emb, blocks, torch.ones(640, device=DEV), unembed)
    T = 90
    ids = rng.integers(0, 50, size=T)
    say(f"model forward T={T} against f64")
    got = model.forward(ids).cpu().numpy()
    cos, sin = pf.rope_constants(T)
    h = emb[ids].astype(np.float64)
    for aref, mref in refs:
        h = attn_f64(h, *aref, cos, sin)
        h, gap = moe_block_f64(h, mref)
        assert gap > 1e-3, f"route gap {gap}: pick another seed"
    hn = h / np.sqrt((h * h).mean(1, keepdims=True) + pf.RMS_EPS)
    want = hn @ uw.T
    err = np.abs(got - want)
    assert (err <= 2e-3 + 1e-2 * np.abs(want)).all(), f"max abs err {err.max()}"
    info = pf.build_label_info(pf.V2_NER_CLASS_NAMES)
    dec = pf.ViterbiDecoder(info)
    assert dec.decode(pf.log_softmax_rows(got[:, :33])) == \
        dec.decode(pf.log_softmax_rows(want[:, :33].astype(np.float32)))


def test_graphed_forward_replays_equal_eager():
    # Replays with eager work and synchronisations between them, each against
    # the eager forward of the same ids (graph nodes must hold no memsets).
    rng = np.random.default_rng(21)
    blocks = [pf.Block(make_attn(rng)[0], moe_block(rng)) for _ in range(2)]
    unembed, _, _ = qlinear(rng, 36, 640, 640, bias=False)
    emb = rng.standard_normal((50, 640)).astype(np.float32)
    model = pf.PrivacyFilterModel(emb, blocks, torch.ones(640, device=DEV), unembed)
    say("graphed forward, lengths 17, 40, 64")
    gf = pf.GraphedForward(model, [17, 40, 64])
    for rep in range(3):
        for t in (40, 17, 64):
            ids = rng.integers(0, 50, size=t)
            got = gf(ids).clone()
            torch.cuda.synchronize()
            want = model.forward(ids)
            torch.cuda.synchronize()
            assert torch.equal(got, want), (rep, t)
    # the graphs pin the workspace: a call that needs more than it holds
    # (a layer whose act and partial products alone are 1.5 GB, more than any
    # earlier test of this process grew it to) is refused before any launch
    # instead of moving it under them; after close() the graphs are gone
    import runntime_amd as rt
    from runntime_amd.errors import RunntimeError
    from runntime_amd.synth import MoeConfig, make_inputs
    big = MoeConfig("pin_T8192", 8192, 2048, 8, 8, 2048, "f16")
    inp = make_inputs(big, seed=1)
    with pytest.raises(RunntimeError, match="pinned"):
        rt.moe_layer(inp.x, inp.router_w, inp.router_b, inp.glu, inp.lin, inp.down, None, big.k)
    torch.cuda.synchronize()
    gf.close()
    with pytest.raises(RuntimeError, match="closed"):
        gf(rng.integers(0, 50, size=17))
    ids = rng.integers(0, 50, size=40)
    assert torch.isfinite(model.forward(ids)).all()


@pytest.mark.parametrize("T,K,N,bias,add", [(1, 640, 1152, True, False), (56, 896, 640, True, True),
                                            (300, 640, 36, False, False), (1031, 37, 8, True, True),
                                            (5, 100, 260, False, True)])
def test_linear_shapes(T, K, N, bias, add):
    say(f"linear T={T} K={K} N={N} bias={bias} addend={add}")
    rng = np.random.default_rng(T + K)
    w = rng.standard_normal((N, K)).astype(np.float32) / np.sqrt(K)
    b = rng.standard_normal(N).astype(np.float32) if bias else None
    lin = Linear.from_torch_layout(w, b, DEV)
    x = rng.standard_normal((T, K)).astype(np.float32)
    a = rng.standard_normal((T, N)).astype(np.float32) if add else None
    got = lin.forward(torch.from_numpy(x).to(DEV), torch.from_numpy(a).to(DEV) if add else None)
    torch.cuda.synchronize()
    want = x.astype(np.float64) @ w.T.astype(np.float64)
    if bias:
        want += b
    if add:
        want += a
    np.testing.assert_allclose(got.cpu().numpy(), want, atol=2e-5, rtol=1e-5)
