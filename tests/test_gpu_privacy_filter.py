"""The privacy-filter attention block (attnBlock.ts:28-57) on the GPU
against an f64 composition of the pinned pieces (rmsNorm, dequantized
Linears, oracle rope_f64 and sdpa_f64, + x), with int8 group-quantized qkv
and out projections; and the model forward (model.ts:62-75) equal to its
own chain of block calls, decoded by the Viterbi decoder."""
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


def moe_block(rng, E=8, k=4, I=640):
    def expert(K, N):
        q = rng.integers(-127, 128, size=(E, K, N)).astype(np.int8)
        sc = rng.uniform(0.5e-3, 2e-3, size=(E, N)).astype(np.float32)
        b = rng.standard_normal((E, N)).astype(np.float32) * 0.01
        words = pack_expert_weights(q, 8)
        d = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(DEV)
        return QuantExpertWeight(QuantW(d(words.view(np.int32)), (E * K, N)), d(sc), d(b))
    return MoeBlock(norm_w=torch.from_numpy(rng.uniform(0.5, 1.5, 640).astype(np.float32)).to(DEV),
                    router_w=torch.from_numpy(rng.standard_normal((640, E)).astype(np.float32) * 0.02).to(DEV),
                    router_b=None, glu=expert(640, I), lin=expert(640, I), down=expert(I, 640),
                    E=E, d=640, I=I, bits=8, group_up=640, group_down=I, k=k)


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
