"""Parity of the pre-norm path (moe_rmsnorm, moe_block) through the C ABI
with the CPU oracle.

rmsNorm is compared bit for bit: the kernel follows the same canonical f32
order as the oracle (lane-strided sums, xor butterfly, correctly rounded
sqrt and division). moe_block (EagerMoeMlp.forward, zoo/privacy-filter/
moeMlp.ts:79-121) is compared as the layer: expert ids bit-exact, outputs
within |got − want| ≤ 2e-3 + 1e-2·|want| of the oracle's f64 products on
the oracle's normalised rows."""
import numpy as np
import pytest
import torch

import runntime_amd as rt
from oracle import ref
from runntime_amd.synth import CONFIGS, make_inputs
from tests.helpers import assert_close
from tests.test_gpu_parity import _edge_tokens
from tests.test_oracle_norm import OPTIONS, SHAPES, inputs

pytestmark = pytest.mark.gpu

DEV = "cuda"


def say(msg):
    print(msg, flush=True)


def tdev(a, dtype):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dtype).to(DEV)


def host(t):
    torch.cuda.synchronize()
    return t.float().cpu().numpy()


TORCH = {"f32": torch.float32, "f16": torch.float16}
NP = {"f32": np.float32, "f16": np.float16}


@pytest.mark.parametrize("dtype", ["f32", "f16"])
@pytest.mark.parametrize("rows,cols", SHAPES)
def test_rmsnorm_bit_exact_reference_shapes(rows, cols, dtype):
    say(f"rmsNorm {dtype} [{rows}, {cols}]")
    x, w, _ = inputs(rows, cols, dtype)
    got = host(rt.rmsNorm(tdev(x, TORCH[dtype]), tdev(w, TORCH[dtype]), 1e-6))
    want = ref.rmsnorm(x, w, 1e-6, dtype=NP[dtype]).astype(np.float32)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("dtype", ["f32", "f16"])
@pytest.mark.parametrize("vec4", [True, False])
@pytest.mark.parametrize("opt", OPTIONS, ids=lambda o: ",".join(f"{k}={v}" for k, v in o.items()))
def test_rmsnorm_bit_exact_options(opt, vec4, dtype):
    group = (8 if vec4 else 6) if opt.get("grouped") else None
    cols = 48 if vec4 else 42
    wlen = cols if (opt.get("sliced") or group is None) else group
    say(f"rmsNorm {dtype} options {opt} cols {cols}")
    x, w, r = inputs(5, cols, dtype, wlen=wlen, residual=opt.get("residual", False))
    eps, scale = opt.get("eps", 1e-6), opt.get("scale", 1.0)
    o = {"scale": scale}
    if group is not None:
        o["group"] = group
    if r is not None:
        o["residual"] = tdev(r, TORCH[dtype])
    got = host(rt.rmsNorm(tdev(x, TORCH[dtype]), tdev(w, TORCH[dtype]), eps, o))
    want = ref.rmsnorm(x, w, eps, group=group, residual=r, scale=scale, dtype=NP[dtype])
    assert np.array_equal(got, want.astype(np.float32))


def test_rmsnorm_wide_random_rows_bit_exact():
    """Many rows of the privacy-filter width (640) and of configs 3-5 (2048),
    with magnitudes spread over decades, so that the sum order matters."""
    g = torch.Generator().manual_seed(4)
    for cols in (640, 2048):
        x = torch.randn((512, cols), generator=g) * torch.exp(torch.randn((512, 1), generator=g) * 3)
        w = 1 + 0.1 * torch.randn(cols, generator=g)
        say(f"rmsNorm wide rows cols={cols}")
        got = host(rt.rmsNorm(x.to(DEV), w.to(DEV), 1e-5))
        want = ref.rmsnorm(x.numpy(), w.numpy(), 1e-5)
        assert np.array_equal(got, want)


def _norm_weight(d, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    return (1 + 0.1 * torch.randn(d, generator=g)).to(TORCH[dtype])


def _oracle_block(inp, norm_w, eps, tokens):
    cfg = inp.cfg
    x = inp.x[tokens].float().cpu().numpy()
    npd = np.float16 if cfg.x_dtype == "f16" else np.float32
    xn = ref.rmsnorm(x, norm_w.float().cpu().numpy(), eps, dtype=npd).astype(np.float32)
    route = ref.topk(ref.router_logits(xn, inp.router_w.cpu().numpy(), inp.router_b.cpu().numpy()),
                     cfg.k)
    pk = {n: ref.pack_ekn(inp.q[n].numpy(), 8) for n in ("glu", "lin", "down")}
    w = {n: (pk[n], getattr(inp, n).scales.cpu().numpy(), getattr(inp, n).bias.cpu().numpy())
         for n in ("glu", "lin", "down")}
    act = ref.moe_up(xn, route, w["glu"], w["lin"], 8, cfg.d, cfg.E)
    out = ref.moe_down(act, route, w["down"], x, 8, cfg.I, cfg.E)
    return route, out


@pytest.mark.parametrize("cid,sample", [(1, None), (2, None), (3, None), (4, 256), (5, 256)])
def test_moe_block_matches_oracle(cid, sample):
    cfg = CONFIGS[cid]
    say(f"moe_block config {cid}: {cfg.name}")
    inp = make_inputs(cfg, seed=20 + cid, keep_q=True, bias_rand=True)
    nw = _norm_weight(cfg.d, cfg.x_dtype, cid).to(DEV)
    out, route = rt.moe_block(inp.x, nw, 1e-5, inp.router_w, inp.router_b, inp.glu, inp.lin,
                              inp.down, cfg.k, return_route=True)
    got_out, got_route = host(out), host(route)
    if sample is None:
        tokens = np.arange(cfg.T)
    else:
        # an even spread plus every token at a row-tile edge of the grouped
        # GEMMs (the prefill path normalises into a copy before them)
        edge = _edge_tokens(got_route[:, :cfg.k], cfg.E, cfg.k)
        tokens = np.array(sorted(set(np.linspace(0, cfg.T - 1, sample).astype(int).tolist()) | edge))
        say(f"  checking {len(tokens)} of {cfg.T} tokens ({len(edge)} at tile edges)")
    want_route, want_out = _oracle_block(inp, nw, 1e-5, tokens)
    k = cfg.k
    assert np.array_equal(got_route[tokens, :k], want_route[:, :k]), "expert ids differ"
    np.testing.assert_allclose(got_route[tokens, k:], want_route[:, k:], atol=1e-7, rtol=1e-5)
    assert_close(got_out[tokens], want_out, what=f"block config {cid}")


@pytest.mark.parametrize("cid,T,x_dtype", [(1, None, None), (3, None, None), (2, 100, None),
                                           (2, 100, "f16"), (2, 40, "f16"), (2, None, "f16"),
                                           (4, None, None)])
def test_moe_block_is_norm_then_layer(cid, T, x_dtype):
    """moe_block = rmsNorm → moe_layer(xn) with residual x, bit for bit.
    The block normalises x while staging it for calls of at most 64 tokens
    whose gate/up product runs on the skinny kernel (configs 1-3 and T = 40:
    the fused router); above 64 tokens it writes a normalised copy first,
    for the register-tiled router (T = 100, whose staged-norm branch is
    refused by the router and so must not be reached: this case passing
    shows the copy path ran) and for the grouped GEMM (config 4)."""
    import dataclasses
    cfg = CONFIGS[cid]
    if T:
        cfg = dataclasses.replace(cfg, T=T)
    if x_dtype:
        cfg = dataclasses.replace(cfg, x_dtype=x_dtype)
    say(f"moe_block composition config {cid} T={cfg.T} {cfg.x_dtype}")
    inp = make_inputs(cfg, seed=30 + cid, bias_rand=True)
    nw = _norm_weight(cfg.d, cfg.x_dtype, 7).to(DEV)
    out, route = rt.moe_block(inp.x, nw, 1e-5, inp.router_w, inp.router_b, inp.glu, inp.lin,
                              inp.down, cfg.k, return_route=True)
    xn = rt.rmsNorm(inp.x, nw, 1e-5)
    o2, r2 = rt.moe_layer(xn, inp.router_w, inp.router_b, inp.glu, inp.lin, inp.down,
                          inp.x.float().contiguous(), cfg.k, return_route=True)
    a, b = host(route), host(r2)
    diff = np.argwhere(a != b)
    assert len(diff) == 0, [(i, j, a[i, j], b[i, j]) for i, j in diff[:8]]
    assert np.array_equal(host(out), host(o2))


@pytest.mark.parametrize("T,d,x_dtype", [(33, 200, "f16"), (10, 2304, None)])
def test_moe_block_staged_norm_row_lengths(T, d, x_dtype):
    """The router's staged pre-norm reads a wavefront's rows together for
    rows of up to 2048 elements (shorter rows in fewer loads per lane) and
    row by row beyond; both stay bit-identical to rmsNorm → moe_layer. T = 33
    leaves the last token tile one token, so most wavefronts have none."""
    import dataclasses
    cfg = dataclasses.replace(CONFIGS[3], T=T, d=d, E=16, I=256)
    if x_dtype:
        cfg = dataclasses.replace(cfg, x_dtype=x_dtype)
    say(f"moe_block staged norm T={T} d={d} {cfg.x_dtype}")
    inp = make_inputs(cfg, seed=40 + d, bias_rand=True)
    nw = _norm_weight(cfg.d, cfg.x_dtype, 9).to(DEV)
    out, route = rt.moe_block(inp.x, nw, 1e-5, inp.router_w, inp.router_b, inp.glu, inp.lin,
                              inp.down, cfg.k, return_route=True)
    xn = rt.rmsNorm(inp.x, nw, 1e-5)
    o2, r2 = rt.moe_layer(xn, inp.router_w, inp.router_b, inp.glu, inp.lin, inp.down,
                          inp.x.float().contiguous(), cfg.k, return_route=True)
    assert np.array_equal(host(route), host(r2))
    assert np.array_equal(host(out), host(o2))
