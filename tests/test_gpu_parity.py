"""Parity of the HIP path (libmoe.so through the C ABI) with the CPU oracle.

Bars: expert ids and the dispatch permutation bit-exact; route weights and
outputs within |got − want| ≤ 2e-3 + 1e-2·|want| of the oracle's f64 result
(the layer bar), and, where the reference's own kernel tests apply, within
their tighter atol 1e-5·K, rtol 1e-4 (moeQuantW.gpu.test.ts:100,127)."""
import math

import numpy as np
import pytest
import torch

import runntime_amd as rt
from oracle import ref
from runntime_amd.quantw import QuantExpertWeight, QuantW
from runntime_amd.synth import CONFIGS, make_inputs
from tests.helpers import assert_close, random_quant_weight, route_for

pytestmark = pytest.mark.gpu

DEV = "cuda"


def say(msg):
    print(msg, flush=True)


def gpu(a, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a))
    if dtype is not None:
        t = t.to(dtype)
    return t.to(DEV)


def host(t):
    torch.cuda.synchronize()
    return t.float().cpu().numpy() if t.dtype != torch.int32 else t.cpu().numpy()


def weight_pair(E, K, N, bits, g, seed, with_bias=True):
    q, sc = random_quant_weight(E, K, N, bits, g, seed)
    bias = ref.lcg_f32(E * N, seed + 2).reshape(E, N) if with_bias else None
    words = ref.pack_ekn(q, bits)
    dev = QuantExpertWeight(QuantW(gpu(words.view(np.int32)), (E * K, N)), gpu(sc),
                            gpu(bias) if with_bias else None)
    return dev, (words, sc, bias)


# -------------------------------------------------------------------- topk


@pytest.mark.parametrize("dtype", ["f32", "f16"])
@pytest.mark.parametrize("shape", [(3, 4), (7, 9), (65, 32), (5, 1000)])
@pytest.mark.parametrize("k", [4, 1, 2, 8])
def test_topk_shapes(dtype, shape, k):
    rows, cols = shape
    if cols < k:
        pytest.skip("fewer columns than k")
    say(f"topk {dtype} {shape} k={k}")
    x = ref.lcg_f32(rows * cols, 1).reshape(rows, cols) * 4
    if dtype == "f16":
        x = x.astype(np.float16).astype(np.float32)
    xt = gpu(x, torch.float16 if dtype == "f16" else torch.float32)
    got = host(rt.topk(xt, k))
    want = ref.topk(x, k)
    assert np.array_equal(got[:, :k], want[:, :k])
    np.testing.assert_allclose(got[:, k:], want[:, k:], atol=1e-7, rtol=1e-5)


def test_topk_ties_and_start_value(vectors):
    say("topk ties")
    v = vectors["topk_ties"]
    got = host(rt.topk(gpu(np.array(v["x"], np.float32)), 4))
    assert got[0, :4].tolist() == v["ids"][0]
    assert got[1, :4].tolist() == v["ids"][1]
    assert got[1, 4:].tolist() == v["weights_row1"]
    v = vectors["topk_neg_inf"]
    x = np.array([[float(a) for a in row] for row in v["x"]], np.float32)
    assert host(rt.topk(gpu(x), 4)).tolist() == v["route"]


def test_topk_k16_many_experts():
    say("topk k=16 E=4096")
    x = (ref.lcg_f32(33 * 4096, 3).reshape(33, 4096) * 8).round()  # many ties
    got = host(rt.topk(gpu(x), 16))
    want = ref.topk(x, 16)
    assert np.array_equal(got[:, :16], want[:, :16])
    np.testing.assert_allclose(got[:, 16:], want[:, 16:], atol=1e-7, rtol=1e-5)


def test_topk_past_grid_stride():
    # topkSelect.gpu.test.ts:74-84: GRID_Y_STRIDE + 5 rows of 4 columns.
    rows = 65535 * 64 + 5
    say(f"topk rows={rows}")
    i = np.arange(rows * 4, dtype=np.int64)
    x = (((i * 7) % 13) - (i % 4)).astype(np.float32).reshape(rows, 4)
    got = host(rt.topk(gpu(x), 4))
    want = ref.topk(x, 4)
    assert np.array_equal(got[:, :4], want[:, :4])
    np.testing.assert_allclose(got[:, 4:], want[:, 4:], atol=1e-7, rtol=1e-5)


# ------------------------------------------------------------------ router


@pytest.mark.parametrize("T,d,E,k,dtype", [
    (64, 512, 8, 2, "f32"), (1, 640, 128, 4, "f32"), (8, 2048, 64, 8, "f16"),
    (300, 2048, 32, 4, "f16"), (257, 200, 128, 8, "f32"), (5, 64, 512, 16, "f32"),
])
def test_router_topk_bit_exact(T, d, E, k, dtype):
    say(f"router T={T} d={d} E={E} k={k} {dtype}")
    g = torch.Generator().manual_seed(T * 7 + E)
    x = torch.randn((T, d), generator=g)
    if dtype == "f16":
        x = x.half()
    w = torch.randn((d, E), generator=g) * 0.02
    b = torch.randn((E,), generator=g) * 0.1
    got = host(rt.router_topk(x.to(DEV), w.to(DEV), b.to(DEV), k))
    logits = ref.router_logits(x.float().numpy(), w.numpy(), b.numpy())
    want = ref.topk(logits, k)
    assert np.array_equal(got[:, :k], want[:, :k]), "expert ids differ"
    np.testing.assert_allclose(got[:, k:], want[:, k:], atol=1e-7, rtol=1e-5)


# ---------------------------------------------------------------- dispatch


@pytest.mark.parametrize("T,k,E", [(1, 4, 128), (8, 8, 64), (4096, 4, 32), (4096, 8, 128),
                                   (1000, 3, 7), (2049, 2, 1024)])
def test_dispatch_bit_exact(T, k, E):
    say(f"dispatch T={T} k={k} E={E}")
    rng = np.random.default_rng(T + k + E)
    route = np.zeros((T, 2 * k), np.float32)
    route[:, :k] = rng.integers(0, E, size=(T, k))
    if T > 8:  # a few ids that are not experts
        route[::97, 0] = -1
        route[::101, k - 1] = E + 3
        route[::103, 0] = 0.5
    perm, offsets = rt.dispatch(gpu(route), E)
    want_perm, _, want_off = ref.dispatch(route, E)
    assert np.array_equal(host(offsets), want_off)
    assert np.array_equal(host(perm), want_perm)


# ---------------------------------------------------- expert products (ops)

# The reference test's shapes (moeQuantW.gpu.test.ts:134-144) plus shapes
# that take the MFMA path (groupSize K or a multiple of 32), with rows per
# expert above 16, K tails and N not a multiple of 64.
REF_SHAPES = [(1, 4, 8, 1, 4), (3, 16, 24, 4, 8), (2, 132, 8, 3, 4), (2, 64, 72, 5, 64),
              (5, 32, 16, 8, 16)]
MFMA_SHAPES = [(3, 64, 72, 5, 64), (40, 96, 136, 6, 32), (100, 100, 80, 3, 100),
               (17, 2048, 1408, 4, 2048), (64, 512, 1024, 8, 512), (9, 640, 640, 16, 64)]


def _check_up(T, K, N, E, g, bits, k=4, xdtype="f32", tol="ref", route=None):
    route = route_for(T, E, k) if route is None else route
    glu, glu_h = weight_pair(E, K, N, bits, g, 10)
    lin, lin_h = weight_pair(E, K, N, bits, g, 20)
    x = (ref.lcg_f32(T * K, 1) * 4).reshape(T, K)
    if xdtype == "f16":
        x = x.astype(np.float16).astype(np.float32)
    xt = gpu(x, torch.float16 if xdtype == "f16" else torch.float32)
    got = host(rt.moeUp(xt, gpu(route), glu, lin, {"bits": bits, "groupSize": g}))
    want = ref.moe_up(x, route, glu_h, lin_h, bits, g, E)
    if tol == "ref":
        np.testing.assert_allclose(got, want, atol=1e-5 * K, rtol=1e-4)
    assert_close(got, want, what="moeUp")


def _check_down(T, K, N, E, g, bits, k=4, route=None):
    route = route_for(T, E, k) if route is None else route
    down, down_h = weight_pair(E, K, N, bits, g, 30)
    act = ref.lcg_f32(T * k * K, 1).reshape(T * k, K)
    res = ref.lcg_f32(T * N, 4).reshape(T, N)
    got = host(rt.moeDown(gpu(act), gpu(route), down, gpu(res), {"bits": bits, "groupSize": g}))
    want = ref.moe_down(act, route, down_h, res, bits, g, E)
    np.testing.assert_allclose(got, want, atol=1e-5 * K, rtol=1e-4)
    assert_close(got, want, what="moeDown")


@pytest.mark.parametrize("bits", [8, 4])
@pytest.mark.parametrize("shape", REF_SHAPES)
def test_moe_up_reference_shapes(bits, shape):
    say(f"moeUp int{bits} {shape}")
    T, K, N, E, g = shape
    _check_up(T, K, N, E, g, bits)


@pytest.mark.parametrize("bits", [8, 4])
@pytest.mark.parametrize("shape", REF_SHAPES)
def test_moe_down_reference_shapes(bits, shape):
    say(f"moeDown int{bits} {shape}")
    T, K, N, E, g = shape
    _check_down(T, K, N, E, g, bits)


@pytest.mark.parametrize("xdtype", ["f32", "f16"])
@pytest.mark.parametrize("shape", MFMA_SHAPES)
@pytest.mark.parametrize("k", [4, 2, 8])
def test_moe_up_mfma(xdtype, shape, k):
    T, K, N, E, g = shape
    if E < k:
        pytest.skip("fewer experts than k")
    say(f"moeUp mfma {xdtype} {shape} k={k}")
    _check_up(T, K, N, E, g, 8, k=k, xdtype=xdtype)


@pytest.mark.parametrize("shape", MFMA_SHAPES)
@pytest.mark.parametrize("k", [4, 8])
def test_moe_down_mfma(shape, k):
    T, K, N, E, g = shape
    if E < k:
        pytest.skip("fewer experts than k")
    say(f"moeDown mfma {shape} k={k}")
    _check_down(T, K, N, E, g, 8, k=k)


# Rows per expert ≥ 64 on average: shapes for the grouped GEMM path. The
# first list keeps K short, below the GEMM's load ring (≥ 18 steps of 32 for
# f16 input, ≥ 12 for f32), so most of it runs the skinny kernel on many rows.
GEMM_SHAPES = [(300, 128, 256, 4, 128), (260, 192, 128, 3, 192), (1000, 256, 384, 8, 256),
               (2048, 512, 640, 16, 512)]
# These take the grouped GEMM: ragged last M-tiles, an N-tile with only part
# of its units (N not a multiple of 256 / 512, and I = 1408's half tile),
# the shortest K the ring takes.
GEMM_UP_SHAPES = [(300, 640, 264, 4, 640), (1000, 768, 1408, 8, 768), (2048, 576, 640, 16, 576),
                  (600, 384, 136, 3, 384)]
# Down: the last two split K into two partial products (few tiles for the
# CUs), added by the combine.
GEMM_DOWN_SHAPES = [(300, 384, 520, 4, 384), (1000, 1408, 2048, 8, 1408), (512, 5632, 256, 4, 5632)]


@pytest.mark.parametrize("xdtype", ["f32", "f16"])
@pytest.mark.parametrize("shape", GEMM_SHAPES + GEMM_UP_SHAPES)
def test_moe_up_grouped_gemm(xdtype, shape):
    T, K, N, E, g = shape
    say(f"moeUp gemm {xdtype} {shape}")
    _check_up(T, K, N, E, g, 8, k=2, xdtype=xdtype)


@pytest.mark.parametrize("shape", GEMM_SHAPES + GEMM_DOWN_SHAPES)
def test_moe_down_grouped_gemm(shape):
    T, K, N, E, g = shape
    say(f"moeDown gemm {shape}")
    _check_down(T, K, N, E, g, 8, k=2)


def _skewed_route(T, k=2):
    """Slot 0 → experts 0-2, slot 1 → experts 5-6 of 8: experts 3, 4 and 7
    get no rows, the others hundreds (uneven)."""
    route = np.zeros((T, 2 * k), np.float32)
    for t in range(T):
        route[t, 0] = t % 3
        route[t, 1] = 5 + (t % 7 == 0)
        route[t, 2:] = (0.625, 0.375)
    return route


@pytest.mark.parametrize("xdtype", ["f32", "f16"])
def test_moe_up_gemm_empty_experts(xdtype):
    say(f"moeUp gemm empty experts {xdtype}")
    T = 1024
    _check_up(T, 640, 264, 8, 640, 8, k=2, xdtype=xdtype, route=_skewed_route(T))


def test_moe_down_gemm_empty_experts():
    say("moeDown gemm empty experts")
    T = 1024
    _check_down(T, 384, 520, 8, 384, 8, k=2, route=_skewed_route(T))


def test_moe_up_past_65535_rows():
    T = math.ceil(65535 / 4) + 1
    say(f"moeUp rows={T * 4}")
    _check_up(T, 4, 8, 2, 4, 8)


def test_moe_down_past_65535_tokens():
    T = 65535 + 2
    say(f"moeDown tokens={T}")
    _check_down(T, 4, 8, 2, 4, 8)


def test_invalid_route_ids_give_zero_rows():
    say("moeUp/moeDown invalid ids")
    E, K, N = 3, 64, 64
    glu, glu_h = weight_pair(E, K, N, 8, K, 10)
    x = ref.lcg_f32(2 * K, 1).reshape(2, K)
    route = np.array([[0, 7, 0.5, 0.5], [-1, 1.5, 0.5, 0.5]], np.float32)
    got = host(rt.moeUp(gpu(x), gpu(route), glu, glu, {"bits": 8, "groupSize": K}))
    want = ref.moe_up(x, route, glu_h, glu_h, 8, K, E)
    assert not got[1:].any()
    assert_close(got, want, what="moeUp")
    out = host(rt.moeDown(gpu(got), gpu(route), glu, gpu(x), {"bits": 8, "groupSize": K}))
    assert_close(out, ref.moe_down(want, route, glu_h, x, 8, K, E), what="moeDown")


# ------------------------------------------------------------- the layer


def _oracle_layer(inp, tokens):
    """Oracle route and output for a subset of tokens (tokens are independent
    in the layer, so a sample checks a full-size run)."""
    cfg = inp.cfg
    x = inp.x[tokens].float().cpu().numpy()
    rw = inp.router_w.cpu().numpy()
    rb = inp.router_b.cpu().numpy()
    logits = ref.router_logits(x, rw, rb)
    route = ref.topk(logits, cfg.k)
    pk = {n: ref.pack_ekn(inp.q[n].numpy(), 8) for n in ("glu", "lin", "down")}
    sc = {n: getattr(inp, n).scales.cpu().numpy() for n in ("glu", "lin", "down")}
    bs = {n: getattr(inp, n).bias.cpu().numpy() for n in ("glu", "lin", "down")}
    act = ref.moe_up(x, route, (pk["glu"], sc["glu"], bs["glu"]), (pk["lin"], sc["lin"], bs["lin"]),
                     8, cfg.d, cfg.E)
    res = inp.residual[tokens].cpu().numpy()
    out = ref.moe_down(act, route, (pk["down"], sc["down"], bs["down"]), res, 8, cfg.I, cfg.E)
    return route, out, logits


def _edge_tokens(ids, E, k, tiles=(128, 64)):
    """Tokens whose assignments sit at the edges of the grouped GEMMs' row
    tiles (128 rows for gate/up, 64 for the int8 down GEMM): each active
    expert's first two rows, the first two and last two rows of its last
    tile of each size, and every row of the hottest expert's last 128-row
    tile (rows in the dispatch's stable order by expert)."""
    flat = ids.astype(np.int64).ravel()
    order = np.argsort(flat, kind="stable")
    counts = np.bincount(flat, minlength=E)
    toks, start = set(), 0
    hot = int(np.argmax(counts))
    for e in range(E):
        n = int(counts[e])
        if n == 0:
            continue
        rows = order[start:start + n]
        pick = list(rows[:2]) + list(rows[-2:])
        for tile in tiles:
            last = (n - 1) // tile * tile
            pick += list(rows[last:last + 2])
            if e == hot and tile == tiles[0]:
                pick += list(rows[last:])
        toks.update(int(a) // k for a in pick)
        start += n
    return toks


@pytest.mark.parametrize("cid,sample", [(1, None), (2, None), (3, None), (4, 256), (5, 256)])
def test_moe_layer_configs(cid, sample):
    cfg = CONFIGS[cid]
    say(f"moe_layer config {cid}: {cfg.name}")
    inp = make_inputs(cfg, seed=cid, keep_q=True, bias_rand=True)
    # a seeded host draw: the test's inputs must not depend on the device RNG
    # state earlier tests leave behind
    g = torch.Generator().manual_seed(100 + cid)
    inp.residual.copy_(torch.randn(tuple(inp.residual.shape), generator=g))
    out, route = rt.moe_layer(inp.x, inp.router_w, inp.router_b, inp.glu, inp.lin, inp.down,
                              inp.residual, cfg.k, return_route=True)
    got_out, got_route = host(out), host(route)
    k = cfg.k
    if sample is None:
        tokens = np.arange(cfg.T)
    else:
        # an even spread of the full-size run plus every token at a row-tile
        # edge of the grouped GEMM
        edge = _edge_tokens(got_route[:, :k], cfg.E, k)
        tokens = np.array(sorted(set(np.linspace(0, cfg.T - 1, sample).astype(int).tolist()) | edge))
        say(f"  checking {len(tokens)} of {cfg.T} tokens ({len(edge)} at tile edges)")
    want_route, want_out, logits = _oracle_layer(inp, tokens)
    assert np.array_equal(got_route[tokens, :k], want_route[:, :k]), "expert ids differ"
    np.testing.assert_allclose(got_route[tokens, k:], want_route[:, k:], atol=1e-7, rtol=1e-5)
    assert_close(got_out[tokens], want_out, what=f"config {cid} output")
    # every token routes to k distinct experts
    ids = got_route[:, :k]
    assert all(len(set(r)) == k for r in ids.tolist())


@pytest.mark.parametrize("T,d,E,k,I,x_dtype", [(1, 640, 128, 4, 640, "f16"), (1, 640, 128, 4, 640, "f32"),
                                               (2, 512, 8, 2, 1024, "f32"), (1, 2048, 64, 8, 1408, "f16"),
                                               (3, 256, 16, 4, 384, "f16")])
def test_moe_layer_small_calls(T, d, E, k, I, x_dtype):
    """Single-token and few-token calls, where the decode kernels split each
    weight stream over four (or two) wavefronts and keep act in dispatch
    order between the products: every token against the oracle."""
    import dataclasses
    cfg = dataclasses.replace(CONFIGS[2], name="small", T=T, d=d, E=E, k=k, I=I, x_dtype=x_dtype)
    say(f"moe_layer small call T={T} d={d} E={E} k={k} I={I} {x_dtype}")
    inp = make_inputs(cfg, seed=40 + T, keep_q=True, bias_rand=True)
    g = torch.Generator().manual_seed(41)
    inp.residual.copy_(torch.randn(tuple(inp.residual.shape), generator=g))
    out, route = rt.moe_layer(inp.x, inp.router_w, inp.router_b, inp.glu, inp.lin, inp.down,
                              inp.residual, k, return_route=True)
    got_out, got_route = host(out), host(route)
    tokens = np.arange(T)
    want_route, want_out, _ = _oracle_layer(inp, tokens)
    assert np.array_equal(got_route[:, :k], want_route[:, :k]), "expert ids differ"
    np.testing.assert_allclose(got_route[:, k:], want_route[:, k:], atol=1e-7, rtol=1e-5)
    assert_close(got_out, want_out, what="small call output")


@pytest.mark.parametrize("d,E,k,x_dtype,calls", [(640, 128, 4, "f32", 1), (2048, 64, 8, "f16", 1),
                                                  (640, 128, 4, "f32", 5), (200, 20, 16, "f16", 1),
                                                  (1024, 256, 2, "f32", 3), (64, 4, 1, "f32", 1),
                                                  (132, 8, 8, "f32", 1), (1024, 256, 16, "f16", 1)])
def test_single_token_route_is_the_routers(d, E, k, x_dtype, calls):
    """A single single-token call takes the router's fold, top-k and
    dispatch into the gate/up kernel's prologue; batched single-token calls
    keep the router's own fold kernel. Either way the route row is the
    standalone router's bit for bit (ids and gates), in every call, and the
    output is the oracle's."""
    import dataclasses
    cfg = dataclasses.replace(CONFIGS[2], name="t1", T=1, d=d, E=E, k=k, I=384, x_dtype=x_dtype)
    say(f"single-token route d={d} E={E} k={k} {x_dtype} calls={calls}")
    from runntime_amd.synth import make_weight_copies
    wc = make_weight_copies(cfg, calls, seed=51, device="cpu")
    g = torch.Generator().manual_seed(52)
    xdt = torch.float16 if x_dtype == "f16" else torch.float32
    x = torch.randn((calls, 1, d), generator=g).to(xdt)
    res = torch.randn((calls, 1, d), generator=g)
    wc.router_b.copy_(torch.randn((calls, E), generator=g) * 0.1)
    dev = lambda t: t.to(DEV)
    dw = lambda w: QuantExpertWeight(QuantW(dev(w.w.words), w.w.dims), dev(w.scales), dev(w.bias))
    out, route = rt.moe_layer_batched(dev(x), dev(wc.router_w), dev(wc.router_b), dw(wc.glu),
                                      dw(wc.lin), dw(wc.down), dev(res), k)
    out, route = host(out), host(route)
    for c in range(calls):
        want = host(rt.router_topk(dev(x[c]), dev(wc.router_w[c]), dev(wc.router_b[c]), k))
        assert np.array_equal(route[c], want), f"call {c}: route differs from the router's"
    xs = x[0].float().numpy()
    wt = lambda w: (w.w.words[0].numpy().view(np.uint32), w.scales[0].numpy(), w.bias[0].numpy())
    want_route = ref.topk(ref.router_logits(xs, wc.router_w[0].numpy(), wc.router_b[0].numpy()), k)
    assert np.array_equal(route[0][:, :k], want_route[:, :k])
    act = ref.moe_up(xs, want_route, wt(wc.glu), wt(wc.lin), 8, d, E)
    want_out = ref.moe_down(act, want_route, wt(wc.down), res[0].numpy(), 8, cfg.I, E)
    assert_close(out[0], want_out, what="single-token call 0")


@pytest.mark.parametrize("T,E,k,x_dtype", [(64, 64, 16, "f32"), (17, 32, 8, "f16"),
                                           (64, 128, 4, "f32"), (65, 16, 4, "f32")])
def test_moe_layer_fused_router_dispatch_limits(T, E, k, x_dtype):
    """Calls of up to 64 tokens (T·k ≤ 1024) route and dispatch in one
    kernel whose wavefronts take several tokens each; 65 tokens take the
    separate dispatch. Routes bit-exact, outputs at the layer bar."""
    from runntime_amd.synth import MoeConfig
    cfg = MoeConfig(f"fused_T{T}_E{E}_k{k}", T, 256, E, k, 256, x_dtype)
    say(f"moe_layer {cfg.name}")
    inp = make_inputs(cfg, seed=T + E, keep_q=True, bias_rand=True)
    out, route = rt.moe_layer(inp.x, inp.router_w, inp.router_b, inp.glu, inp.lin, inp.down,
                              inp.residual, k, return_route=True)
    got_out, got_route = host(out), host(route)
    tokens = np.arange(T)
    want_route, want_out, _ = _oracle_layer(inp, tokens)
    assert np.array_equal(got_route[:, :k], want_route[:, :k]), "expert ids differ"
    assert_close(got_out, want_out, what=f"{cfg.name} output")


def test_moe_layer_matches_ops():
    """moe_layer = topk(router) → moeUp → moeDown composed from the ops."""
    cfg = CONFIGS[1]
    say("moe_layer vs ops")
    inp = make_inputs(cfg, seed=11, bias_rand=True)
    out, route = rt.moe_layer(inp.x, inp.router_w, inp.router_b, inp.glu, inp.lin, inp.down,
                              inp.residual, cfg.k, return_route=True)
    r2 = rt.router_topk(inp.x, inp.router_w, inp.router_b, cfg.k)
    assert torch.equal(route, r2)
    act = rt.moeUp(inp.x, r2, inp.glu, inp.lin, {"bits": 8, "groupSize": cfg.d})
    o2 = rt.moeDown(act, r2, inp.down, inp.residual, {"bits": 8, "groupSize": cfg.I})
    assert_close(host(out), host(o2), atol=1e-5, rtol=1e-5, what="layer vs ops")


# --------------------------------------------------------- batched calls


def _slice_weight(w, c):
    return QuantExpertWeight(QuantW(w.w.words[c], w.w.dims), w.scales[c], w.bias[c])


@pytest.mark.parametrize("T,cfg_id", [(1, 2), (5, 1), (40, 1)])
def test_moe_layer_batched_equals_single_calls(T, cfg_id):
    """Each call of a batch is the same computation as a standalone
    moe_layer call on that call's slices (bit for bit), and the first call
    matches the oracle."""
    from runntime_amd.synth import make_weight_copies
    cfg = CONFIGS[cfg_id]
    C = 3
    say(f"moe_layer_batched T={T} calls={C} {cfg.name}")
    wc = make_weight_copies(cfg, C, seed=5, device="cpu")
    g = torch.Generator().manual_seed(3)
    x = torch.randn((C, T, cfg.d), generator=g)
    res = torch.randn((C, T, cfg.d), generator=g)
    wc.router_b.copy_(torch.randn((C, cfg.E), generator=g) * 0.1)
    for w in (wc.glu, wc.lin, wc.down):
        w.bias.copy_(torch.randn(w.bias.shape, generator=g) * 0.1)
    dev = lambda t: t.to(DEV)
    dw = lambda w: QuantExpertWeight(QuantW(dev(w.w.words), w.w.dims), dev(w.scales), dev(w.bias))
    out, route = rt.moe_layer_batched(dev(x), dev(wc.router_w), dev(wc.router_b), dw(wc.glu),
                                      dw(wc.lin), dw(wc.down), dev(res), cfg.k)
    out, route = host(out), host(route)
    for c in range(C):
        o1, r1 = rt.moe_layer(dev(x[c]), dev(wc.router_w[c]), dev(wc.router_b[c]),
                              dw(_slice_weight(wc.glu, c)), dw(_slice_weight(wc.lin, c)),
                              dw(_slice_weight(wc.down, c)), dev(res[c]), cfg.k, return_route=True)
        assert np.array_equal(host(r1), route[c])
        assert np.array_equal(host(o1), out[c])
    # call 0 against the oracle
    xs = x[0].numpy()
    want_route = ref.topk(ref.router_logits(xs, wc.router_w[0].numpy(), wc.router_b[0].numpy()),
                          cfg.k)
    assert np.array_equal(route[0][:, :cfg.k], want_route[:, :cfg.k])
    wt = lambda w: (w.w.words[0].numpy().view(np.uint32), w.scales[0].numpy(), w.bias[0].numpy())
    act = ref.moe_up(xs, want_route, wt(wc.glu), wt(wc.lin), 8, cfg.d, cfg.E)
    want = ref.moe_down(act, want_route, wt(wc.down), res[0].numpy(), 8, cfg.I, cfg.E)
    assert_close(out[0], want, what="batched call 0")


def test_moe_layer_batched_config3_shape():
    """Batched calls at config 3's shape (f16 x, d = 2048, E = 64, k = 8,
    I = 1408: the launch shape of config 3's bench line, with 4 KB+ weight
    units) equal standalone moe_layer calls on each call's slices, bit for
    bit."""
    from runntime_amd.synth import make_weight_copies
    cfg = CONFIGS[3]
    C = 3
    say(f"moe_layer_batched T={cfg.T} calls={C} {cfg.name}")
    wc = make_weight_copies(cfg, C, seed=11, device=DEV)
    g = torch.Generator(device=DEV).manual_seed(4)
    x = torch.randn((C, cfg.T, cfg.d), generator=g, device=DEV).half()
    res = torch.randn((C, cfg.T, cfg.d), generator=g, device=DEV)
    for w in (wc.glu, wc.lin, wc.down):
        w.bias.copy_(torch.randn(w.bias.shape, generator=g, device=DEV) * 0.1)
    out, route = rt.moe_layer_batched(x, wc.router_w, wc.router_b, wc.glu, wc.lin, wc.down, res,
                                      cfg.k)
    for c in range(C):
        o1, r1 = rt.moe_layer(x[c], wc.router_w[c], wc.router_b[c], _slice_weight(wc.glu, c),
                              _slice_weight(wc.lin, c), _slice_weight(wc.down, c), res[c], cfg.k,
                              return_route=True)
        assert torch.equal(r1, route[c])
        assert torch.equal(o1, out[c])


def test_graph_replay_matches_eager():
    """A captured moe_layer_batched replays correctly several times, with
    eager work and synchronisation between the replays."""
    from runntime_amd import perf
    from runntime_amd.synth import make_weight_copies
    cfg = CONFIGS[2]
    C = 4
    say("graph replay")
    wc = make_weight_copies(cfg, C, seed=8, device=DEV)
    x = torch.randn((C, 1, cfg.d), device=DEV)
    res = torch.zeros((C, 1, cfg.d), device=DEV)
    out = torch.empty((C, 1, cfg.d), device=DEV)
    route = torch.empty((C, 1, 2 * cfg.k), device=DEV)
    run = lambda: rt.moe_layer_batched(x, wc.router_w, wc.router_b, wc.glu, wc.lin, wc.down, res,
                                       cfg.k, out=out, route=route)
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        perf.reserve_batched(C, 1, cfg.d, cfg.I, cfg.E, cfg.k)
        run()
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=s):
            run()
        for i in range(4):
            x.copy_(torch.randn((C, 1, cfg.d), device=DEV))
            run()  # eager reference for these inputs
            torch.cuda.synchronize()
            want_out, want_route = out.clone(), route.clone()
            out.zero_()
            route.zero_()
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(route, want_route), f"replay {i}: route"
            assert torch.equal(out, want_out), f"replay {i}: out"


# -------------------------------------------------------------- quantW pack


@pytest.mark.parametrize("bits", [8, 4])
@pytest.mark.parametrize("E,k,n", [(1, 4, 4), (3, 8, 12), (5, 64, 36), (2, 640, 640)])
def test_pack_quant_w_device_matches_packquantw(bits, E, k, n):
    say(f"pack int{bits} E={E} k={k} n={n}")
    lo, hi = (-8, 8) if bits == 4 else (-128, 128)
    ints = np.random.default_rng(E * 1000 + k + n).integers(lo, hi, size=(E, n, k), dtype=np.int8)
    got = host(rt.pack_quant_w_device(gpu(ints), bits).words).view(np.uint32)
    want = np.concatenate([ref.pack_nk(ints[e], k, n, bits) for e in range(E)])
    np.testing.assert_array_equal(got, want)


# ----------------------------------------------------------- weight upload


@pytest.mark.parametrize("raw", [False, True])
def test_uploaded_weights_match_device_tensors(raw):
    """moeUp through the C ABI with moe_weights_upload's buffers equals moeUp
    with the same weights as torch tensors; raw int8 [E][N][K] is packed on
    the device (packQuantW)."""
    import ctypes
    from runntime_amd import _lib
    say(f"upload raw={raw}")
    T, K, N, E, g, k = 40, 96, 136, 6, 32, 4
    glu, (gw, gs, gb) = weight_pair(E, K, N, 8, g, 10)
    lin, (lw, ls, lb) = weight_pair(E, K, N, 8, g, 20)
    if raw:
        qg = np.stack([ref.unpack(gw, E, K, N, 8)[e].T for e in range(E)])  # [E][N][K]
        ql = np.stack([ref.unpack(lw, E, K, N, 8)[e].T for e in range(E)])
        ug = rt.upload_expert_weight(qg.astype(np.int8), gs, gb, E, K, N, 8, g, raw_int8=True)
        ul = rt.upload_expert_weight(ql.astype(np.int8), ls, lb, E, K, N, 8, g, raw_int8=True)
    else:
        ug = rt.upload_expert_weight(gw, gs, gb, E, K, N, 8, g)
        ul = rt.upload_expert_weight(lw, ls, lb, E, K, N, 8, g)
    route = route_for(T, E, k)
    x = (ref.lcg_f32(T * K, 1) * 4).reshape(T, K)
    xt, rt_route = gpu(x), gpu(route)
    want = host(rt.moeUp(xt, rt_route, glu, lin, {"bits": 8, "groupSize": g}))
    act = torch.empty((T * k, N), device=DEV)
    lib = _lib.load()
    vg, vl = ug.view(), ul.view()
    ctx = _lib.context(0, torch.cuda.current_stream().cuda_stream)
    _lib.check(lib.moe_up(ctx, xt.data_ptr(), _lib.MOE_F32, rt_route.data_ptr(), ctypes.byref(vg),
                          ctypes.byref(vl), T, K, N, E, k, 8, g, act.data_ptr()))
    assert np.array_equal(host(act), want)
    ug.dispose()
    with pytest.raises(rt.RunntimeError) as ei:
        ug.view()
    assert ei.value.code == "RESOURCE_DISPOSED"


def test_upload_rejects_an_empty_shape():
    """moeQuantW.gpu.test.ts:167-171: an empty upload is INVALID_ARGUMENT."""
    say("upload empty")
    with pytest.raises(rt.RunntimeError) as ei:
        rt.upload_expert_weight(np.zeros(0, np.uint32), np.zeros(0, np.float32), None,
                                0, 4, 4, 8, 4)
    assert ei.value.code == "INVALID_ARGUMENT"
    assert "no elements" in str(ei.value)


def test_results_are_ordered_with_torchs_default_stream():
    """Torch reports its default stream as handle 0; the library must then
    enqueue on that same null stream. Torch work issued right after a call
    (a comparison, a host copy) with no explicit synchronisation sees the
    finished results. A ~2 ms prefill layer makes any missing ordering show:
    the copy would run while the kernels still write."""
    cfg = CONFIGS[4]
    say("ordering with the default stream, config 4 layer")
    inp = make_inputs(cfg, seed=41)
    assert torch.cuda.current_stream().cuda_stream == 0
    out = rt.moe_layer(inp.x, inp.router_w, inp.router_b, inp.glu, inp.lin, inp.down,
                       inp.residual, cfg.k)
    again = rt.moe_layer(inp.x, inp.router_w, inp.router_b, inp.glu, inp.lin, inp.down,
                         inp.residual, cfg.k)
    same = torch.equal(out, again)  # a torch kernel, queued right behind the layer
    first = out.cpu()               # a copy on the default stream, no synchronize
    torch.cuda.synchronize()
    assert same
    assert torch.equal(first, out.cpu())
    assert first.abs().sum() > 0


# ------------------------------------------------- single-token calls

# T = 1 (the decode configs' case): routes with distinct experts, one expert
# in three slots (three rows of one expert's group), and ids that are not
# experts.
ROUTES_T1 = {
    "distinct": lambda E: [0, 3 % E, 1, E - 1],
    "duplicate": lambda E: [2 % E, 2 % E, 0, 2 % E],
    "invalid": lambda E: [1, -1, 3 % E, 1.5],
}


def _route_t1(kind, E):
    ids = ROUTES_T1[kind](E)
    return np.array([ids + [0.4, 0.3, 0.2, 0.1]], np.float32)


@pytest.mark.parametrize("kind", list(ROUTES_T1))
@pytest.mark.parametrize("xdtype", ["f32", "f16"])
@pytest.mark.parametrize("K,N,E", [(128, 72, 5), (640, 640, 16), (1408, 136, 6), (256, 2048, 8)])
def test_single_token_up(K, N, E, xdtype, kind):
    say(f"moeUp T=1 {xdtype} K={K} N={N} E={E} {kind}")
    _check_up(1, K, N, E, K, 8, k=4, xdtype=xdtype, route=_route_t1(kind, E))


@pytest.mark.parametrize("kind", list(ROUTES_T1))
@pytest.mark.parametrize("K,N,E", [(128, 72, 5), (640, 640, 16), (512, 2048, 8), (384, 136, 6)])
def test_single_token_down(K, N, E, kind):
    say(f"moeDown T=1 K={K} N={N} E={E} {kind}")
    _check_down(1, K, N, E, K, 8, k=4, route=_route_t1(kind, E))


def test_single_token_batch_on_shared_weights():
    """160 single-token calls on shared config-2 weights (stride 0): calls
    0, 77 and 159 against the oracle; every 16th call against its own
    standalone moe_layer call. (A lone call has few streams and takes the
    K-split variant, a different summation order: equal to ~1e-6, not bit
    for bit.)"""
    cfg = CONFIGS[2]
    C = 160
    say(f"moe_layer_batched T=1 calls={C} shared weights")
    inp = make_inputs(cfg, seed=12, keep_q=True, bias_rand=True)
    g = torch.Generator().manual_seed(8)
    x = torch.randn((C, 1, cfg.d), generator=g).to(DEV)
    res = torch.randn((C, 1, cfg.d), generator=g).to(DEV)
    out, route = rt.moe_layer_batched(x, inp.router_w, inp.router_b, inp.glu, inp.lin, inp.down,
                                      res, cfg.k)
    out, route = host(out), host(route)
    pk = {n: ref.pack_ekn(inp.q[n].numpy(), 8) for n in ("glu", "lin", "down")}
    w = {n: (pk[n], getattr(inp, n).scales.cpu().numpy(), getattr(inp, n).bias.cpu().numpy())
         for n in ("glu", "lin", "down")}
    for c in (0, 77, 159):
        xs = x[c].cpu().numpy()
        want_route = ref.topk(ref.router_logits(xs, inp.router_w.cpu().numpy(),
                                                inp.router_b.cpu().numpy()), cfg.k)
        assert np.array_equal(route[c][:, :cfg.k], want_route[:, :cfg.k])
        act = ref.moe_up(xs, want_route, w["glu"], w["lin"], 8, cfg.d, cfg.E)
        want = ref.moe_down(act, want_route, w["down"], res[c].cpu().numpy(), 8, cfg.I, cfg.E)
        assert_close(out[c], want, what=f"call {c}")
    for c in range(0, C, 16):
        o1 = rt.moe_layer(x[c], inp.router_w, inp.router_b, inp.glu, inp.lin, inp.down,
                          res[c], cfg.k)
        assert_close(host(o1), out[c], atol=1e-5, rtol=1e-5, what=f"call {c} vs its single call")
