"""Pins the CPU oracle (oracle/moe_oracle.c) before it is trusted as the
checker: against the reference tests' known answers (tests/golden), closed
forms, brute force and invariants chosen so that a dropped term, a wrong
sign or index, or a transposed operand fails one of them."""
import math

import numpy as np
import pytest

from oracle import ref
from runntime_amd import pack_expert_weights, pack_quant_w
from tests.helpers import dense_project, random_quant_weight, route_for, swiglu_np

# --------------------------------------------------------------------- LCG


def test_lcg_matches_reference_recurrence():
    # test/gpu.ts:114-122 by integer arithmetic: s = s·1664525 + 1013904223 mod 2^32.
    s = 1
    want = []
    for _ in range(5):
        s = (s * 1664525 + 1013904223) % 2 ** 32
        want.append(np.float32(s / 2 ** 31 - 1))
    got = ref.lcg_f32(5, 1)
    assert got.tolist() == want
    # first value by hand: 1015568748 / 2^31 − 1
    assert got[0] == np.float32(1015568748 / 2147483648 - 1)


def test_lcg_range():
    v = ref.lcg_f32(100000, 7)
    assert v.min() >= -1.0 and v.max() < 1.0


# ------------------------------------------------------------------ quantW

PACKERS = {
    "oracle_nk": lambda ints, k, n, b: ref.pack_nk(np.array(ints, np.int8), k, n, b),
    "oracle_ekn": lambda ints, k, n, b: ref.pack_ekn(
        np.array(ints, np.int8).reshape(n, k).T.reshape(1, k, n), b),
    "product": lambda ints, k, n, b: pack_quant_w(np.array(ints, np.int8), k, n, b),
}


@pytest.mark.parametrize("packer", list(PACKERS))
def test_pack_hand_worked_words(packer, vectors):
    pack = PACKERS[packer]
    for key in ("quantpack_int8_one_tile", "quantpack_int4_one_tile"):
        v = vectors[key]
        words = pack(v["ints_nk"], v["k"], v["n"], v["bits"])
        assert [int(w) for w in words] == v["words"], key


@pytest.mark.parametrize("packer", list(PACKERS))
def test_pack_twos_complement(packer, vectors):
    pack = PACKERS[packer]
    for v in vectors["quantpack_twos_complement"]:
        bits, mask = v["bits"], v["mask"]
        words = pack(v["ints_nk"], 4, 4, bits)
        unpacked = [(int(words[(i * bits) >> 5]) >> ((i * bits) & 31)) & mask for i in range(16)]
        assert unpacked == [x & mask for x in v["ints_nk"]]


@pytest.mark.parametrize("packer", list(PACKERS))
def test_pack_tile_order(packer, vectors):
    v = vectors["quantpack_tile_order"]
    words = PACKERS[packer](v["ints_nk"], v["k"], v["n"], v["bits"])
    assert len(words) == v["n_words"]
    assert [int(words[t * 4]) & 0xFF for t in range(4)] == v["first_bytes"]


@pytest.mark.parametrize("packer", list(PACKERS))
def test_pack_readback(packer, vectors):
    # quantPack.test.ts:165-192: read back as the kernels read it.
    for v in vectors["quantpack_readback_shapes"]:
        bits, k, n = v["bits"], v["k"], v["n"]
        half = 2 ** (bits - 1)
        ints = [((i * 37 + 5) % (2 * half)) - half for i in range(k * n)]
        words = PACKERS[packer](ints, k, n, bits)
        assert len(words) == k * n * bits // 32
        q = ref.unpack(words, 1, k, n, bits)[0]  # logical [k, n]
        assert q.T.reshape(-1).tolist() == ints


def test_pack_many_experts_roundtrip():
    rng = np.random.default_rng(3)
    for bits in (8, 4):
        half = 2 ** (bits - 1)
        q = rng.integers(-half, half, size=(3, 16, 12)).astype(np.int8)
        w_oracle = ref.pack_ekn(q, bits)
        w_prod = pack_expert_weights(q, bits)
        assert np.array_equal(w_oracle, w_prod)
        assert np.array_equal(ref.unpack(w_oracle, 3, 16, 12, bits), q)


# -------------------------------------------------------------------- topk


def test_topk_ties(vectors):
    v = vectors["topk_ties"]
    route = ref.topk(np.array(v["x"], np.float32), 4)
    assert route[0, :4].tolist() == v["ids"][0]
    assert route[1, :4].tolist() == v["ids"][1]
    assert route[1, 4:].tolist() == v["weights_row1"]
    # row 0: logits 7, 7, 7, 5 → weights e^0, e^0, e^0, e^-2 normalised
    z = 3 + math.exp(-2)
    np.testing.assert_allclose(route[0, 4:], [1 / z, 1 / z, 1 / z, math.exp(-2) / z], rtol=1e-6)


def test_topk_neg_inf_start_value(vectors):
    v = vectors["topk_neg_inf"]
    x = np.array([[float(a) for a in row] for row in v["x"]], np.float32)
    assert ref.topk(x, 4).tolist() == v["route"]


def test_topk_all_below_start_value():
    # No candidate at all: every slot keeps (−3.4e38, id 0), weights 1/k.
    x = np.full((1, 6), -np.inf, np.float32)
    assert ref.topk(x, 4).tolist() == [[0, 0, 0, 0, 0.25, 0.25, 0.25, 0.25]]


def test_topk_nan_never_enters():
    x = np.array([[np.nan, 1, np.nan, 3, 2]], np.float32)
    assert ref.topk(x, 3)[0, :3].tolist() == [3, 4, 1]


@pytest.mark.parametrize("k", [1, 2, 4, 8, 16])
def test_topk_brute_force(k):
    """torch.topk semantics (topkSelect.gpu.test.ts:14-30): a stable sort by
    descending logit, then softmax over the picked k, in f64."""
    rng = np.random.default_rng(k)
    for E in (k, k + 3, 64, 200):
        # integer-valued logits make ties frequent
        x = rng.integers(-5, 6, size=(50, E)).astype(np.float32)
        x[::7] = rng.standard_normal((len(x[::7]), E)).astype(np.float32) * 4
        route = ref.topk(x, k)
        for t in range(len(x)):
            ids = sorted(range(E), key=lambda j: (-float(x[t, j]), j))[:k]
            assert route[t, :k].tolist() == ids
            ex = np.exp(x[t, ids].astype(np.float64) - x[t, ids[0]])
            np.testing.assert_allclose(route[t, k:], ex / ex.sum(), rtol=1e-6, atol=1e-7)


# ------------------------------------------------------------------ router


def test_router_exact_on_integers():
    # Small integers: every product and partial sum is exact in f32, so any
    # order gives the integer matmul. Pins the [d, E] indexing and the bias.
    rng = np.random.default_rng(1)
    for d in (5, 64, 200):
        x = rng.integers(-4, 5, size=(7, d)).astype(np.float32)
        w = rng.integers(-4, 5, size=(d, 9)).astype(np.float32)
        b = rng.integers(-10, 11, size=9).astype(np.float32)
        got = ref.router_logits(x, w, b)
        want = x.astype(np.int64) @ w.astype(np.int64) + b.astype(np.int64)
        assert np.array_equal(got, want.astype(np.float32))
        assert np.array_equal(ref.router_logits(x, w), (want - b).astype(np.float32))


def test_router_near_f64():
    rng = np.random.default_rng(2)
    x = rng.standard_normal((16, 2048)).astype(np.float32)
    w = (rng.standard_normal((2048, 128)) * 0.02).astype(np.float32)
    got = ref.router_logits(x, w).astype(np.float64)
    want = x.astype(np.float64) @ w.astype(np.float64)
    bound = 2048 * 2 ** -24 * (np.abs(x).astype(np.float64) @ np.abs(w).astype(np.float64))
    assert (np.abs(got - want) <= bound).all()


def test_router_chunk_order_is_canonical():
    # A case where summation order shows: chunk 0 sums to 2^24, chunk 1 adds
    # 1s that vanish one at a time, and the fold adds chunk totals.
    d = 128
    x = np.ones((1, d), np.float32)
    w = np.zeros((d, 1), np.float32)
    w[0, 0] = 2.0 ** 24
    w[64:, 0] = 1.0
    got = ref.router_logits(x, w)[0, 0]
    # chunk 0 = 2^24, chunk 1 = 64 exactly, fold: 2^24 + 64 (exact)
    assert got == np.float32(2.0 ** 24 + 64)
    # within one chunk the ones are absorbed one by one: 2^24 + 1 rounds to 2^24
    w2 = np.zeros((d, 1), np.float32)
    w2[0, 0] = 2.0 ** 24
    w2[1:64, 0] = 1.0
    assert ref.router_logits(x, w2)[0, 0] == np.float32(2.0 ** 24)


# ----------------------------------------------------------------- SwiGLU


def test_swiglu_closed_forms():
    sig = lambda z: 1 / (1 + math.exp(-z))
    assert ref.swiglu(0.0, 3.0) == 0.0
    assert ref.swiglu(2.0, -1.0) == 0.0  # l + 1 = 0
    assert ref.swiglu(100.0, 100.0) == pytest.approx(7 * sig(1.702 * 7) * 8, rel=1e-15)
    assert ref.swiglu(7.0, -100.0) == pytest.approx(7 * sig(11.914) * -6, rel=1e-15)
    assert ref.swiglu(1.0, 0.0) == pytest.approx(sig(1.702), rel=1e-15)
    assert abs(ref.swiglu(-50.0, 0.0)) < 1e-30
    # the gate is capped but not floored: negative gates pass through σ
    assert ref.swiglu(-1.0, 1.0) == pytest.approx(-sig(-1.702) * 2, rel=1e-15)


# ---------------------------------------------------------- expert products


def _layer(E, K, N, bits, g, seed):
    q, sc = random_quant_weight(E, K, N, bits, g, seed)
    bias = ref.lcg_f32(E * N, seed + 2).reshape(E, N)
    return q, sc, bias, ref.pack_ekn(q, bits)


def test_moe_up_identity_weights():
    # q = I (per expert, scaled by e+1), scales 0.5: glu = (e+1)·x/2 + bias.
    E, K = 3, 8
    q = np.zeros((E, K, K), np.int8)
    for e in range(E):
        q[e] = np.eye(K, dtype=np.int8) * (e + 1)
    sc = np.full((E, K), 0.5, np.float32)
    gb = np.arange(E * K, dtype=np.float32).reshape(E, K) * 0.01
    zero_q = np.zeros_like(q)
    x = np.linspace(-3, 3, 2 * K, dtype=np.float32).reshape(2, K)
    route = np.array([[2, 0, 0.75, 0.25], [1, 2, 0.5, 0.5]], np.float32)
    act = ref.moe_up(x, route, (ref.pack_ekn(q, 8), sc, gb), (ref.pack_ekn(zero_q, 8), sc, None),
                     8, K, E)
    for t in range(2):
        for s in range(2):
            e = int(route[t, s])
            glu = (e + 1) * x[t].astype(np.float64) / 2 + gb[e]
            # lin = 0 → act = min(glu, 7)·σ(1.702·min(glu, 7))
            g = np.minimum(glu, 7)
            want = g / (1 + np.exp(-1.702 * g))
            np.testing.assert_allclose(act[t * 2 + s], want, rtol=1e-6, atol=1e-7)


@pytest.mark.parametrize("bits", [8, 4])
def test_moe_up_dense_path(bits):
    E, K, N, g, T, k = 5, 64, 72, 16, 6, 3
    qg, sg, bg, wg = _layer(E, K, N, bits, g, 10)
    ql, sl, bl, wl = _layer(E, K, N, bits, g, 20)
    x = (ref.lcg_f32(T * K, 1) * 4).reshape(T, K)
    route = route_for(T, E, k)
    act = ref.moe_up(x, route, (wg, sg, bg), (wl, sl, bl), bits, g, E)
    for t in range(T):
        for s in range(k):
            e = int(route[t, s])
            want = swiglu_np(dense_project(x[t], qg, sg, bg, e, g), dense_project(x[t], ql, sl, bl, e, g))
            np.testing.assert_allclose(act[t * k + s], want, rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("bits", [8, 4])
def test_moe_down_dense_path_and_linearity(bits):
    E, K, N, g, T, k = 4, 32, 16, 32, 5, 4
    q, sc, b, w = _layer(E, K, N, bits, g, 30)
    act = ref.lcg_f32(T * k * K, 1).reshape(T * k, K)
    res = ref.lcg_f32(T * N, 4).reshape(T, N)
    route = route_for(T, E, k)
    out = ref.moe_down(act, route, (w, sc, b), res, bits, g, E)
    for t in range(T):
        want = res[t].astype(np.float64)
        for s in range(k):
            e = int(route[t, s])
            want = want + route[t, k + s] * dense_project(act[t * k + s], q, sc, b, e, g)
        np.testing.assert_allclose(out[t], want, rtol=1e-6, atol=1e-6)
    # linear in act once bias and residual are removed
    act2 = ref.lcg_f32(T * k * K, 9).reshape(T * k, K)
    f = lambda a: ref.moe_down(a, route, (w, sc, None), None, bits, g, E).astype(np.float64)
    np.testing.assert_allclose(f(act + act2), f(act) + f(act2), rtol=1e-5, atol=1e-5)


def test_invalid_route_ids_contribute_nothing():
    E, K, N, g = 2, 8, 8, 8
    q, sc, b, w = _layer(E, K, N, 8, g, 5)
    x = ref.lcg_f32(2 * K, 1).reshape(2, K)
    route = np.array([[0, 7, 0.5, 0.5], [-1, 1.5, 0.5, 0.5]], np.float32)  # k = 2
    act = ref.moe_up(x, route, (w, sc, b), (w, sc, b), 8, g, E)
    assert not act[1].any() and not act[2].any() and not act[3].any()
    assert act[0].any()


@pytest.mark.parametrize("bits", [8, 4])
@pytest.mark.parametrize("shape", range(5))
def test_f32_restatement_meets_reference_tolerance(bits, shape, vectors):
    """The f32 restatement of the reference kernels (the CPU baseline) against
    the f64 oracle at the reference test's own bar: atol 1e-5·K, rtol 1e-4
    (moeQuantW.gpu.test.ts:100,127), on the reference test's own shapes and
    inputs (randomQuantWeight seeds 10/20/30, x = 4·randomF32(seed 1))."""
    s = vectors["moe_shapes"][shape]
    T, K, N, E, g = s["tokens"], s["k"], s["n"], s["experts"], s["groupSize"]
    tol = vectors["moe_tolerance"]
    route = route_for(T, E, 4)
    qg, sg, bg, wg = _layer(E, K, N, bits, g, 10)
    ql, sl, bl, wl = _layer(E, K, N, bits, g, 20)
    x = (ref.lcg_f32(T * K, 1) * 4).reshape(T, K)
    a64 = ref.moe_up(x, route, (wg, sg, bg), (wl, sl, bl), bits, g, E)
    a32 = ref.moe_up(x, route, (wg, sg, bg), (wl, sl, bl), bits, g, E, f32ref=True)
    np.testing.assert_allclose(a32, a64, atol=tol["atol_per_k"] * K, rtol=tol["rtol"])
    q, sc, b, w = _layer(E, K, N, bits, g, 30)
    act = ref.lcg_f32(T * 4 * K, 1).reshape(T * 4, K)
    res = ref.lcg_f32(T * N, 4).reshape(T, N)
    o64 = ref.moe_down(act, route, (w, sc, b), res, bits, g, E)
    o32 = ref.moe_down(act, route, (w, sc, b), res, bits, g, E, f32ref=True)
    np.testing.assert_allclose(o32, o64, atol=tol["atol_per_k"] * K, rtol=tol["rtol"])


# ---------------------------------------------------------------- dispatch


def test_dispatch_is_stable_counting_sort():
    rng = np.random.default_rng(4)
    for T, k, E in ((1, 4, 128), (8, 8, 64), (300, 4, 32), (257, 2, 5)):
        route = np.zeros((T, 2 * k), np.float32)
        route[:, :k] = rng.integers(0, E, size=(T, k))
        perm, inv, offsets = ref.dispatch(route, E)
        ids = route[:, :k].reshape(-1).astype(np.int64)
        want = np.argsort(ids, kind="stable")
        assert np.array_equal(perm, want)
        assert np.array_equal(offsets, np.concatenate([[0], np.cumsum(np.bincount(ids, minlength=E))]))
        assert np.array_equal(perm[inv], np.arange(T * k))


def test_dispatch_drops_invalid_ids():
    route = np.array([[1, -1, 0, 0], [2.5, 0, 0, 0], [np.nan, 5, 0, 0]], np.float32)
    perm, inv, offsets = ref.dispatch(route, 3)
    # valid assignments: a=0 (e1), a=3 (e0) — 5 is out of range for E = 3
    assert offsets.tolist() == [0, 1, 2, 2, 2][:4]
    assert perm.tolist() == [3, 0, -1, -1, -1, -1]
    assert inv.tolist() == [1, -1, -1, 0, -1, -1]
