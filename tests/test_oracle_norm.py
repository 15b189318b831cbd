"""Pins the oracle's rmsNorm (orc_rmsnorm) before it is used as the checker.

The reference's own kernel test (test/core/kernels/reduce/rmsNorm.gpu.test.ts)
compares every route against an f64 formula at atol 1e-6 / rtol 1e-5 (f32)
and atol 1e-3 / rtol 2e-3 (f16), on the shapes and options below; the oracle
must meet that bar on the same inputs (randomF32 seeds 1, 2, 3). Closed
forms pin what the tolerance leaves open: exact results on rows whose sums
are exact, the eps term, the residual and scale order of operations."""
import numpy as np
import pytest

from oracle import ref

TOL = {"f32": (1e-6, 1e-5), "f16": (1e-3, 2e-3)}

# rmsNorm.gpu.test.ts:98-110
SHAPES = [(3, 4), (5, 128), (2, 260), (2, 16384), (70000, 4),
          (1, 1), (3, 7), (4, 65), (37, 642), (70000, 3)]


def rms_ref_f64(x, w, eps=1e-6, group=None, residual=None, scale=1.0):
    """rmsNormRef (rmsNorm.gpu.test.ts:33-56), vectorised, in f64."""
    rows, cols = x.shape
    group = cols if group is None else group
    xg = x.astype(np.float64).reshape(rows, cols // group, group)
    inv = 1.0 / np.sqrt((xg ** 2).sum(-1, keepdims=True) / group + eps)
    wv = w.astype(np.float64)
    wv = wv.reshape(1, 1, group) if wv.size == group else wv.reshape(1, cols // group, group)
    out = (xg * inv * wv).reshape(rows, cols)
    if residual is not None:
        out = out + residual.astype(np.float64)
    return out * scale


def inputs(rows, cols, dtype, wlen=None, residual=False):
    rnd = (lambda a: a.astype(np.float16).astype(np.float32)) if dtype == "f16" else (lambda a: a)
    x = rnd(ref.lcg_f32(rows * cols, 1).reshape(rows, cols))
    w = rnd(ref.lcg_f32(wlen or cols, 2))
    r = rnd(ref.lcg_f32(rows * cols, 3).reshape(rows, cols)) if residual else None
    return x, w, r


def check(got, want, dtype):
    atol, rtol = TOL[dtype]
    err = np.abs(got.astype(np.float64) - want)
    assert (err <= atol + rtol * np.abs(want)).all(), err.max()


@pytest.mark.parametrize("dtype", ["f32", "f16"])
@pytest.mark.parametrize("rows,cols", SHAPES)
def test_reference_shapes_within_reference_tolerance(rows, cols, dtype):
    x, w, _ = inputs(rows, cols, dtype)
    npd = np.float16 if dtype == "f16" else np.float32
    got = ref.rmsnorm(x, w, 1e-6, dtype=npd)
    check(got, rms_ref_f64(x, w), dtype)


# rmsNorm.gpu.test.ts:130-160: every option on the vec4 (groups of 8 in rows
# of 48) and scalar (groups of 6 in rows of 42) routes.
OPTIONS = [
    dict(eps=1e-2), dict(residual=True), dict(scale=0.5), dict(residual=True, scale=2.0),
    dict(grouped=True), dict(grouped=True, sliced=True),
    dict(grouped=True, sliced=True, residual=True, scale=0.5),
]


@pytest.mark.parametrize("dtype", ["f32", "f16"])
@pytest.mark.parametrize("vec4", [True, False])
@pytest.mark.parametrize("opt", OPTIONS, ids=lambda o: ",".join(f"{k}={v}" for k, v in o.items()))
def test_options_within_reference_tolerance(opt, vec4, dtype):
    group = (8 if vec4 else 6) if opt.get("grouped") else None
    cols = 48 if vec4 else 42
    rows = 5
    wlen = cols if (opt.get("sliced") or group is None) else group
    x, w, r = inputs(rows, cols, dtype, wlen=wlen, residual=opt.get("residual", False))
    eps = opt.get("eps", 1e-6)
    scale = opt.get("scale", 1.0)
    npd = np.float16 if dtype == "f16" else np.float32
    got = ref.rmsnorm(x, w, eps, group=group, residual=r, scale=scale, dtype=npd)
    check(got, rms_ref_f64(x, w, eps, group, r, scale), dtype)


def test_constant_row_is_exact():
    # x = 0.5 everywhere: every square and partial sum is exact, so the mean
    # is 0.25 and the output is one correctly rounded chain.
    x = np.full((2, 256), 0.5, np.float32)
    w = np.full(256, 2.0, np.float32)
    got = ref.rmsnorm(x, w, 1e-5)
    inv = np.float32(1.0) / np.sqrt(np.float32(0.25) + np.float32(1e-5))
    assert np.array_equal(got, np.full_like(x, (np.float32(0.5) * inv) * np.float32(2.0)))


def test_zero_row_and_eps():
    x = np.zeros((1, 64), np.float32)
    w = np.ones(64, np.float32)
    assert not ref.rmsnorm(x, w, 1e-5).any()
    # with x ≪ sqrt(eps) the eps term dominates: out ≈ x / sqrt(eps)
    x = np.full((1, 64), 1e-6, np.float32)
    got = ref.rmsnorm(x, w, 1e-2)
    np.testing.assert_allclose(got, 1e-6 / np.sqrt(1e-2), rtol=1e-6)


def test_residual_added_before_scale():
    x, w, r = inputs(3, 16, "f32", residual=True)
    a = ref.rmsnorm(x, w, 1e-6, residual=r, scale=2.0)
    b = ref.rmsnorm(x, w, 1e-6)
    np.testing.assert_allclose(a, (b + r) * 2.0, rtol=1e-6, atol=1e-6)


def test_sum_order_is_the_lane_order():
    """The oracle's sum is the 64-lane strided order with a butterfly, not a
    plain sequential sum: on a row where the two differ, the oracle output
    equals the lane-order value and not the sequential one."""
    rng = np.random.default_rng(7)
    found = False
    for _ in range(50):
        x = (rng.standard_normal((1, 1000)) * np.exp(rng.uniform(-8, 8, (1, 1000)))).astype(np.float32)
        w = np.ones(1000, np.float32)
        seq = np.float32(0)
        for v in x[0]:
            seq = np.float32(seq + np.float32(v * v))
        lanes = np.zeros(64, np.float32)
        for q in range(250):
            for j in range(4):
                v = x[0, 4 * q + j]
                lanes[q % 64] = np.float32(lanes[q % 64] + np.float32(v * v))
        for m in (32, 16, 8, 4, 2, 1):
            lanes = (lanes + lanes[np.arange(64) ^ m]).astype(np.float32)
        if lanes[0] == seq:
            continue
        found = True
        inv_l = np.float32(1) / np.sqrt(np.float32(lanes[0] / np.float32(1000)) + np.float32(1e-5))
        got = ref.rmsnorm(x, w, 1e-5)
        assert np.array_equal(got[0], (x[0] * inv_l).astype(np.float32))
        break
    assert found
