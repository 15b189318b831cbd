"""Shared test helpers: the reference tests' input generators and the
tolerance checks."""

import numpy as np

from oracle import ref

# Output bar of the layer: |got − want| ≤ ATOL + RTOL·|want| against the
# oracle's f64 result.
ATOL = 2e-3
RTOL = 1e-2


def assert_close(got, want, atol=ATOL, rtol=RTOL, what=""):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    assert got.shape == want.shape, (got.shape, want.shape)
    assert not np.isnan(got).any(), f"{what}: NaN in result"
    err = np.abs(got - want)
    bound = atol + rtol * np.abs(want)
    bad = err > bound
    if bad.any():
        i = np.unravel_index(np.argmax(err - bound), err.shape)
        raise AssertionError(
            f"{what}: {bad.sum()} of {bad.size} outside atol {atol} rtol {rtol}; worst at {i}: "
            f"got {got[i]!r} want {want[i]!r} (max abs err {err.max():.3g})")


def route_for(tokens, experts, k, gates=(0.4, 0.3, 0.2, 0.1)):
    """moeQuantW.gpu.test.ts:31-40 generalised to k slots: ids (t·3 + s·5) mod E,
    gates rotated per token (for k ≠ 4, k evenly spaced weights summing to 1)."""
    if k != 4:
        gates = [(k - i) / (k * (k + 1) / 2) for i in range(k)]
    route = np.zeros((tokens, 2 * k), np.float32)
    for t in range(tokens):
        for s in range(k):
            route[t, s] = (t * 3 + s * 5) % experts
            route[t, k + s] = gates[(s + t) % k]
    return route


def random_quant_weight(experts, k, n, bits, group_size, seed):
    """randomQuantWeight (test/core/kernels/matmul/quantW.ts:55-92): ints over
    the full signed range of `bits` from the LCG, positive scales
    (|v| + 0.1)/half, row r takes scale row r / groupSize. Returns logical
    q [E, K, N] int8 and scales f32 [E·K/g, N]."""
    rows = experts * k
    half = 2 ** (bits - 1)
    v = ref.lcg_f32(rows * n, seed).astype(np.float64)
    q = np.minimum(half - 1, np.floor(v * half)).astype(np.int8).reshape(experts, k, n)
    s = ref.lcg_f32(rows // group_size * n, seed + 1).astype(np.float64)
    scales = ((np.abs(s) + 0.1) / half).astype(np.float32).reshape(rows // group_size, n)
    return q, scales


def dense_project(x, q, scales, bias, e, group_size):
    """x · (q[e]·scale) + bias[e] in f64 via a dense matmul — an independent
    path from the oracle's packed-word reads."""
    E, K, N = q.shape
    sc = np.repeat(scales.reshape(E, K // group_size, N)[e], group_size, axis=0)
    w = q[e].astype(np.float64) * sc.astype(np.float64)
    out = np.asarray(x, np.float64) @ w
    if bias is not None:
        out = out + bias[e].astype(np.float64)
    return out


def swiglu_np(g, l):
    g = np.minimum(g, 7.0)
    l = np.clip(l, -7.0, 7.0)
    return g / (1.0 + np.exp(-1.702 * g)) * (l + 1.0)
