"""Pins the float-path oracle (matmul_gather_f64, moe_block_float_f64) with
closed forms: identity expert weights select the row block and bias of the
indexed expert; zero weights leave the block as its residual; the SwiGLU of
a constant pre-activation is the textbook value."""
import numpy as np

from oracle import ref


def test_identity_weights_pick_the_expert_block():
    E, K = 3, 4
    w = np.zeros((E * K, K))
    for e in range(E):
        w[e * K:(e + 1) * K] = np.eye(K) * (e + 1)
    bias = np.arange(E * K, dtype=np.float64).reshape(E, K)
    a = np.arange(8, dtype=np.float64).reshape(2, K)
    out = ref.matmul_gather_f64(a, w, bias, [2, 0], K)
    np.testing.assert_array_equal(out[0], 3 * a[0] + bias[2])
    np.testing.assert_array_equal(out[1], 1 * a[1] + bias[0])


def test_invalid_ids_give_zero_rows():
    w = np.ones((8, 4))
    out = ref.matmul_gather_f64(np.ones((4, 4)), w, np.ones((2, 4)), [-1, 2, 0.5, 1], 4)
    assert not out[[0, 1, 2]].any()
    np.testing.assert_array_equal(out[3], np.full(4, 5.0))


def test_block_with_zero_weights_is_its_residual():
    T, d, I, E, k = 3, 8, 4, 4, 2
    x = np.random.default_rng(0).standard_normal((T, d))
    route = np.array([[0, 1, 0.5, 0.5]] * T, np.float32)
    z = lambda r, c: (np.zeros((r, c)), None)
    out = ref.moe_block_float_f64(x, x, route, z(E * d, I), z(E * d, I), z(E * I, d), k)
    np.testing.assert_array_equal(out, x)


def test_block_constant_preactivation():
    """glu bias 1, lin bias 0, zero weights: act = swiglu(1, 0) =
    1/(1+e^-1.702) for every column; down = ones → each output column gets
    I·act per slot, times the gates (summing to 1)."""
    T, d, I, E, k = 2, 4, 4, 2, 2
    x = np.zeros((T, d))
    route = np.array([[0, 1, 0.75, 0.25]] * T, np.float32)
    glu = (np.zeros((E * d, I)), np.ones((E, I)))
    lin = (np.zeros((E * d, I)), np.zeros((E, I)))
    down = (np.ones((E * I, d)), None)
    out = ref.moe_block_float_f64(x, x, route, glu, lin, down, k)
    act = 1.0 / (1.0 + np.exp(-1.702))
    np.testing.assert_allclose(out, np.full((T, d), I * act), rtol=1e-12)
