"""Parity of the float-weight path through the C ABI: matmulGather on the
reference test's cases (matmulGather.gpu.test.ts:56-103) at its tolerance
(f32: atol 1e-6·K, rtol 1e-5; f16: atol 2e-3, rtol 2e-3) against the f64
formula, and the float block (moeMlp.ts:85-100) at the layer bar with
expert ids bit-exact."""
import numpy as np
import pytest
import torch

import runntime_amd as rt
from oracle import ref
from tests.helpers import assert_close

pytestmark = pytest.mark.gpu

DEV = "cuda"
TD = {"f32": torch.float32, "f16": torch.float16}


def say(msg):
    print(msg, flush=True)


def rnd(v, dtype):
    return v.astype(np.float16).astype(np.float32) if dtype == "f16" else v


CASES = [
    ("one row, one expert, one quad", 1, 4, 1, [0]),
    ("odd K", 7, 8, 3, [2, 0, 1]),
    ("the same expert on every row", 16, 12, 4, [3, 3, 3, 3, 3]),
    ("the last expert", 9, 4, 5, [4]),
    ("rows past a workgroup of units", 33, 68, 4, [(i * 7) % 4 for i in range(70)]),
    ("many rows", 4, 8, 3, [i % 3 for i in range(70005)]),
    ("privacy-filter shape", 640, 640, 128, [5, 17, 99, 127, 5, 0]),
]


@pytest.mark.parametrize("dtype", ["f32", "f16"])
@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_matmul_gather_reference_cases(case, dtype):
    name, K, N, E, experts = case
    say(f"matmulGather {dtype} {name}")
    M = len(experts)
    a = rnd(ref.lcg_f32(M * K, 1).reshape(M, K), dtype)
    w = rnd(ref.lcg_f32(E * K * N, 2).reshape(E * K, N), dtype)
    bias = rnd(ref.lcg_f32(E * N, 3).reshape(E, N), dtype)
    idx = np.array(experts, np.float32)
    t = lambda v: torch.from_numpy(np.ascontiguousarray(v)).to(TD[dtype]).to(DEV)
    got = rt.matmulGather(t(a), t(w), torch.from_numpy(idx).to(DEV), {"bias": t(bias)})
    got = got.float().cpu().numpy()
    want = ref.matmul_gather_f64(a, w, bias, idx, K)
    atol, rtol = (2e-3, 2e-3) if dtype == "f16" else (1e-6 * K, 1e-5)
    np.testing.assert_allclose(got, want, atol=atol, rtol=rtol)


def test_matmul_gather_f16_rows_past_2p23_units():
    """matmulGather.gpu.test.ts:105-125: K 1, every weight 1, bias 0, so
    out[i, c] = a[i] exactly, across more than 2^23 column units."""
    m, n = 2100, 16380
    say("matmulGather f16 rows past 2^23 units")
    a = ((np.arange(m) % 7) + 1).astype(np.float16).reshape(m, 1)
    got = rt.matmulGather(torch.from_numpy(a).to(DEV), torch.ones((1, n), dtype=torch.float16, device=DEV),
                          torch.zeros(m, device=DEV), {"bias": torch.zeros((1, n), dtype=torch.float16, device=DEV)})
    assert torch.equal(got, torch.from_numpy(a).to(DEV).expand(m, n))


def test_matmul_gather_invalid_ids_are_zero():
    K, N, E = 8, 8, 2
    say("matmulGather invalid ids")
    a = ref.lcg_f32(4 * K, 1).reshape(4, K)
    w = ref.lcg_f32(E * K * N, 2).reshape(E * K, N)
    bias = ref.lcg_f32(E * N, 3).reshape(E, N)
    idx = np.array([1, -1, 2, 0.5], np.float32)
    got = rt.matmulGather(torch.from_numpy(a).to(DEV), torch.from_numpy(w).to(DEV),
                          torch.from_numpy(idx).to(DEV), {"bias": torch.from_numpy(bias).to(DEV)})
    got = got.cpu().numpy()
    assert not got[1:].any()
    np.testing.assert_allclose(got, ref.matmul_gather_f64(a, w, bias, idx, K), atol=1e-5, rtol=1e-5)


@pytest.mark.parametrize("dtype", ["f32", "f16"])
@pytest.mark.parametrize("T,d,I,E,k", [(1, 640, 640, 128, 4), (5, 640, 640, 128, 4),
                                       (40, 256, 512, 8, 2), (3, 64, 96, 16, 4)])
def test_moe_block_float_matches_oracle(T, d, I, E, k, dtype):
    say(f"moe_block_float {dtype} T={T} d={d} I={I} E={E} k={k}")
    rng = np.random.default_rng(T + d + E)
    x = rnd(rng.standard_normal((T, d)).astype(np.float32), dtype)
    norm = rnd((1 + 0.1 * rng.standard_normal(d)).astype(np.float32), dtype)
    rw = (0.02 * rng.standard_normal((d, E))).astype(np.float32)
    rb = (0.1 * rng.standard_normal(E)).astype(np.float32)
    sd = 1.0 / np.sqrt(d)
    glu = (rnd((sd * rng.standard_normal((E * d, I))).astype(np.float32), dtype),
           rnd((0.1 * rng.standard_normal((E, I))).astype(np.float32), dtype))
    lin = (rnd((sd * rng.standard_normal((E * d, I))).astype(np.float32), dtype),
           rnd((0.1 * rng.standard_normal((E, I))).astype(np.float32), dtype))
    down = (rnd((rng.standard_normal((E * I, d)) / np.sqrt(I)).astype(np.float32), dtype),
            rnd((0.1 * rng.standard_normal((E, d))).astype(np.float32), dtype))
    t = lambda v: torch.from_numpy(np.ascontiguousarray(v)).to(TD[dtype]).to(DEV)
    out, route = rt.moe_block_float(t(x), t(norm), 1e-5, torch.from_numpy(rw).to(DEV),
                                    torch.from_numpy(rb).to(DEV), t(glu[0]), t(glu[1]), t(lin[0]),
                                    t(lin[1]), t(down[0]), t(down[1]), k=k, return_route=True)
    torch.cuda.synchronize()
    npd = np.float16 if dtype == "f16" else np.float32
    xn = ref.rmsnorm(x, norm, 1e-5, dtype=npd).astype(np.float32)
    want_route = ref.topk(ref.router_logits(xn, rw, rb), k)
    got_route = route.cpu().numpy()
    assert np.array_equal(got_route[:, :k], want_route[:, :k]), "expert ids differ"
    want = ref.moe_block_float_f64(x, xn, want_route, glu, lin, down, k)
    assert_close(out.cpu().numpy(), want, what=f"float block {dtype}")
