"""The fused prefill layer (both products on the grouped GEMM; with f16 x act
goes between them as int8 limbs and down runs on the int8 matrix cores)
against the CPU oracle on every token, at shapes that exercise its tiling:
partial 64-row blocks, a last N-tile narrower than 512 columns, experts with
no rows, a hot expert, K with an odd number of step pairs, and the f16 hi +
lo pairs form that f32 x and I not a multiple of 64 take.

Bar: expert ids bit-exact, outputs within 2e-3 + 1e-2·|want| of the oracle
(the north star's layer bar)."""
import numpy as np
import pytest
import torch

import runntime_amd as rt
from oracle import ref
from runntime_amd.synth import MoeConfig, make_inputs
from tests.helpers import assert_close

pytestmark = pytest.mark.gpu

SHAPES = [
    # name, T, d, E, k, I, zipf
    MoeConfig("p_small", 512, 1024, 8, 2, 1024, "f16"),
    MoeConfig("p_ragged", 300, 640, 6, 4, 384, "f16"),          # d = 640: N-tile of 128 columns
    MoeConfig("p_oddpairs", 384, 640, 5, 2, 448, "f16"),        # 7 step pairs
    MoeConfig("p_skew", 512, 640, 16, 2, 384, "f16", zipf=1.2, hot_share=0.5, empty=2),
    # the layer's other prefill forms: f32 x (act as f16 hi + lo pairs, down
    # on the f16 matrix cores), and f16 x with I not a multiple of 64 (the
    # same pairs form: int8 limbs need whole step pairs)
    MoeConfig("p_f32x", 512, 1024, 8, 2, 1024, "f32"),
    MoeConfig("p_i1056", 512, 1024, 8, 2, 1056, "f16"),
]


def _oracle(inp, cfg):
    x = inp.x.float().cpu().numpy()
    logits = ref.router_logits(x, inp.router_w.cpu().numpy(), inp.router_b.cpu().numpy())
    route = ref.topk(logits, cfg.k)
    pk = {n: ref.pack_ekn(inp.q[n].numpy(), 8) for n in ("glu", "lin", "down")}
    w = {n: (pk[n], getattr(inp, n).scales.cpu().numpy(), getattr(inp, n).bias.cpu().numpy())
         for n in ("glu", "lin", "down")}
    act = ref.moe_up(x, route, w["glu"], w["lin"], 8, cfg.d, cfg.E)
    out = ref.moe_down(act, route, w["down"], inp.residual.cpu().numpy(), 8, cfg.I, cfg.E)
    return route, out


@pytest.mark.parametrize("cfg", SHAPES, ids=[c.name for c in SHAPES])
def test_prefill_layer_int8_limbs(cfg):
    print(f"prefill layer {cfg}", flush=True)
    inp = make_inputs(cfg, seed=11, keep_q=True, bias_rand=True)
    g = torch.Generator().manual_seed(5)
    inp.residual.copy_(torch.randn(tuple(inp.residual.shape), generator=g))
    out, route = rt.moe_layer(inp.x, inp.router_w, inp.router_b, inp.glu, inp.lin, inp.down,
                              inp.residual, cfg.k, return_route=True)
    torch.cuda.synchronize()
    got_route, got = route.cpu().numpy(), out.cpu().numpy()
    want_route, want = _oracle(inp, cfg)
    k = cfg.k
    assert np.array_equal(got_route[:, :k], want_route[:, :k]), "expert ids differ"
    counts = np.bincount(got_route[:, :k].astype(np.int64).ravel(), minlength=cfg.E)
    print(f"  rows per expert {counts.tolist()}", flush=True)
    if cfg.zipf:
        assert (counts == 0).any(), "the skewed shape should leave an expert without rows"
    assert_close(got, want, what=f"{cfg.name} output")
