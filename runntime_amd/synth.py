"""Seeded synthetic inputs of the five benchmark configurations.

One generator for every consumer (GPU tests, the bench, the oracle checks):
inputs are drawn on the CPU with a seeded torch.Generator, so the same seed
gives the same bytes everywhere, then moved to the device.

  x        ~ N(0, 1); f32 (configs 1-2) or rounded to f16 (configs 3-5)
  router W ~ N(0, 0.02²) f32 [d, E]; bias 0, or the Zipf bias (config 5)
  q        int8 uniform in [-127, 127]; quantW-packed
  scales   ~ U(0.5e-3, 2e-3) f32, one per output channel (groupSize = K)
  expert biases 0, residual 0 (the reference's ops take the tensors)
"""
from dataclasses import dataclass, field

import numpy as np
import torch

from .quantw import QuantExpertWeight, QuantW, pack_expert_weights_torch


@dataclass(frozen=True)
class MoeConfig:
    name: str
    T: int
    d: int
    E: int
    k: int
    I: int
    x_dtype: str  # "f32" | "f16"
    zipf: float = 0.0  # Zipf exponent of the router bias, 0 = none
    hot_share: float = 0.20  # share of tokens routed to the hottest expert under zipf
    tokens: int = 0  # decode configs: independent single-token calls timed
    empty: int = 0  # under zipf: the coldest `empty` experts get a bias no token overcomes

    @property
    def assignments(self) -> int:
        return self.T * self.k


CONFIGS = {
    1: MoeConfig("c1_T64_d512_E8_k2_I1024_f32", 64, 512, 8, 2, 1024, "f32"),
    2: MoeConfig("c2_decode_T1_d640_E128_k4_I640_f32", 1, 640, 128, 4, 640, "f32", tokens=1000),
    3: MoeConfig("c3_decode_T8_d2048_E64_k8_I1408_f16", 8, 2048, 64, 8, 1408, "f16"),
    4: MoeConfig("c4_prefill_T4096_d2048_E32_k4_I5632_f16", 4096, 2048, 32, 4, 5632, "f16"),
    5: MoeConfig("c5_skewed_T4096_d2048_E128_k8_I1408_f16", 4096, 2048, 128, 8, 1408, "f16",
                 zipf=1.2, empty=6),
}


@dataclass
class MoeInputs:
    cfg: MoeConfig
    x: torch.Tensor
    router_w: torch.Tensor
    router_b: torch.Tensor
    glu: QuantExpertWeight
    lin: QuantExpertWeight
    down: QuantExpertWeight
    residual: torch.Tensor
    q: dict = field(default_factory=dict)  # logical int8 q [E, K, N] per projection (CPU), if kept


def _gen(seed: int) -> torch.Generator:
    g = torch.Generator(device="cpu")
    g.manual_seed(seed)
    return g


def _expert_weight(E, K, N, g, device, keep_q, bias_rand=False):
    q = torch.randint(-127, 128, (E, K, N), generator=g, dtype=torch.int8)
    scales = torch.rand((E, N), generator=g, dtype=torch.float32) * 1.5e-3 + 0.5e-3
    bias = (torch.randn((E, N), generator=g, dtype=torch.float32) * 0.1 if bias_rand
            else torch.zeros((E, N), dtype=torch.float32))
    words = pack_expert_weights_torch(q.to(device))
    w = QuantExpertWeight(QuantW(words, (E * K, N)), scales.to(device), bias.to(device))
    return w, (q if keep_q else None)


def zipf_bias(cfg: MoeConfig, x: torch.Tensor, router_w: torch.Tensor, seed: int) -> torch.Tensor:
    """b_e = c·rank(e)^(−s) over a seeded permutation of the experts, with c
    chosen (bisection, f64 on the CPU) so that about `hot_share` of the
    tokens route to the hottest expert; the `empty` coldest experts (the
    tail of the Zipf ranking) get −1e4 on top, so no token reaches them.

    The share is of tokens, not of the T·k assignments: a token picks an
    expert at most once, so one expert can hold at most 1/k of the
    assignments (12.5% at k = 8), and a search for 20% of them drives c to
    its cap, where every token picks the same k experts."""
    g = _gen(seed + 7)
    perm = torch.randperm(cfg.E, generator=g)
    rank = torch.empty(cfg.E, dtype=torch.float64)
    rank[perm] = torch.arange(1, cfg.E + 1, dtype=torch.float64)
    shape = rank.pow(-cfg.zipf)
    logits = x.double().cpu() @ router_w.double().cpu()
    # The Zipf tail's coldest experts: pushed far below every logit (the
    # logits are O(1)), so they receive no tokens.
    tail = torch.zeros(cfg.E, dtype=torch.float64)
    if cfg.empty:
        tail[rank > cfg.E - cfg.empty] = -1.0e4
    logits = logits + tail

    def hottest(c):
        ids = torch.topk(logits + c * shape, cfg.k, dim=1).indices
        return torch.bincount(ids.reshape(-1), minlength=cfg.E).max().item() / logits.shape[0]

    lo, hi = 0.0, 1.0
    while hottest(hi) < cfg.hot_share and hi < 1e4:
        hi *= 2
    for _ in range(40):
        mid = 0.5 * (lo + hi)
        if hottest(mid) < cfg.hot_share:
            lo = mid
        else:
            hi = mid
    c = float(np.float32(hi))
    return (c * shape + tail).float()


def make_inputs(cfg: MoeConfig, seed: int = 0, device="cuda", keep_q: bool = False,
                bias_rand: bool = False, T: int = None) -> MoeInputs:
    """Draws one layer's inputs. `T` overrides the token count (the decode
    bench draws many independent tokens at once)."""
    T = cfg.T if T is None else T
    g = _gen(seed)
    x = torch.randn((T, cfg.d), generator=g, dtype=torch.float32)
    if cfg.x_dtype == "f16":
        x = x.half()
    router_w = torch.randn((cfg.d, cfg.E), generator=g, dtype=torch.float32) * 0.02
    glu, qg = _expert_weight(cfg.E, cfg.d, cfg.I, g, device, keep_q, bias_rand)
    lin, ql = _expert_weight(cfg.E, cfg.d, cfg.I, g, device, keep_q, bias_rand)
    down, qd = _expert_weight(cfg.E, cfg.I, cfg.d, g, device, keep_q, bias_rand)
    if cfg.zipf:
        router_b = zipf_bias(cfg, x.float(), router_w, seed)
    else:
        router_b = torch.zeros(cfg.E, dtype=torch.float32)
    residual = torch.zeros((T, cfg.d), dtype=torch.float32)
    inp = MoeInputs(cfg, x.to(device), router_w.to(device), router_b.to(device), glu, lin, down,
                    residual.to(device))
    if keep_q:
        inp.q = {"glu": qg, "lin": ql, "down": qd}
    return inp


@dataclass
class WeightCopies:
    """C independent copies of one layer's weights, stacked on a leading
    call dim for moe_layer_batched."""
    cfg: MoeConfig
    router_w: torch.Tensor  # [C, d, E]
    router_b: torch.Tensor  # [C, E]
    glu: QuantExpertWeight  # words [C, n], scales [C, E, N], bias [C, E, N]
    lin: QuantExpertWeight
    down: QuantExpertWeight


def make_weight_copies(cfg: MoeConfig, copies: int, seed: int = 0,
                       device="cuda") -> WeightCopies:
    """`copies` seeded weight sets drawn with a generator on `device` (the
    bench's multi-GB sets are drawn on the GPU; same distributions as
    make_inputs)."""
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    C, E, d, I = copies, cfg.E, cfg.d, cfg.I

    def ew(K, N):
        # Drawn and packed 16 copies at a time into the final tensor, so the
        # int8 draw and its packed copy never both exist for all copies.
        words = torch.empty((C, E * K * N // 4), dtype=torch.int32, device=device)
        for c0 in range(0, C, 16):
            c1 = min(C, c0 + 16)
            q = torch.randint(-127, 128, ((c1 - c0) * E, K, N), generator=g, dtype=torch.int8,
                              device=device)
            words[c0:c1] = pack_expert_weights_torch(q).view(c1 - c0, -1)
            del q
        sc = torch.rand((C, E, N), generator=g, dtype=torch.float32, device=device) * 1.5e-3 + 0.5e-3
        return QuantExpertWeight(QuantW(words, (E * K, N)), sc,
                                 torch.zeros((C, E, N), dtype=torch.float32, device=device))

    rw = torch.randn((C, d, E), generator=g, dtype=torch.float32, device=device) * 0.02
    rb = torch.zeros((C, E), dtype=torch.float32, device=device)
    return WeightCopies(cfg, rw, rb, ew(d, I), ew(d, I), ew(I, d))
