"""nn.Linear of the privacy-filter model on this library's kernels.

Reference: src/core/nn/layers.ts:166-263 (Linear: y = x·W + bias + addend,
W stored [in, out], torch checkpoints transposed once at load; a quantized
checkpoint weight loads as quantW words [in, out] with f32 scales
[in / groupSize, out]), src/core/graph/compose.ts:45-53 (linear).

A quantized Linear is the grouped down product with one expert: quantW
[in, out], scales [in / g, out], bias [1, out], every row routed to expert
0 with gate 1.0 (exact), the addend as the residual (moe_down). A float
Linear is matmulGather with one expert (moe_matmul_gather) and takes no
addend.
"""
from dataclasses import dataclass
from typing import Optional

import numpy as np
import torch

from .errors import RunntimeError
from .quantw import QuantExpertWeight, QuantW, pack_expert_weights


def _route_ones(t: int, device) -> torch.Tensor:
    """[T, 2] route rows (expert 0, gate 1.0) for one-expert calls."""
    r = torch.empty((t, 2), dtype=torch.float32, device=device)
    r[:, 0] = 0.0
    r[:, 1] = 1.0
    return r


@dataclass
class Linear:
    """in_features → out_features. Exactly one of `quant` (QuantExpertWeight
    with E = 1, plus bits and group_size) or `weight` (float [in, out] with
    `bias` [1, out]) is set."""
    in_features: int
    out_features: int
    quant: Optional[QuantExpertWeight] = None
    bits: int = 8
    group_size: int = 0
    weight: Optional[torch.Tensor] = None
    bias: Optional[torch.Tensor] = None

    @staticmethod
    def from_torch_layout(w_out_in: np.ndarray, bias: Optional[np.ndarray], device) -> "Linear":
        """A float checkpoint weight [out, in] (transposed once, as the
        reference's transformStateDict does)."""
        out_f, in_f = w_out_in.shape
        w = torch.from_numpy(np.ascontiguousarray(np.asarray(w_out_in).T)).to(device)
        b = (torch.from_numpy(np.asarray(bias, np.float32).reshape(1, out_f)).to(device).to(w.dtype)
             if bias is not None else torch.zeros((1, out_f), dtype=w.dtype, device=device))
        return Linear(in_f, out_f, weight=w, bias=b)

    @staticmethod
    def from_quant(ints_out_in: np.ndarray, scales_out_groups: np.ndarray, bits: int,
                   bias: Optional[np.ndarray], device, name: str = "weight") -> "Linear":
        """A quantized checkpoint weight: signed ints [out, in] with f32
        scales [out, in / g] (the file's I8 / U8 + F16 `_scale`)."""
        out_f, in_f = ints_out_in.shape
        groups = scales_out_groups.shape[1]
        g = in_f // groups if groups else 0
        if (groups == 0 or in_f % groups or in_f % 4 or g % 4 or out_f % (32 // bits)):
            raise RunntimeError(
                "CHECKPOINT_MISMATCH",
                f"Linear: {name} is int{bits} in groups of {g}, which needs in features a "
                f"multiple of 4 and of the group size, out features a multiple of {32 // bits} "
                f"and a group size a multiple of 4, got [out, in] = [{out_f}, {in_f}]")
        words = pack_expert_weights(np.asarray(ints_out_in, np.int8).T.reshape(1, in_f, out_f),
                                    bits)
        sc = np.ascontiguousarray(np.asarray(scales_out_groups, np.float32).T)  # [in/g, out]
        b = (np.asarray(bias, np.float32).reshape(1, out_f) if bias is not None
             else np.zeros((1, out_f), np.float32))
        dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(device)
        q = QuantExpertWeight(QuantW(dev(words.view(np.int32)), (in_f, out_f)), dev(sc), dev(b))
        return Linear(in_f, out_f, quant=q, bits=bits, group_size=g)

    def forward(self, x: torch.Tensor, addend: Optional[torch.Tensor] = None) -> torch.Tensor:
        """y = x·W + bias (+ addend): [T, in] → [T, out]."""
        from .core import matmulGather, moeDown
        t = x.shape[0]
        if x.dim() != 2 or x.shape[1] != self.in_features:
            raise ValueError(f"Linear: x must be [T, {self.in_features}], got {list(x.shape)}")
        if self.quant is not None:
            route = _route_ones(t, x.device)
            return moeDown(x, route, self.quant, addend,
                           {"bits": self.bits, "groupSize": self.group_size})
        if addend is not None:
            raise ValueError("Linear: a float weight takes no addend here")
        idx = torch.zeros(t, dtype=torch.float32, device=x.device)
        return matmulGather(x, self.weight, idx, {"bias": self.bias})
