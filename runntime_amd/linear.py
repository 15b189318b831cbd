"""nn.Linear of the privacy-filter model on this library's kernels.

Reference: src/core/nn/layers.ts:166-263 (Linear: y = x·W + bias + addend,
W stored [in, out], torch checkpoints transposed once at load; a quantized
checkpoint weight loads as ints with scales [in / groupSize, out] and its
kernel multiplies each int by its group's scale), src/core/graph/
compose.ts:45-53 (linear).

Both kinds run on moe_linear (linear.hip): the weight is kept as f32 [in,
out], a quantized one dequantized once at load (int · its group's scale,
one f32 product per weight). The projections of this model are small (a
few MB per block), and the texts are tens of rows, so the kernel spreads
the work over columns and K slices rather than streaming int8.
"""
from dataclasses import dataclass
from typing import Optional

import numpy as np
import torch

from .errors import RunntimeError


@dataclass
class Linear:
    """in_features → out_features: `weight` f32 [in, out], `bias` f32
    [out] or None. `bits` / `group_size` record a quantized checkpoint's
    format (0 for a float one)."""
    in_features: int
    out_features: int
    weight: torch.Tensor
    bias: Optional[torch.Tensor] = None
    bits: int = 0
    group_size: int = 0

    def __post_init__(self):
        w, b = self.weight, self.bias
        if (w.dtype != torch.float32 or tuple(w.shape) != (self.in_features, self.out_features)
                or not w.is_contiguous()):
            raise ValueError(f"Linear: weight must be contiguous f32 [{self.in_features}, "
                             f"{self.out_features}], got {w.dtype} {list(w.shape)}")
        if b is not None and (b.dtype != torch.float32 or tuple(b.shape) != (self.out_features,)
                              or not b.is_contiguous()):
            raise ValueError(f"Linear: bias must be contiguous f32 [{self.out_features}], got "
                             f"{b.dtype} {list(b.shape)}")

    @staticmethod
    def from_torch_layout(w_out_in: np.ndarray, bias: Optional[np.ndarray], device) -> "Linear":
        """A float checkpoint weight [out, in] (transposed once, as the
        reference's transformStateDict does)."""
        out_f, in_f = w_out_in.shape
        w = torch.from_numpy(np.ascontiguousarray(np.asarray(w_out_in, np.float32).T)).to(device)
        b = (torch.from_numpy(np.asarray(bias, np.float32).reshape(out_f)).to(device)
             if bias is not None else None)
        return Linear(in_f, out_f, w, b)

    @staticmethod
    def from_quant(ints_out_in: np.ndarray, scales_out_groups: np.ndarray, bits: int,
                   bias: Optional[np.ndarray], device, name: str = "weight") -> "Linear":
        """A quantized checkpoint weight: signed ints [out, in] with f32
        scales [out, in / g] (the file's I8 / U8 + F16 `_scale`)."""
        out_f, in_f = ints_out_in.shape
        groups = scales_out_groups.shape[1]
        g = in_f // groups if groups else 0
        if groups == 0 or in_f % groups:
            raise RunntimeError(
                "CHECKPOINT_MISMATCH",
                f"Linear: {name} is int{bits} with {groups} scale groups, which must divide its "
                f"{in_f} in features")
        sc = np.asarray(scales_out_groups, np.float32)
        w = (np.asarray(ints_out_in, np.float32).reshape(out_f, groups, g) * sc[:, :, None])
        lin = Linear.from_torch_layout(w.reshape(out_f, in_f), bias, device)
        lin.bits, lin.group_size = bits, g
        return lin

    def forward(self, x: torch.Tensor, addend: Optional[torch.Tensor] = None) -> torch.Tensor:
        """y = x·W + bias (+ addend): f32 [T, in] → f32 [T, out]."""
        from . import _lib
        from .core import _ctx, _device_of
        if x.dim() != 2 or x.shape[1] != self.in_features or x.dtype != torch.float32:
            raise ValueError(f"Linear: x must be f32 [T, {self.in_features}], got "
                             f"{x.dtype} {list(x.shape)}")
        t = x.shape[0]
        if addend is not None and (addend.dtype != torch.float32
                                   or tuple(addend.shape) != (t, self.out_features)):
            raise ValueError(f"Linear: addend must be f32 [{t}, {self.out_features}]")
        x = x.contiguous()
        if addend is not None:
            addend = addend.contiguous()  # the kernel reads it as dense rows
        dev = _device_of(x, self.weight, *(a for a in (self.bias, addend) if a is not None))
        out = torch.empty((t, self.out_features), dtype=torch.float32, device=dev)
        lib = _lib.load()
        _lib.check(lib.moe_linear(_ctx(dev), x.data_ptr(), self.weight.data_ptr(),
                                  self.bias.data_ptr() if self.bias is not None else None,
                                  addend.data_ptr() if addend is not None else None, t,
                                  self.in_features, self.out_features, out.data_ptr()))
        return out
