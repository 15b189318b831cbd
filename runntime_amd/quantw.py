"""The quantW weight format: packing and the weight value the ops take.

Restates src/core/weights/quantPack.ts:12-28 (packQuantW) and the layout
contract of src/core/kernels/quantCommon.ts:8-15: the logical [E·K, N]
weight is stored as 16-value tiles, one per (expert, 4-column unit, 4-row
chunk); inside a tile values are column-major at `bits` per value, lowest
bits first; tiles are k4-major per (expert, unit), so the tile (e, unit, k4)
starts at word ((e·N/4 + unit)·K/4 + k4)·bits/2.

For int8 the format is a pure byte permutation of q[e, k, n]:
byte order [e][unit][k4][c][r] ↔ q[e, 4·k4 + r, 4·unit + c].
"""
from dataclasses import dataclass

import numpy as np
import torch


def pack_quant_w(ints_nk: np.ndarray, k: int, n: int, bits: int) -> np.ndarray:
    """packQuantW (quantPack.ts:12-28): one expert's output-first [n, k]
    signed ints → uint32 words of the logical [k, n] weight."""
    q = np.asarray(ints_nk, dtype=np.int8).reshape(n, k).T  # logical [k, n]
    return pack_expert_weights(q.reshape(1, k, n), bits)


def pack_expert_weights(q_ekn, bits: int) -> np.ndarray:
    """Logical q [E, K, N] (signed, within `bits`) → quantW uint32 words,
    experts concatenated expert-major (the layout the test suite's packer
    writes, test/core/kernels/matmul/quantW.ts:24-43)."""
    if isinstance(q_ekn, torch.Tensor):
        q_ekn = q_ekn.cpu().numpy()
    q = np.asarray(q_ekn, dtype=np.int8)
    E, K, N = q.shape
    if K % 4 or N % 4:
        raise ValueError(f"packQuantW: K {K} and N {N} must be multiples of 4")
    if bits not in (8, 4):
        raise ValueError(f"packQuantW: bits must be 8 or 4, got {bits}")
    # [e][k4][r][u][c] → [e][u][k4][c][r]
    t = q.reshape(E, K // 4, 4, N // 4, 4).transpose(0, 3, 1, 4, 2)
    t = np.ascontiguousarray(t).reshape(-1)
    if bits == 8:
        return t.view(np.uint8).view(np.uint32).copy()
    nib = (t.view(np.uint8) & 0x0F).astype(np.uint8)
    byte = nib[0::2] | (nib[1::2] << 4)
    return byte.view(np.uint32).copy()


def pack_expert_weights_torch(q_ekn: torch.Tensor) -> torch.Tensor:
    """int8 packing on any torch device (a byte permutation), for weights
    too large to round-trip through host memory. Returns int32 words."""
    E, K, N = q_ekn.shape
    t = q_ekn.reshape(E, K // 4, 4, N // 4, 4).permute(0, 3, 1, 4, 2).contiguous()
    return t.view(-1).view(torch.int32)


@dataclass
class QuantW:
    """A quantW weight value: `words` (int32 tensor of the uint32 words) and
    its logical `dims` [E·K, N] (src/core/graph/value.ts:15-17 — the
    reference counts a quantW value's elems in words)."""

    words: torch.Tensor
    dims: tuple

    @property
    def elems(self) -> int:
        return self.words.numel()


@dataclass
class QuantExpertWeight:
    """One routed layer's weights for all E experts: quantW `w` [E·K, N],
    f32 `scales` [E·K/groupSize, N] and f32 `bias` [E, N]
    (src/core/graph/ops/matmul.ts:212-218)."""

    w: QuantW
    scales: torch.Tensor
    bias: torch.Tensor
