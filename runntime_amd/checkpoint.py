"""Loads the privacy-filter MoE block from its safetensors checkpoint.

The hosted model (`int8g640`, src/zoo/models.ts:71-73) stores each block's
MoE weights pre-packed: quantW words as U32 and f32 scales and biases, under
the module's own parameter names (src/zoo/privacy-filter/moeMlp.ts:34-75):

    block.{n}.mlp.norm.weight (or .scale)  RMSNorm weight [d]
    block.{n}.mlp.gate.weight / .bias      router Linear, torch layout [E, d] / [E]
    block.{n}.mlp.{glu,lin,out}Weight      U32 quantW words of [E·K, N]
    block.{n}.mlp.{glu,lin,out}Scales      f32 [E·K/groupSize, N]
    block.{n}.mlp.{glu,lin,out}Bias        f32 [E, N]

Reference: src/core/nn/loadStateDict.ts:180-215 (binding, shape checks; a
U32 file tensor under a quantW slot counts words), src/core/nn/layers.ts
:196-217 (a Linear's torch-layout weight is transposed once at load; a
quantized one arrives as I8 + F16 `_scale`, src/core/weights/
safetensors.ts:470-520), src/zoo/privacy-filter/stateDictHooks.ts:80-87
(exported files name the norm weight `scale`). The HF-layout float
checkpoint mapping (stateDictHooks.ts:41-78) feeds the float-weight path,
which this package does not have.
"""
from dataclasses import dataclass
from typing import Optional

import numpy as np
import torch

from .errors import RunntimeError
from .quantw import QuantExpertWeight, QuantW
from .safetensors import SafetensorsFile

RMS_EPS = 1e-5  # the block's norm epsilon (moeMlp.ts:23)


def _mismatch(msg: str) -> RunntimeError:
    return RunntimeError("CHECKPOINT_MISMATCH", msg)


@dataclass
class MoeBlock:
    """One privacy-filter MoE block's weights on a device, and its forward:
    EagerMoeMlp.forward for the quantized formats (moeMlp.ts:79-121)."""
    norm_w: torch.Tensor           # [d], the activation dtype
    router_w: torch.Tensor         # f32 [d, E]
    router_b: Optional[torch.Tensor]
    glu: QuantExpertWeight
    lin: QuantExpertWeight
    down: QuantExpertWeight
    E: int
    d: int
    I: int
    bits: int
    group_up: int
    group_down: int
    eps: float = RMS_EPS
    k: int = 4                     # the privacy filter routes to 4 experts

    @property
    def dtype(self) -> torch.dtype:
        return self.norm_w.dtype

    def forward(self, x: torch.Tensor, return_route: bool = False):
        from .core import moe_block
        return moe_block(x, self.norm_w, self.eps, self.router_w, self.router_b, self.glu,
                         self.lin, self.down, self.k, self.bits, self.group_up, self.group_down,
                         return_route=return_route)


def _dequant_rows(q: np.ndarray, scales: np.ndarray, g: int) -> np.ndarray:
    """[out, cols] ints × f32 scales [out, cols/g] → f32."""
    out, cols = q.shape
    return (q.reshape(out, cols // g, g).astype(np.float32) * scales[:, :, None]).reshape(out, cols)


def load_moe_block(path: str, layer: int = 0, device="cuda", experts: Optional[int] = None,
                   hidden: Optional[int] = None, eps: float = RMS_EPS, k: int = 4) -> MoeBlock:
    """Reads block `layer`'s MoE weights. `experts` and `hidden` check the
    file against a model's dims; left out, they come from the router."""
    f = SafetensorsFile(path)
    pre = f"block.{layer}.mlp."

    def name_of(n):
        return pre + n

    def need(n):
        if name_of(n) not in f.names:
            raise _mismatch(f"privacy-filter state dict: missing tensor '{name_of(n)}'")
        return name_of(n)

    # Router (a Linear): torch layout [E, d], float or int8 + F16 scales.
    gname = need("gate.weight")
    if gname in f.quant:
        qt = f.quant[gname]
        gate = _dequant_rows(qt.ints(), qt.scales(), qt.group_size)
    else:
        gate = f.array(gname).astype(np.float32)
    if gate.ndim != 2 or (experts is not None and gate.shape[0] != experts) or (
            hidden is not None and gate.shape[1] != hidden):
        want = [experts if experts is not None else "E", hidden if hidden is not None else "d"]
        raise _mismatch(f"Linear: {gname} has shape {list(gate.shape)}, expected torch layout "
                        f"[{want[0]}, {want[1]}]")
    E, d = gate.shape
    gb = name_of("gate.bias")
    router_b = f.array(gb).astype(np.float32) if gb in f.names else None
    if router_b is not None and router_b.size != E:
        raise _mismatch(f"loadStateDict: '{gb}' checkpoint shape {list(router_b.shape)} "
                        f"({router_b.size} elems) != model [{E}] ({E} elems)")

    # Norm weight (exported files call it `scale`); its dtype is the block's.
    nname = name_of("norm.weight") if name_of("norm.weight") in f.names else name_of("norm.scale")
    if nname not in f.names:
        raise _mismatch(f"privacy-filter state dict: missing tensor '{name_of('norm.weight')}'")
    norm = f.array(nname)
    if norm.size != d:
        raise _mismatch(f"loadStateDict: '{nname}' checkpoint shape {list(norm.shape)} "
                        f"({norm.size} elems) != model [{d}] ({d} elems)")
    norm_dtype = torch.float16 if norm.dtype == np.float16 else torch.float32

    def expert(stem, K):
        sname, wname, bname = need(f"{stem}Scales"), need(f"{stem}Weight"), name_of(f"{stem}Bias")
        sc = f.array(sname)
        if sc.ndim != 2 or sc.dtype != np.float32:
            raise _mismatch(f"loadStateDict: '{sname}' must be f32 [E·K/groupSize, N], got "
                            f"{sc.dtype} {list(sc.shape)}")
        rows, N = sc.shape
        if rows == 0 or (E * K) % rows:
            raise _mismatch(f"loadStateDict: '{sname}' has {rows} rows, which do not divide "
                            f"E·K = {E * K}")
        g = E * K // rows
        info = f.infos[wname]
        if info.dtype != "U32":
            raise _mismatch(f"loadStateDict: '{wname}' is {info.dtype}; the quantized MoE "
                            f"weights load as pre-packed U32 quantW words")
        words = f.array(wname).reshape(-1)
        bits = words.size * 32 // (E * K * N) if E * K * N else 0
        if bits not in (8, 4) or words.size * 32 != bits * E * K * N:
            raise _mismatch(f"loadStateDict: '{wname}' checkpoint shape {info.shape} "
                            f"({words.size} elems) != model [{E * K},{N}] "
                            f"({E * K * N // 4} words)")
        bias = f.array(bname).astype(np.float32) if bname in f.names else None
        if bias is not None and bias.size != E * N:
            raise _mismatch(f"loadStateDict: '{bname}' checkpoint shape {list(bias.shape)} "
                            f"({bias.size} elems) != model [{E},{N}] ({E * N} elems)")
        dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(device)
        w = QuantExpertWeight(QuantW(dev(words.view(np.int32)), (E * K, N)), dev(sc),
                              dev(bias.reshape(E, N)) if bias is not None else None)
        return w, N, bits, g

    glu, I, bits, g_up = expert("glu", d)
    lin, I2, bits2, g_up2 = expert("lin", d)
    down, d2, bits3, g_dn = expert("out", I)
    if I2 != I or bits2 != bits or g_up2 != g_up:
        raise _mismatch(f"privacy-filter state dict: {pre}linWeight does not match {pre}gluWeight "
                        f"(N {I2} vs {I}, int{bits2} vs int{bits}, groupSize {g_up2} vs {g_up})")
    if d2 != d or bits3 != bits:
        raise _mismatch(f"privacy-filter state dict: {pre}outWeight has N {d2} and int{bits3}; "
                        f"the block needs N {d} and int{bits}")
    return MoeBlock(
        norm_w=torch.from_numpy(norm.reshape(d).copy()).to(norm_dtype).to(device),
        router_w=torch.from_numpy(np.ascontiguousarray(gate.T)).to(device),
        router_b=torch.from_numpy(router_b).to(device) if router_b is not None else None,
        glu=glu, lin=lin, down=down, E=E, d=d, I=I, bits=bits, group_up=g_up, group_down=g_dn,
        eps=eps, k=k)


def save_moe_block(path: str, layer: int, norm_w: np.ndarray, gate_w: np.ndarray,
                   gate_b: Optional[np.ndarray], experts: dict, norm_name: str = "scale",
                   metadata: Optional[dict] = None) -> None:
    """Writes a block in the hosted layout (the loader's inverse, for tests
    and for exporting weights built elsewhere). experts: {"glu"|"lin"|"out":
    (words uint32, scales f32 [E·K/g, N], bias f32 [E, N] or None)};
    gate_w f32 [E, d] in torch layout."""
    from .safetensors import write
    pre = f"block.{layer}.mlp."
    t = {}
    nd = "F16" if norm_w.dtype == np.float16 else "F32"
    t[pre + f"norm.{norm_name}"] = (nd, [norm_w.size], norm_w)
    t[pre + "gate.weight"] = ("F32", list(gate_w.shape), gate_w.astype(np.float32))
    if gate_b is not None:
        t[pre + "gate.bias"] = ("F32", [gate_b.size], gate_b.astype(np.float32))
    for stem, (words, sc, bias) in experts.items():
        t[pre + f"{stem}Weight"] = ("U32", [words.size], words.astype(np.uint32))
        t[pre + f"{stem}Scales"] = ("F32", list(sc.shape), sc.astype(np.float32))
        if bias is not None:
            t[pre + f"{stem}Bias"] = ("F32", list(bias.shape), bias.astype(np.float32))
    write(path, t, metadata)
