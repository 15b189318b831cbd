"""The privacy-filter network around the MoE block: YaRN rope tables, the
attention block, the full block, the model forward, and the host-side
decoding (log-softmax, constrained Viterbi, token spans).

Reference (src/zoo/privacy-filter/):
  rope.ts:24-98        computeRopeTables (YaRN: concentration, ramp between
                       the NTK bounds) and ropeConstants (theta 150000,
                       scaling 32, ntk α 1 β 32, context 4096; the tables
                       pair-duplicated and scaled by 64^(−1/4) for q and k)
  attnBlock.ts:17-57   x + out(sdpa(rope(qkv(norm(x))))): qkv row = q(14×64)
                       ‖ k(2×64) ‖ v(2×64), window ±128, f32 sinks
  model.ts:16-76       blocks of attn then MoE, final RMSNorm, unembed
  config.ts:1-86       the 33 BIOES class names and the label info
  viterbi.ts:1-148     log-softmax rows and the constrained Viterbi decoder
  spans.ts:18-70       labels → token spans
Every device op runs on this library's kernels (rmsNorm, Linear over the
grouped down product or matmulGather, rope, sdpa, moe_block); the
embedding table stays on the host as the reference keeps it on the CPU.
"""
import math
from dataclasses import dataclass
from typing import List, Optional

import numpy as np
import torch

from .checkpoint import MoeBlock
from .linear import Linear

HIDDEN = 640
QKV_WIDTH = 1152
ATTN_OUT = 896
Q_HEADS = 14
KV_HEADS = 2
HEAD = 64
WINDOW = 128
K_OFF = Q_HEADS * HEAD       # 896
V_OFF = K_OFF + KV_HEADS * HEAD  # 1024
RMS_EPS = 1e-5
QK_SCALE = 0.3535533905932738  # 64^(-1/4), on q and k


def compute_rope_tables(positions, head_dim, theta, scaling_factor, ntk_alpha, ntk_beta,
                        initial_context_length):
    """YaRN tables (rope.ts:24-63): f32 cos, sin [positions, head_dim / 2]."""
    half = head_dim // 2
    freq = theta ** (2.0 * np.arange(half) / head_dim)
    concentration = 1.0
    if scaling_factor > 1.0:
        concentration = 0.1 * math.log(scaling_factor) + 1.0
        low = half * math.log(initial_context_length / (ntk_beta * 2 * math.pi)) / math.log(theta)
        high = half * math.log(initial_context_length / (ntk_alpha * 2 * math.pi)) / math.log(theta)
        ramp = np.clip((np.arange(half) - low) / (high - low), 0.0, 1.0)
        mask = 1.0 - ramp
        inv = (1.0 / (scaling_factor * freq)) * (1.0 - mask) + (1.0 / freq) * mask
    else:
        inv = 1.0 / freq
    ang = np.arange(positions, dtype=np.float64)[:, None] * inv[None, :]
    return ((np.cos(ang) * concentration).astype(np.float32),
            (np.sin(ang) * concentration).astype(np.float32))


def rope_constants(tokens):
    """ropeConstants (rope.ts:71-94): pair-duplicated [T, 64] tables with
    QK_SCALE folded in (the f32 table times QK_SCALE, rounded to f32)."""
    cos, sin = compute_rope_tables(tokens, HEAD, 150000.0, 32.0, 1.0, 32.0, 4096)
    cos_e = np.repeat(cos.astype(np.float64) * QK_SCALE, 2, axis=1).astype(np.float32)
    sin_e = np.repeat(sin.astype(np.float64) * QK_SCALE, 2, axis=1).astype(np.float32)
    return cos_e, sin_e


@dataclass
class AttnBlock:
    """EagerAttnBlock (attnBlock.ts:28-57)."""
    norm_w: torch.Tensor   # [640]
    qkv: Linear            # 640 → 1152
    out: Linear            # 896 → 640
    sinks: torch.Tensor    # f32 [14]

    def forward(self, x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
        from . import _lib
        from .core import _ctx, _xdtype, rmsNorm
        t = x.shape[0]
        # moe_attention reads cos/sin rows 0..T-1 of 64 columns, 14 sinks and
        # qkv as dense [T, 1152] rows: check what the pointers cannot say.
        for name, tab in (("cos", cos), ("sin", sin)):
            if (tab.dtype != torch.float32 or tab.dim() != 2 or tab.shape[0] < t
                    or tab.shape[1] != HEAD or not tab.is_contiguous() or tab.device != x.device):
                raise ValueError(f"AttnBlock: {name} must be a contiguous f32 [>= {t}, {HEAD}] "
                                 f"table on {x.device}, got {tab.dtype} {list(tab.shape)} on "
                                 f"{tab.device}")
        if (self.sinks.dtype != torch.float32 or tuple(self.sinks.shape) != (Q_HEADS,)
                or not self.sinks.is_contiguous() or self.sinks.device != x.device):
            raise ValueError(f"AttnBlock: sinks must be a contiguous f32 [{Q_HEADS}] on {x.device}")
        qkv = self.qkv.forward(rmsNorm(x, self.norm_w, RMS_EPS))            # [T, 1152] f32
        if tuple(qkv.shape) != (t, K_OFF + 2 * KV_HEADS * HEAD) or not qkv.is_contiguous():
            raise ValueError(f"AttnBlock: qkv projection gave {list(qkv.shape)}")
        # rope(q), rope(k) and the banded sdpa in one kernel (moe_attention)
        attn = torch.empty((t, K_OFF), dtype=qkv.dtype, device=qkv.device)
        _lib.check(_lib.load().moe_attention(
            _ctx(qkv.device), qkv.data_ptr(), _xdtype(qkv), t, Q_HEADS, KV_HEADS, HEAD, WINDOW,
            WINDOW, self.sinks.data_ptr(), cos.data_ptr(), sin.data_ptr(), attn.data_ptr()))
        return self.out.forward(attn, addend=x)


@dataclass
class Block:
    """EagerBlock (model.ts:16-33): attention, then the MoE block."""
    attn: AttnBlock
    mlp: MoeBlock

    def forward(self, x, cos, sin):
        return self.mlp.forward(self.attn.forward(x, cos, sin))


@dataclass
class PrivacyFilterModel:
    """EagerModel (model.ts:44-76): host embedding, blocks, final norm,
    unembed (no bias) → logits [T, classes]."""
    embedding: np.ndarray          # [vocab, 640] on the host
    blocks: List[Block]
    norm_w: torch.Tensor
    unembed: Linear

    def forward(self, token_ids) -> torch.Tensor:
        ids = np.asarray(token_ids, np.int64)
        dev = self.norm_w.device
        t = ids.size
        cos, sin = rope_constants(t)
        cos_t, sin_t = torch.from_numpy(cos).to(dev), torch.from_numpy(sin).to(dev)
        x = torch.from_numpy(np.ascontiguousarray(self.embedding[ids], np.float32)).to(dev)
        for b in self.blocks:
            x = b.forward(x, cos_t, sin_t)
        from .core import rmsNorm
        return self.unembed.forward(rmsNorm(x, self.norm_w, RMS_EPS))


class GraphedForward:
    """The model's forward for a set of text lengths captured as HIP graphs
    (one per length), so a text costs one graph launch instead of ~170
    launches from Python. Each length keeps its own static input (the
    embedding rows are copied in before a replay), rope tables and output.

    The library's context workspace grows by reallocation. A graph holds
    the workspace address it was captured with, so every capture follows an
    eager forward at the longest length (the workspace each op plans grows
    with the rows, so the longest length's covers all), and the workspace is
    pinned while the graphs live: a later call on the same device that needs
    a larger workspace raises EXECUTION_FAILED instead of moving it under
    the graphs. close() (or dropping the object) releases the pin."""

    def __init__(self, model: "PrivacyFilterModel", lengths):
        self.model = model
        dev = model.norm_w.device
        self.stream = torch.cuda.Stream(device=dev)
        self.graphs = {}
        lengths = sorted(set(int(t) for t in lengths), reverse=True)
        cur = torch.cuda.current_stream(dev)
        self.stream.wait_stream(cur)
        with torch.cuda.stream(self.stream):
            for t in lengths[:1]:
                self._body(*self._statics(t, dev))  # grows the workspace once, longest first
        for t in lengths:
            x_in, cos, sin = self._statics(t, dev)
            with torch.cuda.stream(self.stream):
                self._body(x_in, cos, sin)          # warm at this length on the capture stream
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=self.stream):
                out = self._body(x_in, cos, sin)
            self.graphs[t] = (g, x_in, out, cos, sin)
        cur.wait_stream(self.stream)
        from . import _lib
        self._device = dev.index if dev.index is not None else torch.cuda.current_device()
        _lib.pin_workspace(self._device, True)
        self._pinned = True

    def close(self) -> None:
        """Drops the graphs and unpins the workspace."""
        if getattr(self, "_pinned", False):
            from . import _lib
            torch.cuda.synchronize(self._device)
            self.graphs = {}
            _lib.pin_workspace(self._device, False)
            self._pinned = False

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _statics(self, t, dev):
        cos, sin = rope_constants(t)
        return (torch.zeros((t, HIDDEN), dtype=torch.float32, device=dev),
                torch.from_numpy(cos).to(dev), torch.from_numpy(sin).to(dev))

    def _body(self, x, cos, sin):
        from .core import rmsNorm
        for b in self.model.blocks:
            x = b.forward(x, cos, sin)
        return self.model.unembed.forward(rmsNorm(x, self.model.norm_w, RMS_EPS))

    def __call__(self, token_ids) -> torch.Tensor:
        ids = np.asarray(token_ids, np.int64)
        if not getattr(self, "_pinned", False):
            raise RuntimeError("GraphedForward is closed")
        g, x_in, out, _, _ = self.graphs[ids.size]
        x_in.copy_(torch.from_numpy(np.ascontiguousarray(self.model.embedding[ids], np.float32)))
        g.replay()
        return out


# ------------------------------------------------------------ decoding (host)

V2_SPAN_CLASS_NAMES = ["O", "account_number", "private_address", "private_date", "private_email",
                       "private_person", "private_phone", "private_url", "secret"]
V2_NER_CLASS_NAMES = ["O"] + [f"{p}-{base}" for base in V2_SPAN_CLASS_NAMES[1:]
                              for p in ("B", "I", "E", "S")]


@dataclass
class LabelInfo:
    span_class_names: List[str]
    token_to_span_label: dict
    token_boundary_tags: dict
    background_token_label: int
    background_span_label: int
    num_classes: int


def build_label_info(class_names) -> LabelInfo:
    """buildLabelInfo (config.ts:37-75)."""
    spans, lookup = ["O"], {"O": 0}
    to_span, tags, bg = {}, {}, None
    for idx, name in enumerate(class_names):
        if name == "O":
            bg = idx
            to_span[idx], tags[idx] = 0, None
            continue
        dash = name.index("-")
        tag, base = name[:dash], name[dash + 1:]
        if base not in lookup:
            lookup[base] = len(spans)
            spans.append(base)
        to_span[idx], tags[idx] = lookup[base], tag
    if bg is None:
        raise ValueError("Class names must include 'O'")
    return LabelInfo(spans, to_span, tags, bg, 0, len(class_names))


def log_softmax_rows(logits: np.ndarray) -> np.ndarray:
    """logSoftmaxRows (viterbi.ts:5-18), per row in f64, stored f32."""
    x = np.asarray(logits, np.float64)
    m = x.max(axis=1, keepdims=True)
    return (x - (np.log(np.exp(x - m).sum(axis=1, keepdims=True)) + m)).astype(np.float32)


@dataclass
class ViterbiBiases:
    background_stay: float = 0.0
    background_to_start: float = 0.0
    inside_to_continue: float = 0.0
    inside_to_end: float = 0.0
    end_to_background: float = 0.0
    end_to_start: float = 0.0


class ViterbiDecoder:
    """The constrained BIOES decoder (viterbi.ts:20-148): start/end scores
    and a transition matrix of allowed moves (−1e9 elsewhere) with the
    optional biases; ties keep the lower previous label.

    The rules (viterbi.ts:39-77) are the BIOES semantics, so they are stated
    as the reference states them: a label is background when its span class
    is the background one or it is the background token. A next label that
    is neither background nor a tagged span label is never allowed. After a
    label with no span class or no tag, after background, and after an E or
    S tag, only background, B or S may follow; after B or I only I or E of
    the same span class. The bias of an allowed move is looked up on the
    previous label's background status first, then on its tag."""
    NEG_INF = -1e9

    def __init__(self, info: LabelInfo, biases: Optional[ViterbiBiases] = None):
        b = biases or ViterbiBiases()
        n = info.num_classes
        self.n = n
        cls = [info.token_to_span_label.get(i) for i in range(n)]
        tags = [info.token_boundary_tags.get(i) for i in range(n)]
        bg = info.background_token_label
        is_bg = [cls[i] == info.background_span_label or i == bg for i in range(n)]
        opens = [is_bg[i] or tags[i] in ("B", "S") for i in range(n)]  # may follow a closed span

        def allowed(p, q):
            if not is_bg[q] and (cls[q] is None or tags[q] is None):
                return False
            if cls[p] is None or tags[p] is None or is_bg[p] or tags[p] in ("E", "S"):
                return opens[q]
            if tags[p] in ("B", "I"):
                return cls[p] == cls[q] and tags[q] in ("I", "E")
            return False

        def move_bias(p, q):
            if is_bg[p]:
                return (b.background_stay if is_bg[q] else
                        b.background_to_start if tags[q] in ("B", "S") else 0.0)
            if tags[p] in ("B", "I"):
                if cls[p] != cls[q]:
                    return 0.0
                return (b.inside_to_continue if tags[q] == "I" else
                        b.inside_to_end if tags[q] == "E" else 0.0)
            if tags[p] in ("E", "S"):
                return (b.end_to_background if is_bg[q] else
                        b.end_to_start if tags[q] in ("B", "S") else 0.0)
            return 0.0

        self.start = np.array([0.0 if tags[i] in ("B", "S") or i == bg else self.NEG_INF
                               for i in range(n)])
        self.end = np.array([0.0 if tags[i] in ("E", "S") or i == bg else self.NEG_INF
                             for i in range(n)])
        self.trans = np.full((n, n), self.NEG_INF, dtype=np.float64)
        for p in range(n):
            for q in range(n):
                if allowed(p, q):
                    self.trans[p, q] = move_bias(p, q)

    def decode(self, log_probs: np.ndarray) -> List[int]:
        """The library's native decode (moe_viterbi_decode): ties keep the
        lower previous label and the lower last label; with no finite path,
        the per-token argmax."""
        import ctypes
        from . import _lib
        lp = np.ascontiguousarray(log_probs, np.float32)
        if lp.ndim != 2 or lp.shape[1] != self.n:
            raise ValueError(f"Expected width {self.n}, got {lp.shape[-1]}")
        path = np.zeros(lp.shape[0], np.int32)
        p = lambda a: a.ctypes.data_as(ctypes.c_void_p)
        _lib.check(_lib.load().moe_viterbi_decode(p(self.start), p(self.end), p(self.trans), p(lp),
                                                  lp.shape[0], self.n, p(path)))
        return path.tolist()


@dataclass
class TokenSpan:
    label: int
    token_start: int
    token_end: int  # exclusive


def labels_to_spans(labels, info: LabelInfo) -> List[TokenSpan]:
    """labelsToSpans (spans.ts:18-70): token spans from BIOES labels. One
    open span at a time; labels with no span class are skipped, background
    closes the open span, B opens one, I continues the open span of its
    class (or opens one), E closes the open span of its class (or stands
    alone), S stands alone; whatever is open at the end is closed there."""
    out: List[TokenSpan] = []
    open_span = None  # (span class, first token)

    def close(at):
        nonlocal open_span
        if open_span is not None:
            out.append(TokenSpan(open_span[0], open_span[1], at))
        open_span = None

    for i, lab in enumerate(labels):
        c = info.token_to_span_label.get(lab)
        if c is None:
            continue
        kind = "O" if c == info.background_span_label else info.token_boundary_tags.get(lab)
        same = open_span is not None and open_span[0] == c
        if kind == "O":
            close(i)
        elif kind == "B" or (kind == "I" and not same):
            close(i)
            open_span = (c, i)
        elif kind == "E" and same:
            out.append(TokenSpan(c, open_span[1], i + 1))
            open_span = None
        elif kind in ("E", "S"):
            close(i)
            out.append(TokenSpan(c, i, i + 1))
    close(len(labels))
    return out


# ------------------------------------------------------------------ loading

def transform_hf_state_dict(t: dict) -> dict:
    """transformHfPrivacyFilterStateDict (stateDictHooks.ts:41-78): maps the
    official transformers-layout checkpoint ({name: ndarray}) onto this
    model's names. q|k|v projections stack into one qkv weight and bias
    (rows in that order); each expert tensor splits by column into glu and
    lin halves with the expert axis folded into rows ([E, K, 2H] → two
    [E·K, H]; a [E, 2H] bias → two [E, H]); down_proj folds [E, H, K] →
    [E·H, K]; the rest renames; score.bias (all zero) is dropped. Returns a
    new dict; raises CHECKPOINT_MISMATCH for a missing tensor."""
    from .errors import RunntimeError
    src = dict(t)
    out = {}

    def take(name):
        if name not in src:
            raise RunntimeError("CHECKPOINT_MISMATCH",
                                f"privacy-filter state dict: missing tensor '{name}'")
        return src.pop(name)

    def halves(a):
        h = a.shape[-1] // 2
        g, l = a[..., :h], a[..., h:]
        return (np.ascontiguousarray(g.reshape(-1, h)), np.ascontiguousarray(l.reshape(-1, h)))

    n = 0
    while f"model.layers.{n}.input_layernorm.weight" in src:
        hf, d = f"model.layers.{n}", f"block.{n}"
        out[f"{d}.attn.norm.weight"] = take(f"{hf}.input_layernorm.weight")
        out[f"{d}.mlp.norm.weight"] = take(f"{hf}.post_attention_layernorm.weight")
        for suf in ("weight", "bias"):
            out[f"{d}.attn.qkv.{suf}"] = np.concatenate(
                [take(f"{hf}.self_attn.{p_}_proj.{suf}") for p_ in ("q", "k", "v")], axis=0)
            out[f"{d}.attn.out.{suf}"] = take(f"{hf}.self_attn.o_proj.{suf}")
            out[f"{d}.mlp.gate.{suf}"] = take(f"{hf}.mlp.router.{suf}")
        out[f"{d}.attn.sinks"] = take(f"{hf}.self_attn.sinks")
        out[f"{d}.mlp.gluWeight"], out[f"{d}.mlp.linWeight"] = halves(
            take(f"{hf}.mlp.experts.gate_up_proj"))
        out[f"{d}.mlp.gluBias"], out[f"{d}.mlp.linBias"] = halves(
            take(f"{hf}.mlp.experts.gate_up_proj_bias"))
        dp = take(f"{hf}.mlp.experts.down_proj")
        out[f"{d}.mlp.outWeight"] = dp.reshape(-1, dp.shape[-1])
        out[f"{d}.mlp.outBias"] = take(f"{hf}.mlp.experts.down_proj_bias")
        n += 1
    out["embedding.weight"] = take("model.embed_tokens.weight")
    out["norm.weight"] = take("model.norm.weight")
    out["unembedding.weight"] = take("score.weight")
    src.pop("score.bias", None)
    out.update(src)  # anything else passes through under its own name
    return out


@dataclass
class MoeBlockFloat:
    """EagerMoeMlp with float weights (moeMlp.ts:85-100) on moe_block_float:
    glu/lin [E·d, I], out [E·I, d] row-major, biases [E, I] / [E, d]; f32
    here (an f16 or bf16 checkpoint is widened at load, as the network's
    activations are f32)."""
    norm_w: torch.Tensor
    router_w: torch.Tensor      # f32 [d, E]
    router_b: Optional[torch.Tensor]
    glu_w: torch.Tensor
    glu_b: torch.Tensor
    lin_w: torch.Tensor
    lin_b: torch.Tensor
    out_w: torch.Tensor
    out_b: torch.Tensor
    k: int = 4
    eps: float = RMS_EPS

    def forward(self, x):
        from .core import moe_block_float
        return moe_block_float(x, self.norm_w, self.eps, self.router_w, self.router_b, self.glu_w,
                               self.glu_b, self.lin_w, self.lin_b, self.out_w, self.out_b, k=self.k)


def model_from_float_state_dict(sd: dict, device="cuda", k: int = 4) -> "PrivacyFilterModel":
    """The network from float tensors under this model's names (the output
    of transform_hf_state_dict): float Linears, float MoE blocks."""
    from .errors import RunntimeError
    f32 = lambda a: np.ascontiguousarray(np.asarray(a, np.float32))
    dev = lambda a: torch.from_numpy(f32(a)).to(device)

    def need(name):
        if name not in sd:
            raise RunntimeError("CHECKPOINT_MISMATCH",
                                f"privacy-filter state dict: missing tensor '{name}'")
        return sd[name]

    blocks = []
    n = 0
    while f"block.{n}.attn.qkv.weight" in sd:
        p = f"block.{n}"
        attn = AttnBlock(dev(need(f"{p}.attn.norm.weight")).reshape(-1),
                         Linear.from_torch_layout(f32(need(f"{p}.attn.qkv.weight")),
                                                  sd.get(f"{p}.attn.qkv.bias"), device),
                         Linear.from_torch_layout(f32(need(f"{p}.attn.out.weight")),
                                                  sd.get(f"{p}.attn.out.bias"), device),
                         dev(need(f"{p}.attn.sinks")).reshape(-1))
        gate = f32(need(f"{p}.mlp.gate.weight"))        # torch layout [E, d]
        gb = sd.get(f"{p}.mlp.gate.bias")
        mlp = MoeBlockFloat(dev(need(f"{p}.mlp.norm.weight")).reshape(-1), dev(gate.T),
                            dev(gb) if gb is not None else None,
                            dev(need(f"{p}.mlp.gluWeight")), dev(need(f"{p}.mlp.gluBias")),
                            dev(need(f"{p}.mlp.linWeight")), dev(need(f"{p}.mlp.linBias")),
                            dev(need(f"{p}.mlp.outWeight")), dev(need(f"{p}.mlp.outBias")), k=k)
        blocks.append(Block(attn, mlp))
        n += 1
    emb = f32(need("embedding.weight"))
    un = f32(need("unembedding.weight"))
    return PrivacyFilterModel(emb, blocks, dev(need("norm.weight")).reshape(-1),
                              Linear.from_torch_layout(un, None, device))


def load_privacy_filter_hf(path: str, device="cuda", k: int = 4) -> "PrivacyFilterModel":
    """The official transformers-layout checkpoint (no `model` metadata;
    detector.ts:40-48 maps it with transformHfPrivacyFilterStateDict)."""
    from .safetensors import SafetensorsFile
    f = SafetensorsFile(path)
    return model_from_float_state_dict(transform_hf_state_dict({n: f.array(n) for n in f.names}),
                                       device, k)


def _linear_from_file(f, name, in_f, out_f, device, bias_name=None):
    """A Linear from its torch-layout checkpoint weight [out, in]: I8/U8 +
    F16 `_scale` (quantized) or float (layers.ts:193-217)."""
    from .errors import RunntimeError
    if name not in f.names:
        raise RunntimeError("CHECKPOINT_MISMATCH",
                            f"privacy-filter state dict: missing tensor '{name}'")
    bias = f.array(bias_name).astype(np.float32) if bias_name and bias_name in f.names else None
    if name in f.quant:
        qt = f.quant[name]
        if qt.shape != [out_f, in_f]:
            raise RunntimeError("CHECKPOINT_MISMATCH",
                                f"Linear: {name} has shape {qt.shape}, expected torch layout "
                                f"[{out_f}, {in_f}]")
        return Linear.from_quant(qt.ints(), qt.scales(), qt.bits, bias, device, name)
    w = f.array(name)
    if list(w.shape) != [out_f, in_f]:
        raise RunntimeError("CHECKPOINT_MISMATCH",
                            f"Linear: {name} has shape {list(w.shape)}, expected torch layout "
                            f"[{out_f}, {in_f}]")
    return Linear.from_torch_layout(w.astype(np.float32), bias, device)


def load_privacy_filter(path: str, device="cuda", blocks: Optional[int] = None,
                        experts: Optional[int] = None) -> PrivacyFilterModel:
    """The whole network from an exported privacy-filter file (our parameter
    names, RMSNorm scales as `scale` or `weight`; detector.ts:25-90,
    stateDictHooks.ts:80-87): block.{n}.attn.{norm, qkv, out, sinks},
    block.{n}.mlp.* (load_moe_block), embedding.weight, norm, unembedding."""
    from .checkpoint import load_moe_block
    from .errors import RunntimeError
    from .safetensors import SafetensorsFile
    f = SafetensorsFile(path)
    model_meta = f.metadata.get("model") if isinstance(f.metadata, dict) else None
    if model_meta is not None and model_meta != "privacy-filter":
        raise RunntimeError("CHECKPOINT_MISMATCH",
                            f"privacy-filter weights: file is for model '{model_meta}', expected "
                            f"'privacy-filter'")

    def norm(prefix):
        for n in (f"{prefix}.weight", f"{prefix}.scale"):
            if n in f.names:
                return torch.from_numpy(f.array(n).astype(np.float32).reshape(-1)).to(device)
        raise RunntimeError("CHECKPOINT_MISMATCH",
                            f"privacy-filter state dict: missing tensor '{prefix}.weight'")

    def need(name):
        if name not in f.names:
            raise RunntimeError("CHECKPOINT_MISMATCH",
                                f"privacy-filter state dict: missing tensor '{name}'")
        return f.array(name)

    if "embedding.weight" not in f.names:
        raise RunntimeError("CHECKPOINT_MISMATCH", "privacy-filter weights: missing "
                            "'embedding.weight' tensor")
    emb = f.array("embedding.weight").astype(np.float32)
    if emb.ndim != 2 or emb.shape[1] != HIDDEN:
        raise RunntimeError("CHECKPOINT_MISMATCH", f"embedding.weight has shape {list(emb.shape)}, "
                            f"expected [vocab, hidden]")
    n = 0
    while f"block.{n}.attn.qkv.weight" in f.names:
        n += 1
    if blocks is not None and n != blocks:
        raise RunntimeError("CHECKPOINT_MISMATCH",
                            f"privacy-filter weights: {n} blocks in the file, expected {blocks}")
    out_blocks = []
    for b in range(n):
        p = f"block.{b}.attn"
        attn = AttnBlock(norm(f"{p}.norm"),
                         _linear_from_file(f, f"{p}.qkv.weight", HIDDEN, QKV_WIDTH, device,
                                           f"{p}.qkv.bias"),
                         _linear_from_file(f, f"{p}.out.weight", ATTN_OUT, HIDDEN, device,
                                           f"{p}.out.bias"),
                         torch.from_numpy(need(f"{p}.sinks").astype(np.float32)
                                          .reshape(-1)).to(device))
        out_blocks.append(Block(attn, load_moe_block(path, b, device, experts=experts,
                                                     hidden=HIDDEN)))
    un = f.infos["unembedding.weight"].shape if "unembedding.weight" in f.names else None
    if un is None:
        raise RunntimeError("CHECKPOINT_MISMATCH",
                            "privacy-filter state dict: missing tensor 'unembedding.weight'")
    unembed = _linear_from_file(f, "unembedding.weight", HIDDEN, un[0], device)
    return PrivacyFilterModel(emb, out_blocks, norm("norm"), unembed)
