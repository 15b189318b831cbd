"""MI355X-native int8 mixture-of-experts layer with ruNNtime's core MoE op API.

Ops (same names and argument meaning as packages/runntime/src/core):
  topk, moeUp, moeDown, rmsNorm, matmulGather — the reference's graph ops
  router_topk, moe_layer    — the router+topk fusion and the whole layer
  moe_block                 — EagerMoeMlp.forward (pre-norm + layer + residual)
  moe_block_float           — the same block with f32/f16 expert weights
  load_moe_block, MoeBlock  — one block's weights from the hosted safetensors layout
Host-side format helpers: pack_quant_w, pack_expert_weights, QuantW,
QuantExpertWeight. The compute runs in libmoe.so (HIP, gfx950); see
include/runntime_moe.h for its C ABI.
"""
from .errors import RUNNTIME_ERROR_CODES, RunntimeError, is_runntime_error
from .quantw import (QuantExpertWeight, QuantW, pack_expert_weights, pack_expert_weights_torch,
                     pack_quant_w)
from .checkpoint import MoeBlock, load_moe_block, save_moe_block
from .core import (UploadedExpertWeight, dispatch, matmulGather, moe_block, moe_block_float,
                   moe_layer, moe_layer_batched, moeDown, moeUp, pack_quant_w_device, rmsNorm,
                   rope, router_topk, sdpa, sdpaPacked, topk, upload_expert_weight)

__all__ = [
    "RUNNTIME_ERROR_CODES", "RunntimeError", "is_runntime_error", "QuantExpertWeight", "QuantW",
    "pack_expert_weights", "pack_expert_weights_torch", "pack_quant_w", "dispatch", "moe_layer",
    "moe_layer_batched", "pack_quant_w_device",
    "moeDown", "moeUp", "router_topk", "topk", "UploadedExpertWeight", "upload_expert_weight",
    "moe_block", "rmsNorm", "MoeBlock", "load_moe_block", "save_moe_block", "matmulGather",
    "moe_block_float", "rope", "sdpa", "sdpaPacked",
]
