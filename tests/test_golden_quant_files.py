"""The reference's own quantized safetensors fixtures (tools/python/tests/
golden/tiny*.safetensors, written by its quantizer) read through this
package's reader: the int8 and int4 weights and their f16 scales equal the
published quantization of the float file's weight (tools/python/src/
runntime_tools/quantize.py:22-37: per group of in-features, scale =
f16(absmax / (2^(bits−1) − 1)), int = clip(rint(w / scale)), an all-zero
group scale 0), restated here; a quantized Linear made from them runs on
the GPU (moe_down with one expert) against x·dequant(W)ᵀ + b."""
import os

import numpy as np
import pytest

from runntime_amd.safetensors import SafetensorsFile

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def _quantize(w, bits, g):
    largest = 2 ** (bits - 1) - 1
    out_f, in_f = w.shape
    grp = w.reshape(out_f, in_f // g, g)
    scales = (np.abs(grp).max(-1, keepdims=True) / largest).astype(np.float16)
    div = scales.astype(np.float32)
    ratio = np.divide(grp, div, out=np.zeros_like(grp), where=div != 0)
    ints = np.clip(np.rint(ratio), -largest, largest).astype(np.int8)
    return ints.reshape(out_f, in_f), scales[..., 0].astype(np.float32)


@pytest.mark.parametrize("bits", [8, 4])
def test_reader_matches_the_published_quantization(bits):
    f = SafetensorsFile(os.path.join(GOLDEN, "tiny.safetensors"))
    q = SafetensorsFile(os.path.join(GOLDEN, f"tiny.int{bits}.safetensors"))
    assert "layer.weight" in q.quant and "layer.weight_scale" not in q.names
    qt = q.quant["layer.weight"]
    assert (qt.bits, qt.group_size, qt.shape) == (bits, 32, [8, 64])
    ints, scales = _quantize(f.array("layer.weight").astype(np.float32), bits, 32)
    np.testing.assert_array_equal(qt.ints(), ints)
    np.testing.assert_array_equal(qt.scales(), scales)
    # the tensors that stay float pass through unchanged
    for name in ("embed.weight", "layer.bias", "norm.weight"):
        np.testing.assert_array_equal(q.array(name), f.array(name))


@pytest.mark.gpu
@pytest.mark.parametrize("bits", [8, 4])
def test_quantized_linear_from_the_golden_file(bits):
    import torch
    from runntime_amd.linear import Linear
    q = SafetensorsFile(os.path.join(GOLDEN, f"tiny.int{bits}.safetensors"))
    qt = q.quant["layer.weight"]
    bias = q.array("layer.bias")
    lin = Linear.from_quant(qt.ints(), qt.scales(), bits, bias, "cuda")
    rng = np.random.default_rng(5)
    x = rng.standard_normal((37, 64)).astype(np.float32)
    add = rng.standard_normal((37, 8)).astype(np.float32)
    got = lin.forward(torch.from_numpy(x).cuda(), torch.from_numpy(add).cuda())
    w = qt.ints().astype(np.float64).reshape(8, 2, 32) * qt.scales().astype(np.float64)[..., None]
    want = x.astype(np.float64) @ w.reshape(8, 64).T + bias + add
    np.testing.assert_allclose(got.cpu().numpy(), want, atol=1e-5, rtol=1e-5)
