"""Affine group-wise quantize / dequantize on the GPU vs the CPU restatement
of MLX's algorithm: bit-exact codes, scales and biases."""
import json
from pathlib import Path

import numpy as np
import pytest

import mlxq
import oracle as orc
from helpers import bf16_weights, dev, host

pytestmark = pytest.mark.gpu
KAT = json.loads((Path(__file__).resolve().parent / "golden" / "gguf_kat.json").read_text())


def gpu_quantize(w, gs, bits, bf16):
    import torch

    wq, s, b = mlxq.quantize(dev(w, bf16=bf16), gs, bits)
    torch.cuda.synchronize()
    return host(wq), host(s), host(b)


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("gs", [32, 64, 128])
@pytest.mark.parametrize("bf16", [True, False])
def test_codes_bit_exact(torch_gpu, bits, gs, bf16):
    rows, cols = 96, 1024
    w = bf16_weights(1000 + bits + gs, rows, cols)
    if not bf16:
        w = orc.normal(2000 + bits + gs, rows * cols, 0.0, 0.02).reshape(rows, cols)
    w = w.copy()
    # edge cases: constant group, zero group, one outlier, exact ramp
    if bf16:
        w[0, :gs] = orc.f32_to_bf16(np.float32([0.25]))[0]
        w[1, :gs] = 0
        w[2, 5] = orc.f32_to_bf16(np.float32([3.0]))[0]
    else:
        w[0, :gs] = 0.25
        w[1, :gs] = 0
        w[2, 5] = 3.0
        w[3, :gs] = np.arange(gs) % 16
    ref = orc.affine_quantize(w, gs, bits, orc.BF16 if bf16 else orc.F32)
    got = gpu_quantize(w, gs, bits, bf16)
    for r, g in zip(ref, got):
        assert np.array_equal(np.asarray(r).view(np.uint8), np.asarray(g).view(np.uint8))


@pytest.mark.parametrize("bits", [4, 8])
def test_dequantize_bit_exact(torch_gpu, bits):
    import torch

    w = bf16_weights(31 + bits, 64, 512)
    wq, s, b = orc.affine_quantize(w, 64, bits, orc.BF16)
    ref = orc.affine_dequantize(wq, s, b, 64, bits, orc.BF16)
    got = mlxq.dequantize(dev(wq), dev(s, bf16=True), dev(b, bf16=True), 64, bits)
    torch.cuda.synchronize()
    assert np.array_equal(host(got), ref)
    wf = orc.normal(40 + bits, 64 * 512, 0, 0.02).reshape(64, 512)
    wq, s, b = orc.affine_quantize(wf, 64, bits, orc.F32)
    ref = orc.affine_dequantize(wq, s, b, 64, bits, orc.F32)
    got = mlxq.dequantize(dev(wq), dev(s), dev(b), 64, bits)
    torch.cuda.synchronize()
    assert np.array_equal(host(got).view(np.uint32), ref.view(np.uint32))


def test_reference_roundtrip_q8(torch_gpu):
    import torch

    a = KAT["affine"]["roundtrip_q8"]  # quant.rs:91-107
    w = np.float32(a["w"]).reshape(a["shape"])
    wq, s, b = mlxq.quantize(dev(w), 64, 8)
    back = host(mlxq.dequantize(wq, s, b, 64, 8))
    torch.cuda.synchronize()
    assert np.max(np.abs(back - w)) < a["max_abs_err"]


@pytest.mark.parametrize("shape", [(4096, 4096), (14336, 4096), (4096, 14336)])
@pytest.mark.parametrize("bits", [4, 8])
def test_llama_shapes_bit_exact(torch_gpu, shape, bits):
    n, k = shape
    w = bf16_weights(0x5EED0000 + n + k + bits, n, k)
    ref = orc.affine_quantize(w, 64, bits, orc.BF16)
    got = gpu_quantize(w, 64, bits, True)
    for r, g in zip(ref, got):
        assert np.array_equal(r.view(np.uint8), g.view(np.uint8))


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("factor", [1.0, 0.02, 3.0e-5, 7.0, 0.0123457, 3.3e-3, 1.7e-6, 0.7071068, 511.3, 9.9e-2,
                                    3.1e20, 2.0e30])
def test_codes_at_rounding_ties(torch_gpu, bits, factor):
    """Groups whose quotients (w - bias) / scale sit on or within a few ulps
    of half-integers: min 0 and max n_bins (times `factor`) make scale
    -factor and bias max, so every element j + 1/2 (times `factor`) lands on a
    tie of the code rounding; with factor not a power of two the f32 products
    put the quotients a few ulps to either side of it.  The two largest
    factors give scales above 2^60, where the quantizer takes the division
    instead of its unscaled form of it."""
    rng = np.random.default_rng(77 + bits)
    n_bins = (1 << bits) - 1
    gs, rows, cols = 64, 64, 512
    half = rng.integers(0, 2 * n_bins + 1, size=(rows, cols)).astype(np.float32) / 2
    half = half.reshape(rows, cols // gs, gs)
    half[:, :, 0] = 0
    half[:, :, 1] = n_bins
    w = (half.reshape(rows, cols) * np.float32(factor)).astype(np.float32)
    ref = orc.affine_quantize(w, gs, bits, orc.F32)
    got = gpu_quantize(w, gs, bits, False)
    for r, g in zip(ref, got):
        assert np.array_equal(np.asarray(r).view(np.uint8), np.asarray(g).view(np.uint8))
