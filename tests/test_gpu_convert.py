"""Fused on-device GGUF -> MLX requantization (mlxq_gguf_requantize) against
the oracle's restatement of the reference convert chain (convert.rs:131-176):
dequantize -> q/k un-permute -> bf16 -> MLX affine quantize.  Integer codes
and bf16 scales/biases: bit-exact."""
import numpy as np
import pytest

import mlxq
import oracle as orc
from helpers import dev, host

pytestmark = pytest.mark.gpu

TAGS = {"F32": 0, "F16": 1, "BF16": 30, "Q4_0": 2, "Q4_1": 3, "Q5_0": 6, "Q5_1": 7, "Q8_0": 8, "Q2_K": 10,
        "Q3_K": 11, "Q4_K": 12, "Q5_K": 13, "Q6_K": 14, "IQ4_NL": 20, "IQ4_XS": 23, "IQ2_XXS": 16, "IQ2_XS": 17,
        "IQ2_S": 22, "IQ3_XXS": 18, "IQ3_S": 21, "IQ1_S": 19, "IQ1_M": 29}


def blocks(tag, rows, cols, seed):
    w = orc.normal(seed, rows * cols, 0.0, 0.02)
    if tag == 0:
        return w.view(np.uint8).copy()
    if tag == 1:
        return w.astype(np.float16).view(np.uint8).copy()
    if tag == 30:
        return orc.f32_to_bf16(w).view(np.uint8).copy()
    if tag in (2, 8, 12, 14, 20, 23):  # the oracle has llama.cpp-style producers for these
        return orc.gguf_quantize(tag, w)
    # other types: random block bytes with every f16 scale field finite (|d| < 2)
    e, nb = orc.gguf_block(tag)
    raw = np.random.default_rng(seed).integers(0, 256, size=(rows * cols // e, nb), dtype=np.uint8)
    for o in {3: [0, 2], 6: [0], 7: [0, 2], 10: [80, 82], 11: [108], 13: [0, 2]}.get(tag, [0] if tag != 29 else []):
        raw[:, o + 1] &= 0x3B
    if tag == 29:  # IQ1_M: the f16 scale's top nibble is the last scale word's
        raw[:, 55] &= 0x3F
    return raw.ravel()


def run(tag, data, rows, cols, heads, gs, bits):
    import torch

    wq, s, b = mlxq.gguf_requantize(tag, torch.from_numpy(data).cuda(), rows, cols, heads, gs, bits)
    torch.cuda.synchronize()
    return host(wq), host(s), host(b)


@pytest.mark.parametrize("name", list(TAGS))
@pytest.mark.parametrize("bits", [4, 8])
def test_requantize_every_tag(torch_gpu, name, bits):
    tag = TAGS[name]
    rows, cols = 64, 512
    data = blocks(tag, rows, cols, 900 + tag)
    got = run(tag, data, rows, cols, 0, 64, bits)
    want = orc.gguf_requantize(tag, data, rows, cols, 0, 64, bits)
    for g, w in zip(got, want):
        assert np.array_equal(g, w)


@pytest.mark.parametrize("gs", [32, 64, 128])
@pytest.mark.parametrize("heads", [0, 4])
def test_requantize_unpermute(torch_gpu, gs, heads):
    rows, cols = 512, 1024  # 4 heads x 128 rows
    data = blocks(12, rows, cols, 950 + gs)
    got = run(12, data, rows, cols, heads, gs, 4)
    want = orc.gguf_requantize(12, data, rows, cols, heads, gs, 4)
    for g, w in zip(got, want):
        assert np.array_equal(g, w)


@pytest.mark.parametrize("name,rows,cols,heads", [("Q4_K", 1024, 4096, 8), ("Q6_K", 14336, 4096, 0),
                                                  ("IQ4_XS", 4096, 14336, 0)])
def test_requantize_llama3_shapes(torch_gpu, name, rows, cols, heads):
    """Config-4 / Llama-3-8B projection shapes (k_proj un-permuted over 8 KV heads)."""
    tag = TAGS[name]
    data = blocks(tag, rows, cols, 960 + tag)
    got = run(tag, data, rows, cols, heads, 64, 4)
    want = orc.gguf_requantize(tag, data, rows, cols, heads, 64, 4)
    for g, w in zip(got, want):
        assert np.array_equal(g, w)


def test_requantize_errors(torch_gpu):
    import torch

    d = torch.zeros(18 * 4, dtype=torch.uint8, device="cuda")
    with pytest.raises(mlxq.MlxqError):  # data shorter than the blocks (2 rows x 64 Q4_0 = 4 blocks... x2)
        mlxq.gguf_requantize(2, d, 4, 64, 0, 64, 4)
    with pytest.raises(mlxq.Unsupported):  # tag 9 (Q8_1) is not a type the reference decodes
        mlxq.gguf_requantize(9, d, 1, 32, 0, 32, 4)
    with pytest.raises(mlxq.MlxqError):  # odd head_dim
        mlxq.gguf_requantize(2, torch.zeros(18 * 6, dtype=torch.uint8, device="cuda"), 6, 32, 2, 32, 4)
