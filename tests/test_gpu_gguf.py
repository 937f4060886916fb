"""GGUF block dequant on the GPU vs the CPU restatement of src/gguf/dequant.rs:
bit-exact f32 (and bf16 = RNE of that f32)."""
import json
from pathlib import Path

import numpy as np
import pytest

import mlxq
import oracle as orc
from helpers import dev, host

pytestmark = pytest.mark.gpu
KAT = json.loads((Path(__file__).resolve().parent / "golden" / "gguf_kat.json").read_text())
DEVICE_TAGS = [2, 3, 6, 7, 8, 10, 11, 12, 13, 14, 20, 23, 16, 17, 22, 18, 21, 19, 29]
STAR_TAGS = [2, 8, 12, 14, 20, 23]  # Q4_0 Q8_0 Q4_K Q6_K IQ4_NL IQ4_XS
rng = np.random.default_rng(77)


def gpu_dequant(tag, data, n, out_dtype=None, offset=0):
    import torch

    buf = np.zeros(data.size + offset, np.uint8)
    buf[offset:] = data
    d = dev(buf)[offset:]
    out = mlxq.gguf_dequantize(tag, d, n, out_dtype or torch.float32)
    torch.cuda.synchronize()
    return host(out)


def random_blocks(tag, nblk):
    """Random bytes with every f16 scale field forced finite (|d| < 2)."""
    e, b = orc.gguf_block(tag)
    raw = rng.integers(0, 256, size=(nblk, b), dtype=np.uint8)
    d_off = {2: [0], 3: [0, 2], 6: [0], 7: [0, 2], 8: [0], 10: [80, 82], 11: [108], 12: [0, 2], 13: [0, 2],
             14: [208], 20: [0], 23: [0], 16: [0], 17: [0], 22: [0], 18: [0], 21: [0], 19: [0]}.get(tag, [])
    for o in d_off:
        raw[:, o + 1] &= 0x3B  # exponent <= 14: finite, below 2
    if tag == 29:  # IQ1_M: f16 bits 12-15 (sign, exponent top) are the top nibble of the last scale word
        raw[:, 55] &= 0x3F
    return raw.ravel(), e * nblk


@pytest.mark.parametrize("case", KAT["cases"], ids=lambda c: c["name"])
def test_reference_known_answers(torch_gpu, case):
    data = np.frombuffer(bytes.fromhex(case["hex"]), dtype=np.uint8).copy()
    out = gpu_dequant(case["tag"], data, case["n"])
    if "expect_all" in case:
        assert np.array_equal(out, np.float32(case["expect_all"]))
    for i, v in case.get("expect", {}).items():
        assert out[int(i)] == np.float32(v)


@pytest.mark.parametrize("tag", DEVICE_TAGS)
def test_random_blocks_bit_exact(torch_gpu, tag):
    data, n = random_blocks(tag, 3 * 2048 // orc.gguf_block(tag)[0] + 5)  # ragged last chunk
    ref = orc.gguf_dequantize(tag, data, n)
    got = gpu_dequant(tag, data, n)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    got_bf16 = gpu_dequant(tag, data, n, torch_gpu.bfloat16)
    assert np.array_equal(got_bf16, orc.f32_to_bf16(ref))


@pytest.mark.parametrize("tag", DEVICE_TAGS)
def test_ragged_chunk_past_its_first_half(torch_gpu, tag):
    """A last chunk of 1280 elements: the f32 kernels that store a chunk as
    two 1 KB halves (elements tid*4.. and 1024 + tid*4..) write all of the
    first half and part of the second."""
    e = orc.gguf_block(tag)[0]
    data, n = random_blocks(tag, 3 * 2048 // e + 1280 // e)
    ref = orc.gguf_dequantize(tag, data, n)
    got = gpu_dequant(tag, data, n)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    assert np.array_equal(gpu_dequant(tag, data, n, torch_gpu.bfloat16), orc.f32_to_bf16(ref))


@pytest.mark.parametrize("tag", [2, 12, 14, 23])
def test_unaligned_input_pointer(torch_gpu, tag):
    data, n = random_blocks(tag, 40)
    ref = orc.gguf_dequantize(tag, data, n)
    for off in (1, 2, 6):
        assert np.array_equal(gpu_dequant(tag, data, n, offset=off).view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("tag", [0, 1, 30])
def test_float_passthrough(torch_gpu, tag):
    n = 1000
    if tag == 0:
        data = orc.normal(3, n).view(np.uint8)
    else:
        data = rng.integers(0, 2**16, n, dtype=np.uint64).astype(np.uint16)
        data[(data & 0x7C00) == 0x7C00] = 0  # no inf/nan
        data = data.view(np.uint8)
    ref = orc.gguf_dequantize(tag, data, n)
    assert np.array_equal(gpu_dequant(tag, data, n).view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("tag", STAR_TAGS)
def test_config4_full_tensor(torch_gpu, tag):
    """14336 x 4096 blocks quantized from seeded N(0, 0.02) with llama.cpp layouts."""
    n = 14336 * 4096
    x = orc.normal(0x5EED0400 + tag, n, 0.0, 0.02)
    blocks = orc.gguf_quantize(tag, x)
    assert blocks.size == orc.gguf_tensor_byte_len(tag, n)
    ref = orc.gguf_dequantize(tag, blocks, n, threads=16)
    got = gpu_dequant(tag, blocks, n)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    got_bf16 = gpu_dequant(tag, blocks, n, torch_gpu.bfloat16)
    assert np.array_equal(got_bf16, orc.f32_to_bf16(ref))


@pytest.mark.parametrize("tag", DEVICE_TAGS)
def test_random_blocks_any_f16_scale(torch_gpu, tag):
    """Unrestricted block bytes: f16 scales negative, subnormal, infinite or
    NaN (the reference decodes them through half::f16::to_f32 and passes
    them on, dequant.rs:222-225).  Every non-NaN output is bit-exact.  Where
    the output is NaN, the oracle's is too; a NaN that propagates from a NaN
    scale keeps its payload bit for bit; one that an operation creates
    (inf - inf, 0 * inf) is the platform's default NaN, which differs in the
    sign bit between x86 and this GPU, so those are compared as NaN only.
    Types whose outputs combine two f16 scales (d and dmin: Q4_1, Q5_1, Q2_K,
    Q4_K, Q5_K) can meet two NaN operands in one operation; IEEE 754 leaves
    which payload survives to the implementation, so there only the NaN
    positions are compared."""
    e, b = orc.gguf_block(tag)
    nblk = 2048 // e * 3 + 7
    raw = np.random.default_rng(1000 + tag).integers(0, 256, size=nblk * b, dtype=np.uint8)
    n = e * nblk
    ref = orc.gguf_dequantize(tag, raw, n).view(np.uint32)
    got = gpu_dequant(tag, raw, n).view(np.uint32)
    rn = (ref & 0x7FFFFFFF) > 0x7F800000
    gn = (got & 0x7FFFFFFF) > 0x7F800000
    assert np.array_equal(rn, gn)
    assert np.array_equal(got[~rn], ref[~rn])
    if tag not in (3, 7, 10, 12, 13):
        created = (ref[rn] & 0x7FFFFFFF) == 0x7FC00000  # a default NaN, either sign
        assert np.array_equal(got[rn][~created], ref[rn][~created])
        assert np.all((got[rn][created] & 0x7FFFFFFF) == 0x7FC00000)
    got_bf16 = gpu_dequant(tag, raw, n, torch_gpu.bfloat16)
    want_bf16 = orc.f32_to_bf16(ref.view(np.float32))
    bn = (want_bf16 & 0x7FFF) > 0x7F80
    assert np.array_equal((got_bf16 & 0x7FFF) > 0x7F80, bn)
    assert np.array_equal(got_bf16[~bn], want_bf16[~bn])
