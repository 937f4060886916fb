"""The benchmark's device-side GGUF input generator (bench.gguf_blocks) makes
the same blocks as the oracle's llama.cpp-layout quantizer, so the bench's
config-4 leg times blocks of the layouts the reference decodes
(src/gguf/dequant.rs)."""
import importlib.util
from pathlib import Path

import numpy as np
import pytest

import oracle as orc

ROOT = Path(__file__).resolve().parent.parent


def _bench():
    spec = importlib.util.spec_from_file_location("bench_mod", ROOT / "bench.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


@pytest.mark.parametrize("tname", ["Q4_0", "Q8_0", "Q4_K", "Q6_K", "IQ4_NL", "IQ4_XS"])
def test_gguf_blocks_match_oracle_quantizer(tname):
    import torch

    bench = _bench()
    tag = {"Q4_0": 2, "Q8_0": 8, "Q4_K": 12, "Q6_K": 14, "IQ4_NL": 20, "IQ4_XS": 23}[tname]
    n = 256 * 96
    x = orc.normal(0x5EED0400 + tag, n, 0.0, 0.02)
    x[::97] *= 20  # a few large values: the signed-absmax and clamping paths
    got = bench.gguf_blocks(torch, tname, torch.from_numpy(x)).numpy()
    want = orc.gguf_quantize(tag, x)
    assert got.size == want.size == orc.gguf_tensor_byte_len(tag, n)
    assert np.array_equal(got, want)
    # and the blocks decode to the values they came from
    y = orc.gguf_dequantize(tag, got, n)
    assert np.abs(y - x).max() <= 0.2 * np.abs(x).max()
