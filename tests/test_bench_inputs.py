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


def test_profile_facts_follow_the_route(tmp_path, monkeypatch):
    """bench.measured() reports a committed counter figure only while the call
    runs the kernels it was measured on, and says why otherwise."""
    bench = _bench()
    (tmp_path / "a.md").write_text(
        "text\n```json\n"
        '[{"kind": "traffic_bytes", "bits": 4, "m": 1, "k": 4096, "n": 4096, "algo": "auto", '
        '"route": "row::qmv_row_kernel<4, 2, 2, 4, 1, 0>", "value": 123}]\n```\n')
    monkeypatch.setattr(bench, "PROFILES", tmp_path)
    facts = bench.profile_facts()
    assert facts[0]["file"] == "profiles/a.md"

    class Lib:
        ALGO_AUTO, ALGO_QMM, ALGO_QMM_LIB = 0, 2, 3
        route = "row::qmv_row_kernel<4, 2, 2, 4, 1, 0>"

        def qmatmul_route(self, m, n, k, gs, bits, algo=0):
            return self.route

    lib = Lib()
    assert bench.measured(facts, lib, "traffic_bytes", 4, 1, 4096, 4096) == (123, "profiles/a.md")
    lib.route = "row::qmv_row_kernel<4, 1, 2, 4, 1, 0>"
    v, why = bench.measured(facts, lib, "traffic_bytes", 4, 1, 4096, 4096)
    assert v is None and "now runs" in why
    assert bench.measured(facts, lib, "mfma_busy", 4, 1, 4096, 4096) == (None, "not measured")


def test_committed_profile_facts_parse():
    """Every machine-readable block under profiles/ parses and names a route."""
    bench = _bench()
    facts = bench.profile_facts()
    assert facts, "no facts committed"
    for f in facts:
        assert {"kind", "bits", "m", "k", "n", "route", "value"} <= set(f)
        assert f["value"] > 0 and f["route"]
