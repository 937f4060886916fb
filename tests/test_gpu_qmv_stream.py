"""Streaming form of the batched-decode GEMV (qmv_tile.hip,
qmv_stream_kernel): a workgroup owns its weight rows over a run of K slices,
with the next slices' codes and activations in flight while it works on the
current one.  Forced onto small shapes through MLXQ_QMV_TILE_STREAM (waves,
Q4 chunks per wave, K parts, K splits) and checked against the f64 CPU
oracle; the default dispatch is checked at the Llama-3-8B shapes it is chosen
for.  Bar: max|y - ref| / max|ref| <= 4e-3 (bf16 output rounding)."""
import numpy as np
import pytest

import oracle as orc
from helpers import bf16_acts, rel_err
from test_gpu_qmatmul import TIGHT, make_layer, run

pytestmark = pytest.mark.gpu


@pytest.fixture
def stream(monkeypatch):
    monkeypatch.setenv("MLXQ_QMV_TILE_ALL", "1")
    monkeypatch.delenv("MLXQ_QMV_TILE", raising=False)
    return monkeypatch


# (config, K): K slices of 512 (Q4 chunks x K parts x 128 codes) give 1, 2,
# 3, 4 and 8 steps per workgroup; splits divide the steps
CASES = [
    ("8,2,2,1", 512),    # one step
    ("8,2,2,1", 1536),   # three steps (odd: the loop's second half skipped at the end)
    ("8,2,2,1", 4096),   # eight steps
    ("8,4,2,1", 2048),   # two steps of 1024
    ("8,4,2,1", 3072),   # three steps of 1024
    ("8,2,4,1", 2048),   # K parts of 4 (two row groups)
    ("4,2,1,1", 1024),   # one K part
    ("4,4,1,1", 1536),
    ("8,2,1,1", 2048),   # eight row groups
    ("8,4,1,1", 1024),
    ("8,2,2,2", 4096),   # two splits of four steps
    ("8,2,2,4", 4096),   # four splits of two steps
    ("8,2,2,4", 2048),   # four splits of one step
    ("4,4,1,4", 4096),
    ("8,2,8,1", 2048),   # eight K parts: one step (M blocks of 16 above 16 rows)
    ("8,2,8,1", 6144),   # three steps
    ("8,2,8,2", 8192),   # two splits of two steps
]


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("cfg,k", CASES)
@pytest.mark.parametrize("m", [5, 16, 17, 32])
def test_stream_configs(torch_gpu, stream, bits, cfg, k, m):
    stream.setenv("MLXQ_QMV_TILE_STREAM", cfg)
    n = 200  # not a multiple of the row group (rows past N repeat N-1, dropped)
    wq, s, b = make_layer(90 + bits, n, k, 64, bits)
    x = bf16_acts(91 + m, m, k)
    ref = orc.qmatmul_f64(x, wq, s, b, 64, bits)
    assert rel_err(run(x, wq, s, b, 64, bits), ref) <= TIGHT


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("cfg", ["8,4,2,1", "8,2,2,4"])
def test_stream_bias_and_outliers(torch_gpu, stream, bits, cfg):
    stream.setenv("MLXQ_QMV_TILE_STREAM", cfg)
    n, k, m = 640, 4096, 24
    wq, s, b = make_layer(95 + bits, n, k, 64, bits, outlier_cols=8)
    x = bf16_acts(96, m, k)
    bias = orc.f32_to_bf16(np.random.default_rng(97).normal(0, 1, n).astype(np.float32))
    ref = orc.qmatmul_f64(x, wq, s, b, 64, bits) + orc.bf16_to_f32(bias)[None, :].astype(np.float64)
    assert rel_err(run(x, wq, s, b, 64, bits, bias=bias), ref) <= TIGHT


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("proj,m", [("gate_up", 8), ("gate_up", 16), ("gate_up", 32), ("down", 12), ("down", 16), ("down", 32)])
def test_stream_default_llama(torch_gpu, monkeypatch, bits, proj, m):
    """The shapes the default dispatch streams (no overrides), sampled rows
    against the oracle."""
    for v in ("MLXQ_QMV_TILE_STREAM", "MLXQ_QMV_TILE", "MLXQ_QMV_TILE_ALL"):
        monkeypatch.delenv(v, raising=False)
    k, n = {"gate_up": (4096, 14336), "down": (14336, 4096)}[proj]
    wq, s, b = make_layer(98 + bits, n, k, 64, bits)
    x = bf16_acts(99 + m, m, k)
    y = run(x, wq, s, b, 64, bits)
    rows = np.random.default_rng(100).choice(n, 256, replace=False)
    ref = orc.qmatmul_f64(x, wq[rows], s[rows], b[rows], 64, bits)
    assert rel_err(y[:, rows], ref) <= TIGHT


def test_stream_graph_replay_bit_exact(torch_gpu, stream):
    """HIP-graph replays of the streaming form (with K splits and without)
    equal the eager call bit for bit, with eager work between replays."""
    import torch

    import mlxq
    from helpers import dev

    stream.setenv("MLXQ_QMV_TILE_STREAM", "8,2,2,2")
    n, k, m = 512, 4096, 32
    wq, s, b = make_layer(101, n, k, 64, 4)
    x = bf16_acts(102, m, k)
    xd, wd, sd, bd = dev(x, bf16=True), dev(wq), dev(s, bf16=True), dev(b, bf16=True)
    y = torch.empty((m, n), dtype=torch.bfloat16, device="cuda")
    call = mlxq.bind_qmatmul(xd, wd, sd, bd, 64, 4, out=y)
    call()
    torch.cuda.synchronize()
    eager = y.clone()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        call()
    for i in range(3):
        y.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, eager), i
        mlxq.qmatmul(xd, wd, sd, bd, 64, 4)  # eager work on the same workspace in between
        torch.cuda.synchronize()


@pytest.fixture(scope="module")
def tall_layers():
    """A ragged very tall gate/up-like matrix (65544 rows, an lm_head's
    shape class) per bit width, quantized once by the oracle."""
    return {bits: make_layer(0x7A11 + bits, 65544, 4096, 64, bits) for bits in (4, 8)}


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("m", [4, 16, 32])
def test_stream_default_very_tall(torch_gpu, monkeypatch, tall_layers, bits, m):
    """Very tall matrices (N >= 65536) stream in 4-wave workgroups under the
    default dispatch; sampled rows (the ragged last ones included) against
    the oracle."""
    for v in ("MLXQ_QMV_TILE_STREAM", "MLXQ_QMV_TILE", "MLXQ_QMV_TILE_ALL"):
        monkeypatch.delenv(v, raising=False)
    n, k = 65544, 4096
    wq, s, b = tall_layers[bits]
    x = bf16_acts(0x7A12 + m, m, k)
    y = run(x, wq, s, b, 64, bits)
    rows = np.concatenate([np.random.default_rng(0x7A13).choice(n - 8, 248, replace=False), np.arange(n - 8, n)])
    ref = orc.qmatmul_f64(x, wq[rows], s[rows], b[rows], 64, bits)
    assert rel_err(y[:, rows], ref) <= TIGHT


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("m,force", [(65, False), (96, False), (128, False), (33, True), (200, True)])
def test_stream64_short_prefill(torch_gpu, monkeypatch, bits, m, force):
    """Short prefills of gate/up-like matrices on the 64-row streaming form
    (grid z = blocks of 64 activation rows, ragged last block): taken by
    default at 65..128 rows (no workspace), forced outside that range with
    MLXQ_QMV_STREAM64=1; sampled rows with a bias against the oracle."""
    import mlxq
    for v in ("MLXQ_QMV_TILE_STREAM", "MLXQ_QMV_TILE", "MLXQ_QMV_TILE_ALL", "MLXQ_QMV_STREAM64"):
        monkeypatch.delenv(v, raising=False)
    if force:
        monkeypatch.setenv("MLXQ_QMV_STREAM64", "1")
    mlxq.reload_overrides()
    k, n = 4096, 14336
    if not force:
        assert mlxq.workspace_size(m, n, k, 64, bits) == 0
    wq, s, b = make_layer(0x6400 + bits, n, k, 64, bits)
    x = bf16_acts(0x6401 + m, m, k)
    bias = orc.f32_to_bf16(np.linspace(-1, 1, n, dtype=np.float32))
    y = run(x, wq, s, b, 64, bits, bias=bias)
    rows = np.concatenate([np.random.default_rng(0x6402).choice(n - 8, 120, replace=False), np.arange(n - 8, n)])
    ref = orc.qmatmul_f64(x, wq[rows], s[rows], b[rows], 64, bits) + orc.bf16_to_f32(bias[rows]).astype(np.float64)
    assert rel_err(y[:, rows], ref) <= TIGHT
    monkeypatch.delenv("MLXQ_QMV_STREAM64", raising=False)
    mlxq.reload_overrides()


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("m", [40, 100])
def test_stream64_down_like_forced(torch_gpu, monkeypatch, bits, m):
    """The 64-row streaming form on a down-like matrix (four K splits through
    the workspace, then the reduction launch), forced with
    MLXQ_QMV_STREAM64=1 (not the default there); against the oracle."""
    import mlxq
    monkeypatch.setenv("MLXQ_QMV_STREAM64", "1")
    mlxq.reload_overrides()
    k, n = 14336, 4096
    assert mlxq.workspace_size(m, n, k, 64, bits) == 4 * m * n * 4
    wq, s, b = make_layer(0x6410 + bits, n, k, 64, bits)
    x = bf16_acts(0x6411 + m, m, k)
    y = run(x, wq, s, b, 64, bits)
    rows = np.random.default_rng(0x6412).choice(n, 128, replace=False)
    assert rel_err(y[:, rows], orc.qmatmul_f64(x, wq[rows], s[rows], b[rows], 64, bits)) <= TIGHT
    monkeypatch.delenv("MLXQ_QMV_STREAM64")
    mlxq.reload_overrides()

