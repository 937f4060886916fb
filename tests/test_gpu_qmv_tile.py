"""Batched-decode GEMV with activations shared through LDS and K split across
workgroups (qmv_tile.hip), forced onto shapes it would not be chosen for,
against the f64 CPU oracle.  Bar: max|y - ref| / max|ref| <= 4e-3 (bf16
output rounding).  Covers every (waves, slice) configuration, padded rows and
activation rows, the split-K reduction kernel, workspace reuse across shapes,
a workspace too small for any split (falls back to the block kernel) and
HIP-graph replay."""
import numpy as np
import pytest

import mlxq
import oracle as orc
from helpers import bf16_acts, dev, host, rel_err
from test_gpu_qmatmul import TIGHT, make_layer, run

pytestmark = pytest.mark.gpu


@pytest.fixture
def tile_all(monkeypatch):
    monkeypatch.setenv("MLXQ_QMV_TILE_ALL", "1")
    monkeypatch.delenv("MLXQ_QMV_TILE", raising=False)
    return monkeypatch


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("cfg", ["4,4", "4,8", "8,4", "8,8", "8,16"])
@pytest.mark.parametrize("m", [5, 16, 17, 32])
def test_tile_configs(torch_gpu, tile_all, bits, cfg, m):
    tile_all.setenv("MLXQ_QMV_TILE", cfg)
    n, k = 200, 2048  # N not a multiple of 64 (masked rows); K gives 1..8 splits
    wq, s, b = make_layer(40 + bits, n, k, 64, bits)
    x = bf16_acts(50 + m, m, k)
    ref = orc.qmatmul_f64(x, wq, s, b, 64, bits)
    assert rel_err(run(x, wq, s, b, 64, bits), ref) <= TIGHT


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("cfg", ["4,4", "8,8,2", "8,4,4"])
@pytest.mark.parametrize("m", [17, 32])
def test_tile_m_blocks(torch_gpu, tile_all, bits, cfg, m):
    """Activation rows in M blocks of 16 (one workgroup per block and row
    tile, over the same weight rows)."""
    tile_all.setenv("MLXQ_QMV_TILE", cfg)
    tile_all.setenv("MLXQ_QMV_TILE_MB", "1")
    n, k = 200, 2048
    wq, s, b = make_layer(42 + bits, n, k, 64, bits)
    x = bf16_acts(52 + m, m, k)
    assert rel_err(run(x, wq, s, b, 64, bits), orc.qmatmul_f64(x, wq, s, b, 64, bits)) <= TIGHT


@pytest.mark.parametrize("bits,cfg", [(4, "8,4,8"), (8, "8,4,8"), (8, "8,8,8")])
@pytest.mark.parametrize("k", [4096, 8192])
@pytest.mark.parametrize("m", [5, 16, 17, 32])
def test_tile_eight_k_parts(torch_gpu, tile_all, bits, cfg, k, m):
    """Eight K parts of one 16-row group: a 4096-k slice (the whole K, or two
    splits at K = 8192; 2048 for Q8 with 4 chunks per wave), M blocks of 16
    above 16 rows."""
    tile_all.setenv("MLXQ_QMV_TILE", cfg)
    n = 200
    wq, s, b = make_layer(44 + bits, n, k, 64, bits)
    x = bf16_acts(54 + m, m, k)
    assert rel_err(run(x, wq, s, b, 64, bits), orc.qmatmul_f64(x, wq, s, b, 64, bits)) <= TIGHT


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("proj,m", [("k", 6), ("k", 16), ("k", 32), ("q", 8), ("q", 12), ("q", 16), ("q", 32)])
def test_tile_default_short(torch_gpu, monkeypatch, bits, proj, m):
    """The short Llama-3-8B projections under the default dispatch (the
    whole-K eight-part form where it fits one round of CUs), sampled rows
    against the oracle."""
    for v in ("MLXQ_QMV_TILE", "MLXQ_QMV_TILE_ALL", "MLXQ_QMV_TILE_MB", "MLXQ_QMV_TILE_STREAM"):
        monkeypatch.delenv(v, raising=False)
    n = {"k": 1024, "q": 4096}[proj]
    k = 4096
    wq, s, b = make_layer(46 + bits, n, k, 64, bits)
    x = bf16_acts(56 + m, m, k)
    y = run(x, wq, s, b, 64, bits)
    rows = np.random.default_rng(57).choice(n, 256, replace=False)
    assert rel_err(y[:, rows], orc.qmatmul_f64(x, wq[rows], s[rows], b[rows], 64, bits)) <= TIGHT


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("m", [8, 32])
def test_tile_bias_and_outliers(torch_gpu, tile_all, bits, m):
    n, k = 640, 4096
    wq, s, b = make_layer(60 + bits, n, k, 64, bits, outlier_cols=8)
    x = bf16_acts(61, m, k)
    bias = orc.f32_to_bf16(np.random.default_rng(62).normal(0, 1, n).astype(np.float32))
    ref = orc.qmatmul_f64(x, wq, s, b, 64, bits) + orc.bf16_to_f32(bias)[None, :].astype(np.float64)
    assert rel_err(run(x, wq, s, b, 64, bits, bias=bias), ref) <= TIGHT


def test_tile_deterministic_and_shared_workspace(torch_gpu, tile_all):
    """Partials are added in split order: repeated calls agree bit-for-bit,
    also with calls of other shapes (other tile and split counts) on the same
    workspace in between."""
    a = make_layer(70, 1024, 4096, 64, 4)
    bq = make_layer(71, 4096, 1024, 64, 8)
    xa = bf16_acts(72, 32, 4096)
    xb = bf16_acts(73, 16, 1024)
    ya = run(xa, *a, 64, 4)
    for i in range(3):
        yb = run(xb, *bq, 64, 8)
        assert np.array_equal(run(xa, *a, 64, 4), ya), i
    assert rel_err(ya, orc.qmatmul_f64(xa, *a, 64, 4)) <= TIGHT
    assert rel_err(yb, orc.qmatmul_f64(xb, *bq, 64, 8)) <= TIGHT


def test_tile_small_workspace_falls_back(torch_gpu, tile_all):
    """A workspace with room for no split: the call still succeeds (block
    kernel) and matches."""
    import torch

    n, k, m = 256, 4096, 16
    wq, s, b = make_layer(80, n, k, 64, 4)
    x = bf16_acts(81, m, k)
    ws = torch.zeros(4096, dtype=torch.uint8, device="cuda")
    y = torch.empty((m, n), dtype=torch.bfloat16, device="cuda")
    xd, wd, sd, bd = dev(x, bf16=True), dev(wq), dev(s, bf16=True), dev(b, bf16=True)
    rc = mlxq.lib().mlxq_qmatmul(xd.data_ptr(), m, wd.data_ptr(), sd.data_ptr(), bd.data_ptr(), None, n, k, 64, 4,
                                 y.data_ptr(), ws.data_ptr(), ws.numel(), torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert rc == 0
    assert rel_err(orc.bf16_to_f32(host(y)), orc.qmatmul_f64(x, wq, s, b, 64, 4)) <= TIGHT


def test_tile_graph_replay(torch_gpu, tile_all):
    """Captured split-K calls (partials kernel + reduction kernel) replay
    correctly with eager calls of another shape on the same workspace in
    between."""
    import torch

    wq, s, b = make_layer(90, 1024, 4096, 64, 4)
    d = [dev(wq), dev(s, bf16=True), dev(b, bf16=True)]
    x = dev(bf16_acts(91, 32, 4096), bf16=True)
    c = mlxq.bind_qmatmul(x, *d, 64, 4)
    e = c().clone()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        c()
    for i in range(4):
        c.out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(c.out, e), f"replay {i}"
        mlxq.qmatmul(x[:8], *d, 64, 4)
        torch.cuda.synchronize()


@pytest.mark.parametrize("m", [17, 32])
def test_tile_whole_k_32_row_workgroups_ragged(torch_gpu, monkeypatch, m):
    """Q4 q/o-like matrices past one round of 16-row tiles take 32 rows per
    workgroup (two row groups x four K parts) under the default dispatch;
    N = 4008 leaves the last workgroup 8 real rows.  Sampled rows (the last
    ones included) against the oracle, with a bias, and the 16-row form
    (MLXQ_QMV_TILE_FUSED_RG=1) agrees to the same bar."""
    for v in ("MLXQ_QMV_TILE", "MLXQ_QMV_TILE_ALL", "MLXQ_QMV_TILE_MB", "MLXQ_QMV_TILE_STREAM",
              "MLXQ_QMV_TILE_FUSED_RG"):
        monkeypatch.delenv(v, raising=False)
    mlxq.reload_overrides()
    n, k = 4008, 4096
    wq, s, b = make_layer(90 + m, n, k, 64, 4)
    x = bf16_acts(91 + m, m, k)
    bias = orc.f32_to_bf16(np.linspace(-1, 1, n, dtype=np.float32))
    rows = np.concatenate([np.random.default_rng(92).choice(n - 8, 120, replace=False), np.arange(n - 8, n)])
    ref = orc.qmatmul_f64(x, wq[rows], s[rows], b[rows], 64, 4) + orc.bf16_to_f32(bias[rows]).astype(np.float64)
    y = run(x, wq, s, b, 64, 4, bias=bias)
    assert rel_err(y[:, rows], ref) <= TIGHT
    monkeypatch.setenv("MLXQ_QMV_TILE_FUSED_RG", "1")
    mlxq.reload_overrides()
    y16 = run(x, wq, s, b, 64, 4, bias=bias)
    monkeypatch.delenv("MLXQ_QMV_TILE_FUSED_RG")
    mlxq.reload_overrides()
    assert rel_err(y16[:, rows], ref) <= TIGHT
