"""Quantized matmul (qmv decode GEMV, qmm MFMA GEMM) on the GPU vs the f64 CPU
oracle over the same bf16 inputs.  Bar: max|y - ref| / max|ref| <= 1e-2
(bf16 output, f32 accumulation); in practice the error is bf16 output
rounding, so a tighter 4e-3 is asserted too."""
import numpy as np
import pytest

import mlxq
import oracle as orc
from helpers import bf16_acts, bf16_weights, dev, host, rel_err, rel_err_elem

pytestmark = pytest.mark.gpu
TOL = 1e-2
TIGHT = 4e-3     # what the kernels actually achieve (bf16 output rounding ~2e-3)
ELEM_TOL = 2e-2  # element-wise |y - ref| / |ref| over outputs >= 1% of the largest
LLAMA = {"q_o": (4096, 4096), "k_v": (4096, 1024), "gate_up": (4096, 14336), "down": (14336, 4096)}


def make_layer(seed, n, k, gs=64, bits=4, outlier_cols=0):
    w = bf16_weights(seed, n, k)
    if outlier_cols:
        # scale a few input channels x20 to stress per-group scales (config 3)
        cols = np.random.default_rng(seed).choice(k, outlier_cols, replace=False)
        wf = orc.bf16_to_f32(w)
        wf[:, cols] *= 20
        w = orc.f32_to_bf16(wf)
    wq, s, b = orc.affine_quantize(w, gs, bits, orc.BF16)
    return wq, s, b


def run(x, wq, s, b, gs, bits, algo=mlxq.ALGO_AUTO, bias=None):
    import torch

    y = mlxq.qmatmul(dev(x, bf16=True), dev(wq), dev(s, bf16=True), dev(b, bf16=True), gs, bits,
                     bias=None if bias is None else dev(bias, bf16=True), algo=algo)
    torch.cuda.synchronize()
    return orc.bf16_to_f32(host(y))


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("gs", [32, 64, 128])
@pytest.mark.parametrize("m", [1, 3, 16, 17, 32])
def test_qmv_small(torch_gpu, bits, gs, m):
    n, k = 200, 1024  # N not a multiple of 64: masked rows
    wq, s, b = make_layer(10 + bits + gs, n, k, gs, bits)
    x = bf16_acts(20 + m, m, k)
    ref = orc.qmatmul_f64(x, wq, s, b, gs, bits)
    y = run(x, wq, s, b, gs, bits, mlxq.ALGO_QMV)
    assert rel_err(y, ref) <= TIGHT


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("name", list(LLAMA))
@pytest.mark.parametrize("m", [1, 3, 4, 16, 32])
def test_qmv_llama_shapes(torch_gpu, bits, name, m):
    k, n = LLAMA[name]
    wq, s, b = make_layer(0x5EED0000 + k + n + bits, n, k, 64, bits)
    x = bf16_acts(0x5EED1000 + m, m, k)
    ref = orc.qmatmul_f64(x, wq, s, b, 64, bits)
    y = run(x, wq, s, b, 64, bits)
    err = rel_err(y, ref)
    # element-wise relative error beside the max-normalised bar, over the
    # outputs at least 1% of the largest (bf16 output rounding is 2^-9)
    elem = rel_err_elem(y, ref, floor=1e-2)
    print(f"Q{bits} {name} M={m}: rel_err {err:.2e}, elementwise {elem:.2e}")
    assert err <= TIGHT, err
    assert err <= TOL
    assert elem <= ELEM_TOL, elem


def test_qmv_config1_single_decode(torch_gpu):
    """Config 1: W 4096x4096 from N(0,0.02), Q4 g64, x 1x4096 N(0,1)."""
    wq, s, b = make_layer(0x5EED0001, 4096, 4096, 64, 4)
    x = bf16_acts(0x5EED0002, 1, 4096)
    ref = orc.qmatmul_f64(x, wq, s, b, 64, 4)
    y = run(x, wq, s, b, 64, 4)
    assert rel_err(y, ref) <= TIGHT
    assert rel_err_elem(y, ref, floor=1e-2) <= ELEM_TOL


def test_qmv_repeat_reuses_workspace(torch_gpu):
    """Back-to-back calls sharing the split-K scratch agree bit-for-bit."""
    wq, s, b = make_layer(5, 4096, 4096, 64, 4)
    x = bf16_acts(6, 4, 4096)
    y1 = run(x, wq, s, b, 64, 4)
    y2 = run(x, wq, s, b, 64, 4)
    y3 = run(x[:1], wq, s, b, 64, 4)
    assert np.array_equal(y1, y2)
    assert np.array_equal(y3[0], y1[0]) or rel_err(y3, orc.qmatmul_f64(x[:1], wq, s, b, 64, 4)) <= TIGHT


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("gs", [32, 64, 128])
@pytest.mark.parametrize("m", [16, 300])
def test_qmm_small(torch_gpu, bits, gs, m):
    n, k = 200, 1024
    wq, s, b = make_layer(50 + bits + gs, n, k, gs, bits)
    x = bf16_acts(60 + m, m, k)
    ref = orc.qmatmul_f64(x, wq, s, b, gs, bits)
    y = run(x, wq, s, b, gs, bits, mlxq.ALGO_QMM)
    assert rel_err(y, ref) <= TIGHT


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("gs", [32, 64, 128])
@pytest.mark.parametrize("splits", [2, 8])
@pytest.mark.parametrize("n", [200, 202])
def test_qmm_split_k(torch_gpu, monkeypatch, bits, gs, splits, n):
    """qmm with K split across workgroups (f32 partials in the workspace,
    summed in slice order by the reduce kernel): the 4-wide reduce (N % 4 ==
    0) and the scalar one, a bias vector, M not a multiple of the tile."""
    monkeypatch.setenv("MLXQ_QMM_SPLIT", str(splits))
    monkeypatch.setenv("MLXQ_QMM_FUSED", "1")
    # slices of whole 512-K periods and 8-group scale batches
    m, k = 300, 4096 if splits * max(512, 8 * gs) <= 4096 else 8192
    assert mlxq.workspace_size(m, n, k, gs, bits) == splits * m * n * 4
    wq, s, b = make_layer(90 + bits + gs + n, n, k, gs, bits)
    x = bf16_acts(91 + splits, m, k)
    bias = orc.f32_to_bf16(orc.normal(92, n, 0, 1))
    ref = orc.qmatmul_f64(x, wq, s, b, gs, bits) + orc.bf16_to_f32(bias)[None, :]
    # the bf16 rounding of each dequantized weight adds noise growing as sqrt(K)
    assert rel_err(run(x, wq, s, b, gs, bits, mlxq.ALGO_QMM, bias=bias), ref) <= TIGHT * (k / 4096) ** 0.5


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("gs", [32, 64, 128])
@pytest.mark.parametrize("cfg", [82, 42])
@pytest.mark.parametrize("n", [448, 300])
def test_qmm_tile_configs(torch_gpu, monkeypatch, bits, gs, cfg, n):
    """Both qmm workgroup tiles (256 and 128 activation rows, four waves
    along N) with a bias, M and N not multiples of the tile (N = 300: the
    element-wise store tail), K = 2048 (four unrolled periods)."""
    monkeypatch.setenv("MLXQ_QMM_CFG", str(cfg))
    monkeypatch.setenv("MLXQ_QMM_SPLIT", "1")
    m, k = 300, 2048
    wq, s, b = make_layer(95 + bits + n + gs, n, k, gs, bits)
    x = bf16_acts(96 + cfg, m, k)
    bias = orc.f32_to_bf16(orc.normal(97, n, 0, 1))
    ref = orc.qmatmul_f64(x, wq, s, b, gs, bits) + orc.bf16_to_f32(bias)[None, :]
    assert rel_err(run(x, wq, s, b, gs, bits, mlxq.ALGO_QMM, bias=bias), ref) <= TIGHT


def test_bias_vector(torch_gpu):
    n, k = 192, 256
    wq, s, b = make_layer(70, n, k)
    x = bf16_acts(71, 5, k)
    bias = orc.f32_to_bf16(orc.normal(72, n, 0, 1))
    ref = orc.qmatmul_f64(x, wq, s, b) + orc.bf16_to_f32(bias)[None, :]
    for algo in (mlxq.ALGO_QMV, mlxq.ALGO_QMM):
        assert rel_err(run(x, wq, s, b, 64, 4, algo, bias=bias), ref) <= TIGHT


@pytest.mark.parametrize("algo", ["auto", "qmm"])
@pytest.mark.parametrize("name", ["gate_up", "down"])
def test_qmm_config3_prefill(torch_gpu, name, algo):
    """Config 3: M=2048, Q4 g64, 0.1% outlier input channels x20, on the
    default route and forced onto the hand-written qmm kernel (256-row tiles
    for gate/up, 128-row tiles for down; 64 and 224 K steps); the oracle
    checks a seeded sample of 64 rows (rows are independent)."""
    k, n = LLAMA[name]
    wq, s, b = make_layer(0x5EED0300 + k, n, k, 64, 4, outlier_cols=(k + 999) // 1000)
    x = bf16_acts(0x5EED0301, 2048, k)
    y = run(x, wq, s, b, 64, 4, mlxq.ALGO_QMM if algo == "qmm" else mlxq.ALGO_AUTO)
    rows = np.sort(np.random.default_rng(3).choice(2048, 64, replace=False))
    ref = orc.qmatmul_f64(x[rows], wq, s, b, 64, 4)
    err = rel_err(y[rows], ref)
    elem = rel_err_elem(y[rows], ref, floor=1e-2)
    # reported, not asserted: the prefill path rounds each dequantized
    # weight to bf16 (the values MLX's qmm stages), and with the x20 outlier
    # channels the largest outputs are far above the typical one, so the
    # outputs near 1% of the largest carry relative errors of several %
    print(f"prefill {name} ({algo}): rel_err {err:.2e}, elementwise {elem:.2e}")
    assert err <= TIGHT, err


def test_qmv_and_qmm_agree(torch_gpu):
    wq, s, b = make_layer(80, 1024, 2048)
    x = bf16_acts(81, 32, 2048)
    ref = orc.qmatmul_f64(x, wq, s, b)
    assert rel_err(run(x, wq, s, b, 64, 4, mlxq.ALGO_QMV), ref) <= TIGHT
    assert rel_err(run(x, wq, s, b, 64, 4, mlxq.ALGO_QMM), ref) <= TIGHT


def test_reference_matmul_q8(torch_gpu):
    import json
    from pathlib import Path

    a = json.loads((Path(__file__).resolve().parent / "golden" / "gguf_kat.json").read_text())["affine"]["matmul_q8"]
    w = np.float32(a["w"]).reshape(a["shape"])
    x = np.float32(a["x"]).reshape(1, 64)
    wq, s, b = orc.affine_quantize(orc.f32_to_bf16(w), 64, 8, orc.BF16)
    y = run(orc.f32_to_bf16(x), wq, s, b, 64, 8)
    dense = x.astype(np.float64) @ w.astype(np.float64).T
    assert np.max(np.abs(y - dense)) < a["max_abs_err"]  # quant.rs:111-125


def test_graph_replay_matches_eager(torch_gpu):
    """Capture qmv (split-K tickets) + qmm in one HIP graph; replay it several
    times with eager work and synchronizations in between; every replay must
    equal the eager result bit-for-bit."""
    torch = torch_gpu
    wq, s, b = make_layer(90, 4096, 4096)
    x1 = dev(bf16_acts(91, 4, 4096), bf16=True)
    x2 = dev(bf16_acts(92, 64, 4096), bf16=True)
    d = [dev(t) for t in (wq,)] + [dev(t, bf16=True) for t in (s, b)]
    c1 = mlxq.bind_qmatmul(x1, *d, 64, 4)
    c2 = mlxq.bind_qmatmul(x2, *d, 64, 4)
    e1, e2 = c1().clone(), c2().clone()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        c1()
        c2()
    for i in range(4):
        c1.out.zero_()
        c2.out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(c1.out, e1) and torch.equal(c2.out, e2), f"replay {i}"
        mlxq.qmatmul(x1, *d, 64, 4)  # eager work between replays
        torch.cuda.synchronize()


def test_workspace_shared_across_shapes(torch_gpu):
    """Alternate shapes with different tile counts and split counts on one
    workspace: tickets stay valid (regression: partials once overlapped tickets)."""
    shapes = [(4096, 4096), (4096, 14336), (4096, 1024), (14336, 4096), (4096, 14336)]
    for i, (k, n) in enumerate(shapes):
        wq, s, b = make_layer(100 + i, n, k)
        x = bf16_acts(200 + i, 8, k)
        assert rel_err(run(x, wq, s, b, 64, 4), orc.qmatmul_f64(x, wq, s, b)) <= TIGHT


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("k", [192, 320])
def test_qmv_odd_k_uses_narrow_loader(torch_gpu, bits, k):
    """K*bits/8 not a multiple of 64 bytes: the 8-byte group loader path."""
    wq, s, b = make_layer(300 + k + bits, 130, k, 64, bits)
    x = bf16_acts(301 + k, 3, k)
    assert rel_err(run(x, wq, s, b, 64, bits, mlxq.ALGO_QMV), orc.qmatmul_f64(x, wq, s, b, 64, bits)) <= TIGHT


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("m", [1, 32])
def test_qmv_forced_narrow_loader(torch_gpu, monkeypatch, bits, m):
    monkeypatch.setenv("MLXQ_QMV_NARROW", "1")
    k, n = LLAMA["down"]
    wq, s, b = make_layer(400 + bits, n, k, 64, bits)
    x = bf16_acts(401 + m, m, k)
    assert rel_err(run(x, wq, s, b, 64, bits), orc.qmatmul_f64(x, wq, s, b, 64, bits)) <= TIGHT


@pytest.mark.parametrize("sub", ["1", "2", "4"])
def test_qmv_every_tile_height(torch_gpu, monkeypatch, sub):
    monkeypatch.setenv("MLXQ_QMV_SUB", sub)
    wq, s, b = make_layer(500, 1000, 2048, 64, 4)
    x = bf16_acts(501, 20, 2048)
    assert rel_err(run(x, wq, s, b, 64, 4), orc.qmatmul_f64(x, wq, s, b, 64, 4)) <= TIGHT


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("gs", [32, 64, 128])
@pytest.mark.parametrize("m", [1, 2, 3, 4])
@pytest.mark.parametrize("k", [384, 1152])
def test_qmv_dot_decode_rows(torch_gpu, bits, gs, m, k):
    """M <= 4 runs on the vector-ALU kernel; K=384/1152 give ragged chunk tails."""
    if k % gs:
        pytest.skip("K not a multiple of the group")
    wq, s, b = make_layer(600 + bits + gs + k, 333, k, gs, bits)
    x = bf16_acts(601 + m + k, m, k)
    assert rel_err(run(x, wq, s, b, gs, bits), orc.qmatmul_f64(x, wq, s, b, gs, bits)) <= TIGHT


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("m", [1, 4])
def test_qmv_mfma_path_for_decode_rows(torch_gpu, monkeypatch, bits, m):
    monkeypatch.setenv("MLXQ_QMV_MFMA", "1")
    k, n = LLAMA["q_o"]
    wq, s, b = make_layer(700 + bits, n, k, 64, bits)
    x = bf16_acts(701 + m, m, k)
    assert rel_err(run(x, wq, s, b, 64, bits), orc.qmatmul_f64(x, wq, s, b, 64, bits)) <= TIGHT


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("cfg", ["1,4", "1,8", "2,4", "2,8"])
@pytest.mark.parametrize("k", [512, 1024])
def test_qmv_dot_short_rows_every_config(torch_gpu, monkeypatch, bits, cfg, k):
    """Short rows leave most waves of a workgroup with an empty chunk range:
    they must fetch nothing (every load stays inside the row), for each
    rows-per-workgroup / waves-per-workgroup configuration."""
    monkeypatch.setenv("MLXQ_QMV_DOT", cfg)
    wq, s, b = make_layer(800 + bits + k, 1000, k, 64, bits)
    x = bf16_acts(801 + k, 2, k)
    assert rel_err(run(x, wq, s, b, 64, bits), orc.qmatmul_f64(x, wq, s, b, 64, bits)) <= TIGHT


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("m", [2, 3, 4])
@pytest.mark.parametrize("kernel", ["MLXQ_QMV_DOT_ALL", "MLXQ_QMV_MFMA"])
def test_decode_kernels_forced(torch_gpu, monkeypatch, bits, m, kernel):
    """M = 2..4 on both decode kernels (the dispatcher picks one per shape)."""
    monkeypatch.setenv(kernel, "1")
    n, k = 320, 2048
    wq, s, b = make_layer(30 + bits + m, n, k, 64, bits)
    x = bf16_acts(31 + m, m, k)
    assert rel_err(run(x, wq, s, b, 64, bits), orc.qmatmul_f64(x, wq, s, b, 64, bits)) <= TIGHT


ROW_K = {4: [2048, 4096, 8192, 14336], 8: [1024, 2048, 4096, 7168, 8192, 14336, 16384]}


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("gs", [32, 64, 128])
@pytest.mark.parametrize("geom", ["auto", "1,4", "2,4", "4,4", "1,8", "2,8", "1,16"])
def test_qmv_row_batch1(torch_gpu, monkeypatch, bits, gs, geom):
    """Batch-1 whole-row kernel (qmv_row.hip) at every row length it is
    built for (1..16 KB of codes), every forced (rows per wave, waves per
    workgroup), group sizes 32/64/128, N not a multiple of the rows per
    workgroup (203) and smaller than one workgroup (8), with a bias vector."""
    if geom != "auto":
        r, w = geom.split(",")
        monkeypatch.setenv("MLXQ_QMV_ROW_R", r)
        monkeypatch.setenv("MLXQ_QMV_ROW_W", w)
    for k in ROW_K[bits]:
        for n in (203, 8):
            wq, s, b = make_layer(0x60 + bits + gs + k + n, n, k, gs, bits)
            x = bf16_acts(0x61 + k, 1, k)
            bias = orc.f32_to_bf16(np.linspace(-1, 1, n, dtype=np.float32))
            ref = orc.qmatmul_f64(x, wq, s, b, gs, bits) + orc.bf16_to_f32(bias).astype(np.float64)
            y = run(x, wq, s, b, gs, bits, bias=bias)
            assert rel_err(y, ref) <= TIGHT, (k, n)


def test_qmv_row_skipped_kernel_agrees(torch_gpu, monkeypatch):
    """MLXQ_QMV_NO_ROW=1 (the previous batch-1 kernel) and the row kernel
    agree to bf16 rounding on a Llama shape."""
    wq, s, b = make_layer(0x62, 4096, 4096, 64, 4)
    x = bf16_acts(0x63, 1, 4096)
    a = run(x, wq, s, b, 64, 4)
    monkeypatch.setenv("MLXQ_QMV_NO_ROW", "1")
    c = run(x, wq, s, b, 64, 4)
    assert rel_err(a, c.astype(np.float64)) <= TIGHT


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("m", [2, 3, 4])
@pytest.mark.parametrize("gs", [32, 64, 128])
def test_qmv_row_several_rows(torch_gpu, monkeypatch, bits, m, gs):
    """The whole-row kernel with 2..4 activation rows (K <= 4096), forced on
    a tall ragged matrix and taken by default on a short one, with a bias."""
    monkeypatch.setenv("MLXQ_QMV_ROW_ALL", "1")
    for n, k in ((203, 4096), (1024, 2048), (8, 1024 * 8 // bits)):
        wq, s, b = make_layer(0x70 + bits + m + gs + n, n, k, gs, bits)
        x = bf16_acts(0x71 + m, m, k)
        bias = orc.f32_to_bf16(np.linspace(-1, 1, n, dtype=np.float32))
        ref = orc.qmatmul_f64(x, wq, s, b, gs, bits) + orc.bf16_to_f32(bias).astype(np.float64)[None, :]
        assert rel_err(run(x, wq, s, b, gs, bits, bias=bias), ref) <= TIGHT, (n, k)


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("name,m", [("q_o", 128), ("q_o", 512), ("k_v", 256), ("down", 128), ("down", 256)])
def test_qmm_small_grids_split_on_narrow_tiles(torch_gpu, bits, name, m):
    """The fused prefill kernel at grids that no split of 256 x 256 tiles
    fills: 128 x 128 tiles with K split (partials in the workspace); sampled
    output columns against the oracle."""
    k, n = LLAMA[name]
    assert mlxq.workspace_size(m, n, k, 64, bits) > 0 or name == "down"
    wq, s, b = make_layer(0x600 + m + bits, n, k, 64, bits)
    x = bf16_acts(0x601 + m, m, k)
    y = run(x, wq, s, b, 64, bits, mlxq.ALGO_QMM)
    cols = np.sort(np.random.default_rng(m).choice(n, 128, replace=False))
    assert rel_err(y[:, cols], orc.qmatmul_f64(x, wq[cols], s[cols], b[cols], 64, bits)) <= TIGHT


def test_route_query_names_the_kernels(torch_gpu):
    """mlxq_qmatmul_route runs the library's own dispatch with launches
    suppressed: the families it names are the route each call takes."""
    r = mlxq.qmatmul_route
    assert r(1, 4096, 4096, 64, 4).startswith("row::qmv_row_kernel<4,")           # decode GEMV
    assert r(2048, 4096, 14336, 64, 4) == "qmm_kernel<4, 64, 4, 2>"              # down-like prefill
    gate = r(2048, 14336, 4096, 64, 4)                                           # gate/up-like, M >= 1024
    assert gate.startswith("dequant_bf16_kernel<4>") and gate.endswith(" + hipBLASLt GEMM"), gate
    assert r(2048, 14336, 4096, 64, 4, algo=mlxq.ALGO_QMM) == "qmm_kernel<4, 64, 8, 2>"
    assert r(2048, 14336, 4096, 64, 4, noalloc=True) == "qmm_kernel<4, 64, 8, 2>"  # never the library
    assert r(48, 14336, 4096, 64, 4, noalloc=True) == r(48, 14336, 4096, 64, 4)  # 32-row decode chunks
    assert r(96, 14336, 4096, 64, 4, noalloc=True) == r(96, 14336, 4096, 64, 4)  # 64-row streaming form
    assert "split_reduce" in r(512, 4096, 4096, 64, 4)                           # qmm with K split
    assert r(512, 4096, 4096, 64, 4, workspace_bytes=0) == "qmm_kernel<4, 64, 4, 2>"  # no workspace: unsplit
