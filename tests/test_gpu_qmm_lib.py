"""Prefill routes other than the fused kernel: dequantize + the library's
bf16 GEMM (qmm_lib.hip: the weight dequantized into the workspace, then
hipBLASLt), forced onto small shapes with MLXQ_QMM_LIB=1 and checked against
the f64 CPU oracle and against the fused prefill kernel (the same
dequantized bf16 values, so the two differ only in summation order); and
short calls run as 32-row batched-decode chunks.  Bar: max|y - ref| /
max|ref| <= 4e-3 (bf16 output rounding)."""
import numpy as np
import pytest

import mlxq
import oracle as orc
from helpers import bf16_acts, dev, host, rel_err
from test_gpu_qmatmul import LLAMA, TIGHT, make_layer, run

pytestmark = pytest.mark.gpu


@pytest.fixture
def lib_all(monkeypatch):
    monkeypatch.setenv("MLXQ_QMM_LIB", "1")
    monkeypatch.delenv("MLXQ_QMM_FUSED", raising=False)
    mlxq.reload_overrides()
    yield monkeypatch
    monkeypatch.delenv("MLXQ_QMM_LIB", raising=False)
    mlxq.reload_overrides()


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("gs", [32, 64, 128])
@pytest.mark.parametrize("m,n,k", [(33, 200, 1024), (100, 640, 2048), (512, 96, 4096)])
def test_lib_against_oracle(torch_gpu, lib_all, bits, gs, m, n, k):
    print(f"qmm_lib bits={bits} gs={gs} m={m} n={n} k={k}", flush=True)
    wq, s, b = make_layer(300 + bits + gs, n, k, gs, bits)
    x = bf16_acts(301 + m, m, k)
    assert rel_err(run(x, wq, s, b, gs, bits), orc.qmatmul_f64(x, wq, s, b, gs, bits)) <= TIGHT


@pytest.mark.parametrize("bits", [4, 8])
def test_lib_bias_and_outliers(torch_gpu, lib_all, bits):
    n, k, m = 640, 4096, 300
    wq, s, b = make_layer(310 + bits, n, k, 64, bits, outlier_cols=8)
    x = bf16_acts(311, m, k)
    bias = orc.f32_to_bf16(np.random.default_rng(312).normal(0, 1, n).astype(np.float32))
    ref = orc.qmatmul_f64(x, wq, s, b, 64, bits) + orc.bf16_to_f32(bias)[None, :].astype(np.float64)
    assert rel_err(run(x, wq, s, b, 64, bits, bias=bias), ref) <= TIGHT
    # the same call without the bias (a second plan of the same shape)
    assert rel_err(run(x, wq, s, b, 64, bits), orc.qmatmul_f64(x, wq, s, b, 64, bits)) <= TIGHT


@pytest.mark.parametrize("bits", [4, 8])
def test_lib_matches_fused_kernel(torch_gpu, lib_all, bits):
    """Same dequantized values as the fused kernel: the outputs agree to
    bf16 output rounding of the two summation orders (one bf16 ulp of an
    output apart at most: <= 4e-3 of the largest)."""
    n, k, m = 1024, 4096, 256
    wq, s, b = make_layer(320 + bits, n, k, 64, bits)
    x = bf16_acts(321, m, k)
    lib = run(x, wq, s, b, 64, bits, mlxq.ALGO_QMM_LIB)
    fused = run(x, wq, s, b, 64, bits, mlxq.ALGO_QMM)
    assert np.max(np.abs(lib - fused)) / np.max(np.abs(fused)) <= TIGHT


@pytest.mark.parametrize("name,m", [("gate_up", 1024), ("q_o", 1024), ("gate_up", 2048), ("down", 4096)])
def test_lib_default_llama(torch_gpu, monkeypatch, name, m):
    """The default dispatch at shapes where it takes the library GEMM;
    seeded sample of 64 output columns (weight rows) against the oracle."""
    for v in ("MLXQ_QMM_LIB", "MLXQ_QMM_FUSED"):
        monkeypatch.delenv(v, raising=False)
    mlxq.reload_overrides()
    k, n = LLAMA[name]
    need = mlxq.workspace_size(m, n, k, 64, 4)
    assert need >= n * k * 2  # the dequantized weight lives in the workspace
    wq, s, b = make_layer(330, n, k, 64, 4)
    x = bf16_acts(331, m, k)
    y = run(x, wq, s, b, 64, 4)
    cols = np.sort(np.random.default_rng(332).choice(n, 64, replace=False))
    assert rel_err(y[:, cols], orc.qmatmul_f64(x, wq[cols], s[cols], b[cols], 64, 4)) <= TIGHT


def test_lib_small_workspace_takes_fused_kernel(torch_gpu, lib_all):
    """A workspace smaller than the dequantized weight: the AUTO call runs
    the fused kernel instead and still matches; the explicit algorithm
    reports the workspace error."""
    torch = torch_gpu
    n, k, m = 512, 2048, 64
    wq, s, b = make_layer(340, n, k, 64, 4)
    x = bf16_acts(341, m, k)
    xd, wd, sd, bd = dev(x, bf16=True), dev(wq), dev(s, bf16=True), dev(b, bf16=True)
    ws = torch.zeros(1 << 20, dtype=torch.uint8, device="cuda")
    y = torch.empty((m, n), dtype=torch.bfloat16, device="cuda")
    st = torch.cuda.current_stream().cuda_stream
    args = (xd.data_ptr(), m, wd.data_ptr(), sd.data_ptr(), bd.data_ptr(), None, n, k, 64, 4, y.data_ptr(),
            ws.data_ptr(), ws.numel())
    assert mlxq.lib().mlxq_qmatmul_algo(*args, mlxq.ALGO_AUTO, st) == 0
    torch.cuda.synchronize()
    assert rel_err(orc.bf16_to_f32(host(y)), orc.qmatmul_f64(x, wq, s, b, 64, 4)) <= TIGHT
    assert mlxq.lib().mlxq_qmatmul_algo(*args, mlxq.ALGO_QMM_LIB, st) == mlxq.ERR_WORKSPACE


def test_lib_graph_replay_bit_exact(torch_gpu, lib_all):
    """HIP-graph replays of dequantize + GEMM equal the eager call bit for
    bit, with eager work on the same workspace between replays."""
    torch = torch_gpu
    wq, s, b = make_layer(350, 1024, 4096, 64, 4)
    x = dev(bf16_acts(351, 128, 4096), bf16=True)
    d = [dev(wq), dev(s, bf16=True), dev(b, bf16=True)]
    call = mlxq.bind_qmatmul(x, *d, 64, 4)
    eager = call().clone()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        call()
    other = make_layer(352, 768, 4096, 64, 8)
    od = [dev(other[0]), dev(other[1], bf16=True), dev(other[2], bf16=True)]
    for i in range(3):
        call.out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(call.out, eager), i
        mlxq.qmatmul(x, *od, 64, 8)  # another weight through the same workspace
        torch.cuda.synchronize()


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("m,n,k", [(33, 200, 1024), (64, 640, 4096), (48, 256, 8192), (64, 96, 2048)])
def test_prefill_short_calls_in_decode_chunks(torch_gpu, monkeypatch, bits, m, n, k):
    """33..64 rows run as 32-row calls of the batched-decode kernels under
    the default dispatch (with a bias: each chunk adds it)."""
    for v in ("MLXQ_QMM_LIB", "MLXQ_QMM_FUSED"):
        monkeypatch.delenv(v, raising=False)
    wq, s, b = make_layer(360 + bits, n, k, 64, bits)
    x = bf16_acts(361 + m, m, k)
    bias = orc.f32_to_bf16(np.random.default_rng(362).normal(0, 1, n).astype(np.float32))
    ref = orc.qmatmul_f64(x, wq, s, b, 64, bits) + orc.bf16_to_f32(bias)[None, :].astype(np.float64)
    assert rel_err(run(x, wq, s, b, 64, bits, bias=bias), ref) <= TIGHT
