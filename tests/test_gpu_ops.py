"""Decode-chain bf16 ops on the GPU (libmlxq.so) against the CPU oracle.

add and repeat_kv are pure bf16 rounding / data movement: bit-exact.
rms_norm sums squares in f32 in a different order than the oracle's f64 sum,
and silu uses the device expf; either can move a value across a bf16 rounding
boundary, so those allow a one-ulp difference on a small fraction of elements.
"""
import numpy as np
import pytest

import mlxq
import oracle as orc
from helpers import dev, host

pytestmark = pytest.mark.gpu


def _ulp_close(got, want, frac=1e-3):
    g, w = orc.bf16_to_f32(got).astype(np.float64), orc.bf16_to_f32(want).astype(np.float64)
    diff = got != want
    assert diff.mean() <= frac, f"{diff.sum()} of {diff.size} differ"
    assert np.all(np.abs(g - w)[diff] <= np.abs(w)[diff] * 2 ** -7 + 1e-30)


@pytest.mark.parametrize("rows,dim", [(1, 4096), (16, 4096), (3, 14336), (2, 8), (2, 32768)])
def test_rms_norm(torch_gpu, rows, dim):
    x = orc.f32_to_bf16(orc.normal(100 + rows, rows * dim, 0.0, 2.0)).reshape(rows, dim)
    w = orc.f32_to_bf16(orc.normal(200 + dim, dim, 1.0, 0.2))
    want = orc.rms_norm(x, w, 1e-5)
    got = host(mlxq.rms_norm(dev(x, True), dev(w, True), 1e-5))
    _ulp_close(got, want)


@pytest.mark.parametrize("rows,dim", [(1, 4096), (16, 4096), (3, 14336), (2, 8)])
def test_add_rms_norm(torch_gpu, rows, dim):
    """One launch of the residual add and the next norm: the sum bit-exact
    with the oracle's add, the norm as rms_norm of that sum, and both
    bit-identical to the separate add and rms_norm kernels."""
    a = orc.f32_to_bf16(orc.normal(500 + rows, rows * dim, 0.0, 2.0)).reshape(rows, dim)
    b = orc.f32_to_bf16(orc.normal(501 + rows, rows * dim, 0.0, 1.0)).reshape(rows, dim)
    w = orc.f32_to_bf16(orc.normal(502 + dim, dim, 1.0, 0.2))
    s, y = mlxq.add_rms_norm(dev(a, True), dev(b, True), dev(w, True), 1e-5)
    want_s = orc.add(a, b)
    assert np.array_equal(host(s), want_s)
    _ulp_close(host(y), orc.rms_norm(want_s, w, 1e-5))
    s2 = mlxq.add(dev(a, True), dev(b, True))
    assert np.array_equal(host(y), host(mlxq.rms_norm(s2, dev(w, True), 1e-5)))


@pytest.mark.parametrize("alias", ["a", "b"])
@pytest.mark.parametrize("rows,dim", [(16, 4096), (3, 14336), (2, 8)])
def test_add_rms_norm_in_place(torch_gpu, alias, rows, dim):
    """sum written over one of its inputs (the residual update h = h + x):
    the same sum and norm as with a separate output."""
    a = orc.f32_to_bf16(orc.normal(510 + rows, rows * dim, 0.0, 2.0)).reshape(rows, dim)
    b = orc.f32_to_bf16(orc.normal(511 + rows, rows * dim, 0.0, 1.0)).reshape(rows, dim)
    w = orc.f32_to_bf16(orc.normal(512 + dim, dim, 1.0, 0.2))
    ad, bd = dev(a, True), dev(b, True)
    s, y = mlxq.add_rms_norm(ad, bd, dev(w, True), 1e-5, sum_out=ad if alias == "a" else bd)
    want_s = orc.add(a, b)
    assert np.array_equal(host(s), want_s)
    assert np.array_equal(host(ad if alias == "a" else bd), want_s)
    _ulp_close(host(y), orc.rms_norm(want_s, w, 1e-5))
    s2, y2 = mlxq.add_rms_norm(dev(a, True), dev(b, True), dev(w, True), 1e-5)
    assert np.array_equal(host(y), host(y2))


def test_silu_mul(torch_gpu):
    n = 16 * 14336
    g = orc.f32_to_bf16(orc.normal(300, n, 0.0, 3.0))
    u = orc.f32_to_bf16(orc.normal(301, n, 0.0, 1.0))
    _ulp_close(host(mlxq.silu_mul(dev(g, True), dev(u, True))), orc.silu_mul(g, u))


def test_add_bit_exact(torch_gpu):
    n = 16 * 4096 + 8
    a = orc.f32_to_bf16(orc.normal(400, n, 0.0, 3.0))
    b = orc.f32_to_bf16(orc.normal(401, n, 0.0, 1.0))
    assert np.array_equal(host(mlxq.add(dev(a, True), dev(b, True))), orc.add(a, b))


@pytest.mark.parametrize("rows,kvh,hd,groups", [(1, 8, 128, 4), (16, 8, 128, 4), (3, 2, 8, 1), (2, 4, 64, 3)])
def test_repeat_kv_bit_exact(torch_gpu, rows, kvh, hd, groups):
    x = orc.f32_to_bf16(orc.normal(500, rows * kvh * hd, 0.0, 1.0)).reshape(rows, kvh * hd)
    got = host(mlxq.repeat_kv(dev(x, True), kvh, hd, groups))
    assert np.array_equal(got, orc.repeat_kv(x, kvh, hd, groups))


def test_ops_reject_bad_shapes(torch_gpu):
    import torch

    x = torch.zeros(12, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(mlxq.MlxqError):
        mlxq.add(x, x)  # 12 is not a multiple of 8
    with pytest.raises(mlxq.MlxqError):
        mlxq.rms_norm(x.view(1, 12), x, 1e-5)


@pytest.mark.parametrize("bits,m,k,n,with_bias", [
    (4, 16, 14336, 4096, False),  # split K: the sum, add and norm in the second launch
    (4, 32, 14336, 4096, True),
    (8, 16, 14336, 4096, False),
    (8, 32, 14336, 4096, True),
    (4, 16, 14336, 1024, True),   # a split-K single-slice form, one piece of 8 per thread
    (4, 20, 16384, 8192, False),  # four pieces per thread
    (4, 24, 4096, 4096, False),   # one K slice: the projection, then add and norm
    (4, 2, 14336, 4096, False),   # batch 2: the unfused calls
    (8, 40, 2048, 1024, True),    # prefill rows
])
def test_qmatmul_add_rms_norm(torch_gpu, bits, m, k, n, with_bias):
    """Down projection + residual + next norm (llama.rs:729-733, :698) in one
    call: bit-identical to mlxq_qmatmul followed by mlxq_add_rms_norm, and
    the sum within twice the qmatmul bar of the f64 oracle."""
    from helpers import bf16_acts, rel_err
    from test_gpu_qmatmul import TIGHT, make_layer
    wq, s, b = make_layer(600 + bits + m, n, k, 64, bits)
    x = bf16_acts(601 + m, m, k)
    r = orc.f32_to_bf16(orc.normal(602 + m, m * n, 0.0, 1.0)).reshape(m, n)
    w = orc.f32_to_bf16(orc.normal(603, n, 1.0, 0.2))
    bias = orc.f32_to_bf16(orc.normal(604, n, 0.0, 1.0)) if with_bias else None
    xd, wd, sd, bd, rd, gw = dev(x, True), dev(wq), dev(s, True), dev(b, True), dev(r, True), dev(w, True)
    biasd = dev(bias, True) if with_bias else None
    print(f"qmatmul_add_rms_norm bits={bits} m={m} k={k} n={n} bias={with_bias}", flush=True)
    s_got, y_got = mlxq.qmatmul_add_rms_norm(xd, wd, sd, bd, rd, gw, 1e-5, 64, bits, bias=biasd)
    d = mlxq.qmatmul(xd, wd, sd, bd, 64, bits, bias=biasd)
    s_want, y_want = mlxq.add_rms_norm(rd, d, gw, 1e-5)
    assert np.array_equal(host(s_got), host(s_want))
    assert np.array_equal(host(y_got), host(y_want))
    ref = orc.qmatmul_f64(x, wq, s, b, 64, bits) + orc.bf16_to_f32(r).astype(np.float64)
    if with_bias:
        ref += orc.bf16_to_f32(bias)[None, :].astype(np.float64)
    # two bf16 roundings (the projection's output, then the sum): twice the bar
    assert rel_err(orc.bf16_to_f32(host(s_got)), ref) <= 2 * TIGHT


def test_qmatmul_add_rms_norm_graph_replay(torch_gpu):
    """Captured in a HIP graph (split-K sum, add and norm in the second
    launch), replayed three times with other eager work on the same
    workspace in between: every replay bit-identical to the eager call."""
    torch = torch_gpu
    from test_gpu_qmatmul import make_layer
    m, k, n = 16, 14336, 4096
    wq, s, b = make_layer(700, n, k, 64, 4)
    x = dev(orc.f32_to_bf16(orc.normal(701, m * k, 0.0, 1.0)).reshape(m, k), True)
    r = dev(orc.f32_to_bf16(orc.normal(702, m * n, 0.0, 1.0)).reshape(m, n), True)
    w = dev(orc.f32_to_bf16(orc.normal(703, n, 1.0, 0.2)), True)
    wd, sd, bd = dev(wq), dev(s, True), dev(b, True)
    s_out = torch.empty((m, n), dtype=torch.bfloat16, device="cuda")
    y_out = torch.empty((m, n), dtype=torch.bfloat16, device="cuda")
    mlxq.qmatmul_add_rms_norm(x, wd, sd, bd, r, w, 1e-5, 64, 4, sum_out=s_out, out=y_out)
    torch.cuda.synchronize()
    s_eager, y_eager = s_out.clone(), y_out.clone()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        mlxq.qmatmul_add_rms_norm(x, wd, sd, bd, r, w, 1e-5, 64, 4, sum_out=s_out, out=y_out)
    other = make_layer(704, 4096, 14336, 64, 8)
    od = (dev(other[0]), dev(other[1], True), dev(other[2], True))
    for i in range(3):
        s_out.zero_()
        y_out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(s_out, s_eager) and torch.equal(y_out, y_eager), i
        mlxq.qmatmul(x, *od, 64, 8)  # eager work through the same workspace
        torch.cuda.synchronize()
