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


@pytest.mark.parametrize("rows,dim", [(1, 4096), (16, 4096), (3, 14336), (2, 8)])
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
