"""Fused decode launches (mlxq_qmatmul_fused) against the CPU oracle's chain
of the same unfused ops: rms_norm / repeat_kv -> quantized projections ->
residual add / SwiGLU, same packed weights, same bf16 rounding points.
Bar: max|y - ref| / max|ref| <= 1e-2 (the qmatmul parity bar)."""
import numpy as np
import pytest

import mlxq
import oracle as orc
from helpers import bf16_acts, bf16_weights, dev, host, rel_err

pytestmark = pytest.mark.gpu
TOL = 1e-2


def qlayer(seed, n, k, gs, bits):
    wq, s, b = orc.affine_quantize(bf16_weights(seed, n, k), gs, bits, orc.BF16)
    return (wq, s, b), {"wq": dev(wq), "scales": dev(s, True), "biases": dev(b, True)}


def out_like(m, n):
    import torch

    return torch.empty((m, n), dtype=torch.bfloat16, device="cuda")


def check(got, want):
    assert rel_err(orc.bf16_to_f32(host(got)), orc.bf16_to_f32(want).astype(np.float64)) <= TOL


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("m", [1, 2, 4])
@pytest.mark.parametrize("gs", [32, 64, 128])
def test_norm_qkv(torch_gpu, bits, m, gs):
    k = 2048
    x = bf16_acts(10 + m, m, k)
    w = orc.f32_to_bf16(orc.normal(11, k, 1.0, 0.1))
    shapes = [2048, 512, 512]
    host_w, projs = [], []
    for i, n in enumerate(shapes):
        hw, dw = qlayer(20 + i + bits, n, k, gs, bits)
        host_w.append(hw)
        dw["y"] = out_like(m, n)
        projs.append(dw)
    mlxq.qmatmul_fused(dev(x, True), projs, gs, bits, norm_weight=dev(w, True), eps=1e-5)
    xn = orc.rms_norm(x, w, 1e-5)
    for hw, p in zip(host_w, projs):
        check(p["y"], orc.qlinear_bf16(xn, hw, gs, bits))


@pytest.mark.parametrize("m", [1, 3])
def test_repeat_o_residual(torch_gpu, m):
    kvh, hd, groups = 8, 128, 4
    k = kvh * hd * groups
    v = bf16_acts(30 + m, m, kvh * hd)
    r = bf16_acts(31 + m, m, 4096)
    hw, dw = qlayer(32, 4096, k, 64, 4)
    dw["y"] = out_like(m, 4096)
    dw["residual"] = dev(r, True)
    mlxq.qmatmul_fused(dev(v, True), [dw], 64, 4, repeat=(kvh, hd, groups))
    want = orc.add(r, orc.qlinear_bf16(orc.repeat_kv(v, kvh, hd, groups), hw, 64, 4))
    check(dw["y"], want)


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("m", [1, 2])
def test_norm_gate_up_swiglu(torch_gpu, bits, m):
    k, n = 4096, 14336
    x = bf16_acts(40 + m, m, k)
    w = orc.f32_to_bf16(orc.normal(41, k, 1.0, 0.1))
    hg, dg = qlayer(42, n, k, 64, bits)
    hu, du = qlayer(43, n, k, 64, bits)
    dg["y"], du["y"] = out_like(m, n), out_like(m, n)
    mlxq.qmatmul_fused(dev(x, True), [dg, du], 64, bits, norm_weight=dev(w, True), eps=1e-5, swiglu=True)
    xn = orc.rms_norm(x, w, 1e-5)
    want = orc.silu_mul(orc.qlinear_bf16(xn, hg, 64, bits), orc.qlinear_bf16(xn, hu, 64, bits))
    check(dg["y"], want)


def test_down_residual_and_short_gate(torch_gpu):
    """Residual epilogue at K = 14336; and a gate/up pair whose N is not a
    multiple of 16 (ragged last row tile)."""
    m = 2
    a = bf16_acts(50, m, 14336)
    r = bf16_acts(51, m, 4096)
    hw, dw = qlayer(52, 4096, 14336, 64, 4)
    dw["y"], dw["residual"] = out_like(m, 4096), dev(r, True)
    mlxq.qmatmul_fused(dev(a, True), [dw], 64, 4)
    check(dw["y"], orc.add(r, orc.qlinear_bf16(a, hw, 64, 4)))

    x = bf16_acts(53, 1, 1024)
    w = orc.f32_to_bf16(orc.normal(54, 1024, 1.0, 0.1))
    hg, dg = qlayer(55, 1000, 1024, 64, 4)
    hu, du = qlayer(56, 1000, 1024, 64, 4)
    dg["y"], du["y"] = out_like(1, 1000), out_like(1, 1000)
    mlxq.qmatmul_fused(dev(x, True), [dg, du], 64, 4, norm_weight=dev(w, True), eps=1e-5, swiglu=True)
    xn = orc.rms_norm(x, w, 1e-5)
    check(dg["y"], orc.silu_mul(orc.qlinear_bf16(xn, hg, 64, 4), orc.qlinear_bf16(xn, hu, 64, 4)))


@pytest.mark.parametrize("m", [5, 16, 32])
def test_matrix_core_residual_multi(torch_gpu, m):
    """M > 4 runs the matrix-core form: several projections and residuals."""
    x = bf16_acts(70 + m, m, 4096)
    outs, want = [], []
    for i, n in enumerate([4096, 1024]):
        hw, dw = qlayer(71 + i, n, 4096, 64, 4)
        r = bf16_acts(75 + i, m, n)
        dw["y"], dw["residual"] = out_like(m, n), dev(r, True)
        outs.append(dw)
        want.append(orc.add(r, orc.qlinear_bf16(x, hw, 64, 4)))
    mlxq.qmatmul_fused(dev(x, True), outs, 64, 4)
    for d, w in zip(outs, want):
        check(d["y"], w)


def test_unsupported_shapes_launch_nothing(torch_gpu):
    hw, dw = qlayer(60, 256, 512, 64, 4)
    dw["y"] = out_like(5, 256)
    w = dev(orc.f32_to_bf16(np.ones(512, dtype=np.float32)), True)
    with pytest.raises(mlxq.Unsupported):  # the norm form needs M <= 4
        mlxq.qmatmul_fused(dev(bf16_acts(61, 5, 512), True), [dw], 64, 4, norm_weight=w, eps=1e-5)
    with pytest.raises(mlxq.Unsupported):  # more than 32 rows
        mlxq.qmatmul_fused(dev(bf16_acts(61, 33, 512), True), [dw], 64, 4)
    with pytest.raises(mlxq.Unsupported):  # SwiGLU without a norm weight
        mlxq.qmatmul_fused(dev(bf16_acts(61, 1, 512), True), [dw, dict(dw)], 64, 4, swiglu=True)


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("gs", [32, 64, 128])
@pytest.mark.parametrize("k", [2048, 4096])
def test_norm_gate_up_swiglu_batch1_ragged(torch_gpu, bits, gs, k):
    """Batch-1 norm + gate/up + SwiGLU at every group size and both widths,
    N (1002) not a multiple of the kernel's outputs per workgroup."""
    n = 1002
    x = bf16_acts(80 + k, 1, k)
    w = orc.f32_to_bf16(orc.normal(81, k, 1.0, 0.1))
    hg, dg = qlayer(82 + bits + gs, n, k, gs, bits)
    hu, du = qlayer(83 + bits + gs, n, k, gs, bits)
    dg["y"], du["y"] = out_like(1, n), out_like(1, n)
    mlxq.qmatmul_fused(dev(x, True), [dg, du], gs, bits, norm_weight=dev(w, True), eps=1e-5, swiglu=True)
    xn = orc.rms_norm(x, w, 1e-5)
    check(dg["y"], orc.silu_mul(orc.qlinear_bf16(xn, hg, gs, bits), orc.qlinear_bf16(xn, hu, gs, bits)))


@pytest.mark.parametrize("path", ["row", "dot"])
@pytest.mark.parametrize("bits", [4, 8])
def test_batch1_forms_both_kernels(torch_gpu, monkeypatch, path, bits):
    """The batch-1 fused forms on both kernels that serve them: the whole-row
    kernel (the default where it covers the shape) and the vector-ALU kernel
    (MLXQ_QMV_NO_ROW=1): norm + q/k/v, head repeat + o + residual, norm +
    gate/up + SwiGLU, ragged N, against the oracle's unfused chain."""
    if path == "dot":
        monkeypatch.setenv("MLXQ_QMV_NO_ROW", "1")
    else:
        monkeypatch.delenv("MLXQ_QMV_NO_ROW", raising=False)
    k, gs = 4096, 64
    x = bf16_acts(140 + bits, 1, k)
    w = orc.f32_to_bf16(orc.normal(141, k, 1.0, 0.1))
    xn = orc.rms_norm(x, w, 1e-5)
    host_w, projs = [], []
    for i, n in enumerate([4096, 1000, 1000]):
        hw, dw = qlayer(142 + i + bits, n, k, gs, bits)
        host_w.append(hw)
        dw["y"] = out_like(1, n)
        projs.append(dw)
    mlxq.qmatmul_fused(dev(x, True), projs, gs, bits, norm_weight=dev(w, True), eps=1e-5)
    for hw, p in zip(host_w, projs):
        check(p["y"], orc.qlinear_bf16(xn, hw, gs, bits))
    # head repeat + o + residual
    kvh, hd, groups = 8, 128, 4
    v = bf16_acts(146, 1, kvh * hd)
    r = bf16_acts(147, 1, 4000)
    ho, do = qlayer(148 + bits, 4000, k, gs, bits)
    do["y"] = out_like(1, 4000)
    do["residual"] = dev(r, True)
    mlxq.qmatmul_fused(dev(v, True), [do], gs, bits, repeat=(kvh, hd, groups))
    xr = orc.repeat_kv(v, kvh, hd, groups)
    check(do["y"], orc.add(r, orc.qlinear_bf16(xr, ho, gs, bits)))
    # norm + gate/up + SwiGLU
    hg, dg = qlayer(149 + bits, 1500, k, gs, bits)
    hu, du = qlayer(150 + bits, 1500, k, gs, bits)
    dg["y"], du["y"] = out_like(1, 1500), out_like(1, 1500)
    mlxq.qmatmul_fused(dev(x, True), [dg, du], gs, bits, norm_weight=dev(w, True), eps=1e-5, swiglu=True)
    check(dg["y"], orc.silu_mul(orc.qlinear_bf16(xn, hg, gs, bits), orc.qlinear_bf16(xn, hu, gs, bits)))
    # down + residual at K = 14336 (Q4: 7 KB rows on the whole-row kernel)
    hd_, dd = qlayer(151 + bits, 1000, 14336, gs, bits)
    a = bf16_acts(152, 1, 14336)
    r2 = bf16_acts(153, 1, 1000)
    dd["y"], dd["residual"] = out_like(1, 1000), dev(r2, True)
    mlxq.qmatmul_fused(dev(a, True), [dd], gs, bits)
    check(dd["y"], orc.add(r2, orc.qlinear_bf16(a, hd_, gs, bits)))


@pytest.mark.parametrize("bits,k", [(4, 4096), (8, 4096), (8, 2048)])
@pytest.mark.parametrize("m", [5, 16, 17, 32])
def test_tile_norm_qkv_batched(torch_gpu, bits, k, m):
    """5..32 rows on the whole-K tile form: three projections of the same
    activations (ragged N), a bias on one, after the norm kernel (the fused
    norm form is not taken above 4 rows: every workgroup would normalise the
    same rows again)."""
    x = bf16_acts(50 + m, m, k)
    w = orc.f32_to_bf16(orc.normal(51, k, 1.0, 0.1))
    shapes = [1000, 256, 200]
    host_w, projs = [], []
    bias = orc.f32_to_bf16(orc.normal(52, 256, 0.0, 1.0))
    for i, n in enumerate(shapes):
        hw, dw = qlayer(53 + i + bits, n, k, 64, bits)
        host_w.append(hw)
        dw["y"] = out_like(m, n)
        if i == 1:
            dw["bias"] = dev(bias, True)
        projs.append(dw)
    with pytest.raises(mlxq.Unsupported):
        mlxq.qmatmul_fused(dev(x, True), projs, 64, bits, norm_weight=dev(w, True), eps=1e-5)
    mlxq.qmatmul_fused(mlxq.rms_norm(dev(x, True), dev(w, True), 1e-5), projs, 64, bits)
    xn = orc.rms_norm(x, w, 1e-5)
    for i, (hw, p) in enumerate(zip(host_w, projs)):
        want = orc.qlinear_bf16(xn, hw, 64, bits)
        if i == 1:
            want = orc.f32_to_bf16(orc.bf16_to_f32(want) + orc.bf16_to_f32(bias)[None, :])
        check(p["y"], want)


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("m", [5, 16, 32])
def test_tile_repeat_o_residual_batched(torch_gpu, bits, m):
    """5..32 rows on the whole-K tile form: GQA head repeat by remapped
    activation loads, o projection, residual epilogue."""
    kvh, hd, groups = 8, 128, 4
    k = kvh * hd * groups
    v = bf16_acts(60 + m, m, kvh * hd)
    r = bf16_acts(61 + m, m, 4096)
    hw, dw = qlayer(62 + bits, 4096, k, 64, bits)
    dw["y"] = out_like(m, 4096)
    dw["residual"] = dev(r, True)
    mlxq.qmatmul_fused(dev(v, True), [dw], 64, bits, repeat=(kvh, hd, groups))
    want = orc.add(r, orc.qlinear_bf16(orc.repeat_kv(v, kvh, hd, groups), hw, 64, bits))
    check(dw["y"], want)


def test_tile_fused_matches_legacy_form(torch_gpu, monkeypatch):
    """The tile form and the streaming matrix-core form (MLXQ_QMV_LEGACY=1)
    agree on a residual multi-projection call (both round at the same points)."""
    import torch

    m, k = 16, 4096
    x = bf16_acts(70, m, k)
    r = bf16_acts(71, m, 1024)
    outs = []
    for legacy in (False, True):
        if legacy:
            monkeypatch.setenv("MLXQ_QMV_LEGACY", "1")
        projs = []
        for i, n in enumerate([1024, 512]):
            _, dw = qlayer(72 + i, n, k, 64, 4)
            dw["y"] = out_like(m, n)
            if i == 0:
                dw["residual"] = dev(r, True)
            projs.append(dw)
        mlxq.qmatmul_fused(dev(x, True), projs, 64, 4)
        torch.cuda.synchronize()
        outs.append([orc.bf16_to_f32(host(p["y"])) for p in projs])
    for a, b in zip(*outs):
        assert np.max(np.abs(a - b)) / np.max(np.abs(b)) <= 8e-3


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("m", [5, 16, 17, 32])
@pytest.mark.parametrize("n", [14336, 8200])
def test_tile_swiglu_batched(torch_gpu, bits, m, n):
    """5..32 rows: gate and up row groups paired in one streaming launch,
    y = silu(gate) * up at MLX's rounding points (no norm: the caller ran it);
    ragged N, a bias on the gate."""
    k = 4096
    x = bf16_acts(80 + m, m, k)
    hg, dg = qlayer(81 + bits, n, k, 64, bits)
    hu, du = qlayer(82 + bits, n, k, 64, bits)
    bias = orc.f32_to_bf16(orc.normal(83, n, 0.0, 1.0))
    dg["y"], du["y"], dg["bias"] = out_like(m, n), out_like(m, n), dev(bias, True)
    mlxq.qmatmul_fused(dev(x, True), [dg, du], 64, bits, swiglu=True)
    g = orc.f32_to_bf16(orc.bf16_to_f32(orc.qlinear_bf16(x, hg, 64, bits)) + orc.bf16_to_f32(bias)[None, :])
    check(dg["y"], orc.silu_mul(g, orc.qlinear_bf16(x, hu, 64, bits)))


def test_swiglu_without_norm_needs_more_rows(torch_gpu):
    hw, dw = qlayer(90, 256, 512, 64, 4)
    dw["y"] = out_like(4, 256)
    with pytest.raises(mlxq.Unsupported):
        mlxq.qmatmul_fused(dev(bf16_acts(91, 4, 512), True), [dw, dict(dw)], 64, 4, swiglu=True)


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("m", [16, 24])
def test_tile_fused_32_row_workgroups_ragged(torch_gpu, bits, m):
    """Three projections whose 16-row tiles exceed one round of CUs take 32
    rows per workgroup (ragged N = 4008 / 1032 / 1032); one projection has a
    residual, so the launch loads residual values early and the other
    segments read their dummy values from y.  Against the oracle chain."""
    k = 4096
    x = bf16_acts(70 + m, m, k)
    r = bf16_acts(71 + m, m, 1032)
    shapes = [4008, 1032, 1032]
    host_w, projs = [], []
    for i, n in enumerate(shapes):
        hw, dw = qlayer(72 + i + bits, n, k, 64, bits)
        host_w.append(hw)
        dw["y"] = out_like(m, n)
        if i == 2:
            dw["residual"] = dev(r, True)
        projs.append(dw)
    mlxq.qmatmul_fused(dev(x, True), projs, 64, bits)
    for i, (hw, p) in enumerate(zip(host_w, projs)):
        want = orc.qlinear_bf16(x, hw, 64, bits)
        if i == 2:
            want = orc.add(r, want)
        check(p["y"], want)
