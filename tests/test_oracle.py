"""Pin the CPU oracle (oracle/liboracle.so) before it is trusted as the checker.

Each check compares the oracle with something other than itself: the
reference's own known-answer vectors (tests/golden/gguf_kat.json), published
generator outputs, numpy/torch IEEE conversions, closed forms and exhaustive
enumeration.  No GPU.
"""
import json
from pathlib import Path

import numpy as np
import pytest

import oracle as orc

KAT = json.loads((Path(__file__).resolve().parent / "golden" / "gguf_kat.json").read_text())
rng = np.random.default_rng(1234)


# ---------------------------------------------------------------- generators
def test_splitmix64_published_outputs():
    # SplitMix64 reference outputs for state 0 (Vigna's splitmix64.c), the
    # generator of src/primitives/sampler.rs:40-55.
    got = orc.splitmix64(0, 3)
    assert [int(v) for v in got] == [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F]


def test_next_f32_is_24bit_fraction():
    import ctypes

    st = ctypes.c_uint64(7)
    st2 = ctypes.c_uint64(7)
    for _ in range(100):
        f = orc.lib().orc_splitmix64_next_f32(ctypes.byref(st))
        u = orc.lib().orc_splitmix64_next(ctypes.byref(st2))
        assert f == np.float32((u >> 40) / float(1 << 24))  # sampler.rs:57-59
        assert 0.0 <= f < 1.0


def test_normal_moments():
    x = orc.normal(0x5EED, 1_000_000, 0.0, 1.0).astype(np.float64)
    assert abs(x.mean()) < 5e-3
    assert abs(x.std() - 1.0) < 5e-3
    assert abs(((x - x.mean()) ** 4).mean() / x.var() ** 2 - 3.0) < 0.05  # Gaussian kurtosis
    y = orc.normal(1, 100_000, 0.0, 0.02)
    assert abs(y.std() - 0.02) < 5e-4
    assert not np.array_equal(orc.normal(1, 16), orc.normal(2, 16))
    assert np.array_equal(orc.normal(3, 16), orc.normal(3, 16))


# ---------------------------------------------------------------- conversions
def test_f16_to_f32_exhaustive():
    L = orc.lib()
    bits = np.arange(65536, dtype=np.uint16)
    ref = bits.view(np.float16).astype(np.float32)
    got = np.array([L.orc_f16_to_f32(int(b)) for b in bits], dtype=np.float32)
    finite = np.isfinite(ref)
    assert np.array_equal(got[finite].view(np.uint32), ref[finite].view(np.uint32))
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    assert np.array_equal(np.isinf(got), np.isinf(ref))


def test_f32_to_f16_matches_numpy():
    L = orc.lib()
    u = rng.integers(0, 2**32, size=20000, dtype=np.uint64).astype(np.uint32)
    # bias the sample toward the f16 range, including subnormals and ties
    vals = np.concatenate([u.view(np.float32), rng.normal(0, 0.02, 20000).astype(np.float32),
                           (np.arange(-70000, 70000, 7) / 7.0).astype(np.float32),
                           np.float32([6e-8, 3e-8, 2.98e-8, 65504, 65519.99, 65520, -0.0, 0.0])])
    vals = vals[np.isfinite(vals)]
    with np.errstate(over="ignore"):
        ref = vals.astype(np.float16).view(np.uint16)
    got = np.array([L.orc_f32_to_f16(float(v)) for v in vals], dtype=np.uint16)
    assert np.array_equal(got, ref)


def test_f32_to_bf16_matches_torch():
    import torch

    L = orc.lib()
    u = rng.integers(0, 2**32, size=20000, dtype=np.uint64).astype(np.uint32)
    vals = np.concatenate([u.view(np.float32), np.float32([1.0 + 2**-8, 1.0 + 3 * 2**-8, -0.0, np.inf, -np.inf])])
    vals = vals[~np.isnan(vals)]
    ref = torch.from_numpy(vals).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    got = np.array([L.orc_f32_to_bf16(float(v)) for v in vals], dtype=np.uint16)
    assert np.array_equal(got, ref)
    assert np.array_equal(orc.f32_to_bf16(vals), ref)


# ---------------------------------------------------------------- GGUF
def test_geometry_matches_reference_table():
    for tag, (e, b) in KAT["geometry"].items():
        assert orc.gguf_block(int(tag)) == (e, b)
    for tag, n, nbytes in KAT["byte_len"]:
        assert orc.gguf_tensor_byte_len(tag, n) == nbytes
    for tag in KAT["unsupported_tags"]:
        with pytest.raises(orc.OracleError) as e:
            orc.gguf_block(tag)
        assert e.value.status == 3


@pytest.mark.parametrize("case", KAT["cases"], ids=lambda c: c["name"])
def test_reference_known_answers(case):
    data = np.frombuffer(bytes.fromhex(case["hex"]), dtype=np.uint8)
    out = orc.gguf_dequantize(case["tag"], data, case["n"])
    if "expect_all" in case:
        assert np.array_equal(out, np.float32(case["expect_all"]))
    for i, v in case.get("expect", {}).items():
        assert out[int(i)] == np.float32(v)


def test_error_paths():
    with pytest.raises(orc.OracleError) as e:  # dequant.rs:159-163
        orc.gguf_dequantize(2, np.zeros(18, np.uint8), 31)
    assert e.value.status == 2
    with pytest.raises(orc.OracleError) as e:  # dequant.rs:166-171
        orc.gguf_dequantize(2, np.zeros(17, np.uint8), 32)
    assert e.value.status == 4
    with pytest.raises(orc.OracleError) as e:  # dequant.rs:109-111
        orc.gguf_dequantize(9, np.zeros(64, np.uint8), 32)
    assert e.value.status == 3


def _blocks(tag, nblk, d=1.0, fill=None):
    e, b = orc.gguf_block(tag)
    raw = rng.integers(0, 256, size=(nblk, b), dtype=np.uint8) if fill is None else np.full((nblk, b), fill, np.uint8)
    return raw, e, b


def test_q8_0_exhaustive_bytes():
    # every byte value with d = 1: y = (int8)byte exactly
    blk = np.zeros((8, 34), np.uint8)
    blk[:, 0:2] = [0x00, 0x3C]
    blk[:, 2:] = np.arange(256, dtype=np.uint16).reshape(8, 32).astype(np.uint8)
    out = orc.gguf_dequantize(8, blk, 256)
    assert np.array_equal(out, np.arange(256).astype(np.uint8).view(np.int8).astype(np.float32))


def test_q4_0_and_iq4_nl_exhaustive_nibbles():
    blk = np.zeros((16, 18), np.uint8)
    blk[:, 0:2] = [0x00, 0x3C]  # d = 1
    blk[:, 2:] = np.arange(256, dtype=np.uint16).reshape(16, 16).astype(np.uint8)
    q = blk[:, 2:]
    out = orc.gguf_dequantize(2, blk, 512).reshape(16, 32)
    assert np.array_equal(out[:, :16], (q & 15).astype(np.float32) - 8)
    assert np.array_equal(out[:, 16:], (q >> 4).astype(np.float32) - 8)
    nl = orc.gguf_dequantize(20, blk, 512).reshape(16, 32)
    # row 0 holds bytes 0..15, i.e. every low nibble once: that is the codebook.
    # It is strictly increasing and has the two values the reference pins.
    table = nl[0, :16]
    assert table[0] == -127 and table[8] == 1  # dequant.rs:773-778
    assert np.all(np.diff(table) > 0)
    assert np.array_equal(nl[:, :16], table[q & 15])
    assert np.array_equal(nl[:, 16:], table[q >> 4])


def test_q5_family_reduces_to_q4_family():
    # with qh = 0 the fifth bit is absent: Q5_0 = Q4_0 - 8d, Q5_1 = Q4_1 (exact)
    n = 64
    q4 = rng.integers(0, 256, size=(n, 18), dtype=np.uint8)
    q4[:, 1] &= 0x3B  # keep d finite and moderate
    q5 = np.zeros((n, 22), np.uint8)
    q5[:, 0:2] = q4[:, 0:2]
    q5[:, 6:] = q4[:, 2:]
    a = orc.gguf_dequantize(2, q4, 32 * n).reshape(n, 32)
    b = orc.gguf_dequantize(6, q5, 32 * n).reshape(n, 32)
    d = np.array([orc.lib().orc_f16_to_f32(int(q4[i, 0]) | (int(q4[i, 1]) << 8)) for i in range(n)], np.float32)
    assert np.array_equal(b + 8 * d[:, None], a)
    q41 = rng.integers(0, 256, size=(n, 20), dtype=np.uint8)
    q41[:, 1] &= 0x3B
    q41[:, 3] &= 0x3B
    q51 = np.zeros((n, 24), np.uint8)
    q51[:, 0:4] = q41[:, 0:4]
    q51[:, 8:] = q41[:, 4:]
    assert np.array_equal(orc.gguf_dequantize(3, q41, 32 * n), orc.gguf_dequantize(7, q51, 32 * n))
    # qh all ones adds exactly 16*d (Q5_0) to every element
    q5h = q5.copy()
    q5h[:, 2:6] = 0xFF
    c = orc.gguf_dequantize(6, q5h, 32 * n).reshape(n, 32)
    assert np.allclose(c - b, 16 * d[:, None], rtol=0, atol=0)


def test_q4_k_closed_form():
    # d = 1, dmin = 1; six-bit scales sc_j and mins m_j chosen per sub-block;
    # the reference's formula then gives y = sc_j * nibble - m_j exactly.
    sc = [1, 2, 3, 63, 17, 32, 5, 40]
    mn = [0, 1, 2, 3, 63, 20, 9, 33]
    s = np.zeros(12, np.uint8)
    for j in range(8):  # 12-byte packing described at dequant.rs:373-383
        if j < 4:
            s[j] |= sc[j]
            s[j + 4] |= mn[j]
        else:
            s[j + 4] = (sc[j] & 15) | ((mn[j] & 15) << 4)
            s[j - 4] |= (sc[j] >> 4) << 6
            s[j] |= (mn[j] >> 4) << 6
    qs = rng.integers(0, 256, size=128, dtype=np.uint8)
    blk = np.concatenate([np.uint8([0x00, 0x3C, 0x00, 0x3C]), s, qs])
    y = orc.gguf_dequantize(12, blk, 256)
    nib = np.zeros(256, np.int64)
    for c in range(4):  # 32 bytes per 64 elements: low nibbles first, then high
        nib[64 * c:64 * c + 32] = qs[32 * c:32 * c + 32] & 15
        nib[64 * c + 32:64 * c + 64] = qs[32 * c:32 * c + 32] >> 4
    want = np.array([sc[e // 32] * nib[e] - mn[e // 32] for e in range(256)], np.float32)
    assert np.array_equal(y, want)


def test_iq4_xs_with_unit_subscales_equals_iq4_nl():
    # ls = 33 -> dl = d*(33-32) = d, so each 32-element sub-block decodes like
    # an IQ4_NL block with the same d and 16 qs bytes.
    n = 16
    xs = np.zeros((n, 136), np.uint8)
    nl = np.zeros((n * 8, 18), np.uint8)
    for i in range(n):
        d = rng.integers(0x2000, 0x3C00)
        xs[i, 0:2] = [d & 0xFF, d >> 8]
        xs[i, 2:4] = [0x55, 0x55]  # high 2 bits = 1 for all 8 sub-blocks (ls = 16 + low)
        xs[i, 4:8] = 0x11          # low nibble 1 -> ls = 17 ... adjusted below
        xs[i, 8:] = rng.integers(0, 256, size=128, dtype=np.uint8)
        for ib in range(8):
            nl[8 * i + ib, 0:2] = xs[i, 0:2]
            nl[8 * i + ib, 2:] = xs[i, 8 + 16 * ib:8 + 16 * ib + 16]
    # ls = low | high<<4 = 1 | 1<<5? high bits 01 -> 16; low 1 -> ls=17 -> dl=-15d
    y17 = orc.gguf_dequantize(23, xs, 256 * n)
    ynl = orc.gguf_dequantize(20, nl, 256 * n)
    d = np.repeat([orc.lib().orc_f16_to_f32(int(xs[i, 0]) | (int(xs[i, 1]) << 8)) for i in range(n)], 256)
    kv = (ynl / d)  # codebook values, exact (d * kv is exact: 11 x 8 bits)
    assert np.array_equal((np.float32(d) * np.float32(-15)) * kv.astype(np.float32), y17)
    xs[:, 2:4] = [0xAA, 0xAA]  # high bits 10 -> 32; low nibble 1 -> ls = 33
    assert np.array_equal(orc.gguf_dequantize(23, xs, 256 * n), ynl)


def test_q6_k_structure():
    # q = 32 everywhere (ql nibble 0, qh pairs = 2) -> zero (dequant.rs:854-875),
    # and q = 33 (ql nibble 1) -> d * scale exactly, sub-block by sub-block.
    blk = np.zeros(210, np.uint8)
    blk[128:192] = 0xAA
    sc = rng.integers(-128, 128, size=16).astype(np.int8)
    blk[192:208] = sc.view(np.uint8)
    blk[208:210] = [0x00, 0x3C]
    assert np.all(orc.gguf_dequantize(14, blk, 256) == 0)
    blk[0:128] = 0x11
    y = orc.gguf_dequantize(14, blk, 256)
    assert np.array_equal(y, np.repeat(sc.astype(np.float32), 16))


@pytest.mark.parametrize("tag,rel", [(2, 0.12), (8, 0.01), (12, 0.12), (14, 0.04), (20, 0.12), (23, 0.12)])
def test_producer_roundtrip(tag, rel):
    x = orc.normal(0x5EED0000 + tag, 64 * 256, 0.0, 0.02)
    blocks = orc.gguf_quantize(tag, x)
    y = orc.gguf_dequantize(tag, blocks, x.size)
    err = np.sqrt(np.mean((y - x) ** 2)) / np.sqrt(np.mean(x ** 2))
    assert err < rel, err


# ---------------------------------------------------------------- affine quantize
def _unpack(wq, bits, cols):
    per = 32 // bits
    k = np.arange(cols)
    return ((wq[:, k // per] >> ((k % per) * bits).astype(np.uint32)) & ((1 << bits) - 1)).astype(np.int64)


def test_affine_packing_closed_form():
    # w = k % 16 in a 64-group: min 0, max 15 -> scale = -1, bias = 15, code = 15 - w
    w = np.tile(np.arange(64) % 16, (2, 1)).astype(np.float32)
    wq, s, b = orc.affine_quantize(w, 64, 4, orc.F32)
    assert np.all(s == -1.0) and np.all(b == 15.0)
    want = 0
    for i in range(8):
        want |= (15 - i % 16) << (4 * i)
    assert wq[0, 0] == want
    assert np.array_equal(_unpack(wq, 4, 64), 15 - w.astype(np.int64))
    wq8, s8, b8 = orc.affine_quantize(w * 17, 64, 8, orc.F32)  # 0..255
    assert np.array_equal(_unpack(wq8, 8, 64), 255 - (w * 17).astype(np.int64))


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("gs", [32, 64, 128])
def test_affine_grid_invariants_f32(bits, gs):
    rows, cols = 64, 512
    w = orc.normal(99 + bits + gs, rows * cols, 0.0, 0.02).reshape(rows, cols)
    w[3, :gs] = 0.125  # constant group
    w[5, gs:2 * gs] = np.linspace(-1, 1, gs)
    wq, s, b = orc.affine_quantize(w, gs, bits, orc.F32)
    q = _unpack(wq, bits, cols)
    nb = (1 << bits) - 1
    assert q.min() >= 0 and q.max() <= nb
    sg = np.repeat(s, gs, axis=1).astype(np.float64)
    bg = np.repeat(b, gs, axis=1).astype(np.float64)
    rec = sg * q + bg
    err = np.abs(rec - w)
    # interior codes: within half a step.  The scale is snapped so that 0 is on
    # the grid (|q0| >= n_bins/2), which can leave the far extreme up to
    # n_bins * 0.5/|q0| <= 1 step beyond the last grid point (clamped code).
    interior = (q > 0) & (q < nb)
    assert np.all(err[interior] <= np.abs(sg[interior]) * (0.5 + 1e-5) + 1e-12)
    assert np.all(err <= np.abs(sg) * (1.5 + 1e-5) + 1e-12)
    # nearest grid point: no other code is closer (rint, not floor/trunc)
    lo = np.abs(sg * np.clip(q - 1, 0, nb) + bg - w)
    hi = np.abs(sg * np.clip(q + 1, 0, nb) + bg - w)
    # (f32 rounding of (w - bias)/scale can flip exact ties: 1e-4 step slack)
    assert np.all(err <= lo + 1e-4 * np.abs(sg)) and np.all(err <= hi + 1e-4 * np.abs(sg))
    # the edge element (largest magnitude) reconstructs to the bias exactly
    for r in range(0, rows, 7):
        for g in range(cols // gs):
            grp = w[r, g * gs:(g + 1) * gs]
            if b[r, g] != 0:
                assert b[r, g] in grp
                j = int(np.argmax(grp == b[r, g]))
                assert q[r, g * gs + j] == 0
    assert len(set(q[3, :gs])) == 1


def test_affine_bf16_inputs_bounded():
    rows, cols = 32, 256
    w = orc.f32_to_bf16(orc.normal(5, rows * cols, 0.0, 0.02)).reshape(rows, cols)
    wq, s, b = orc.affine_quantize(w, 64, 4, orc.BF16)
    wf = orc.bf16_to_f32(w).astype(np.float64)
    sg = np.repeat(orc.bf16_to_f32(s), 64, axis=1).astype(np.float64)
    bg = np.repeat(orc.bf16_to_f32(b), 64, axis=1).astype(np.float64)
    q = _unpack(wq, 4, cols)
    err = np.abs(sg * q + bg - wf)
    # half a step (1.5 at the clamped ends) plus bf16 rounding of scale and bias
    interior = (q > 0) & (q < 15)
    tol = np.abs(bg) * 2**-8 + np.abs(sg) * 15 * 2**-8 + 1e-9
    assert np.all(err[interior] <= (np.abs(sg) * 0.5 + tol)[interior])
    assert np.all(err <= np.abs(sg) * 1.5 + tol)
    deq = orc.bf16_to_f32(orc.affine_dequantize(wq, s, b, 64, 4, orc.BF16))
    assert np.array_equal(deq, orc.bf16_to_f32(orc.f32_to_bf16((sg * q + bg).astype(np.float32))))


def test_reference_roundtrip_q8():
    a = KAT["affine"]["roundtrip_q8"]  # quant.rs:91-107
    w = np.float32(a["w"]).reshape(a["shape"])
    wq, s, b = orc.affine_quantize(w, a["group_size"], a["bits"], orc.F32)
    back = orc.affine_dequantize(wq, s, b, a["group_size"], a["bits"], orc.F32)
    assert np.max(np.abs(back - w)) < a["max_abs_err"]


def test_reference_matmul_q8_and_f64_gemm():
    a = KAT["affine"]["matmul_q8"]  # quant.rs:111-125 (bf16 activations here)
    w = np.float32(a["w"]).reshape(a["shape"])
    x = np.float32(a["x"]).reshape(1, 64)
    wq, s, b = orc.affine_quantize(orc.f32_to_bf16(w), 64, 8, orc.BF16)
    y = orc.qmatmul_f64(orc.f32_to_bf16(x), wq, s, b, 64, 8)
    dense = x.astype(np.float64) @ w.astype(np.float64).T
    assert np.max(np.abs(y - dense)) < a["max_abs_err"]


@pytest.mark.parametrize("bits", [4, 8])
def test_f64_gemm_matches_numpy(bits):
    m, n, k = 5, 48, 256
    w = orc.f32_to_bf16(orc.normal(11, n * k, 0, 0.02)).reshape(n, k)
    x = orc.f32_to_bf16(orc.normal(12, m * k)).reshape(m, k)
    wq, s, b = orc.affine_quantize(w, 64, bits, orc.BF16)
    q = _unpack(wq, bits, k).astype(np.float64)
    wd = np.repeat(orc.bf16_to_f32(s), 64, 1) * q + np.repeat(orc.bf16_to_f32(b), 64, 1)
    ref = orc.bf16_to_f32(x).astype(np.float64) @ wd.T
    got = orc.qmatmul_f64(x, wq, s, b, 64, bits)
    assert np.allclose(got, ref, rtol=1e-12, atol=1e-12)
    got32 = orc.qmatmul_f32(x, wq, s, b, 64, bits, threads=2)
    assert np.max(np.abs(got32 - ref)) <= 1e-4 * np.max(np.abs(ref))


# ---------------------------------------------------------------- decode layer chain ops
def _torch_bf16(a: np.ndarray) -> np.ndarray:
    """f32 -> bf16 bits through torch's own cast (an implementation independent of the oracle)."""
    import torch

    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def test_rms_norm_known_answer():
    # x = [3, 4] (mean square 12.5), w = 1, eps = 0: x / sqrt(12.5) = [0.848528.., 1.131370..]
    x = orc.f32_to_bf16(np.array([[3.0, 4.0]], dtype=np.float32))
    w = orc.f32_to_bf16(np.ones(2, dtype=np.float32))
    y = orc.bf16_to_f32(orc.rms_norm(x, w, 0.0))
    want = _torch_bf16(np.array([3 / np.sqrt(12.5), 4 / np.sqrt(12.5)], dtype=np.float32))
    assert np.array_equal(orc.f32_to_bf16(y).ravel(), want)


def test_rms_norm_invariants():
    x = orc.f32_to_bf16(orc.normal(5, 4 * 512, 0.0, 3.0)).reshape(4, 512)
    ones = orc.f32_to_bf16(np.ones(512, dtype=np.float32))
    y = orc.rms_norm(x, ones, 0.0)
    # scaling the input by a power of two leaves the output unchanged (eps = 0)
    x4 = orc.f32_to_bf16(orc.bf16_to_f32(x) * 4.0)
    assert np.array_equal(orc.rms_norm(x4, ones, 0.0), y)
    # a weight of 2 doubles every output exactly; unit weight gives unit RMS
    twos = orc.f32_to_bf16(np.full(512, 2.0, dtype=np.float32))
    assert np.array_equal(orc.bf16_to_f32(orc.rms_norm(x, twos, 0.0)), 2.0 * orc.bf16_to_f32(y))
    rms = np.sqrt(np.mean(orc.bf16_to_f32(y).astype(np.float64) ** 2, axis=1))
    assert np.all(np.abs(rms - 1.0) < 4e-3)
    # eps enters under the root: a zero row stays zero, a tiny row is damped
    z = np.zeros((1, 512), dtype=np.uint16)
    assert not orc.bf16_to_f32(orc.rms_norm(z, ones, 1e-5)).any()


def test_rms_norm_matches_float64_formula_within_a_bf16_step():
    x = orc.f32_to_bf16(orc.normal(6, 8 * 256, 0.0, 1.0)).reshape(8, 256)
    w = orc.f32_to_bf16(orc.normal(7, 256, 1.0, 0.1))
    xf, wf = orc.bf16_to_f32(x).astype(np.float64), orc.bf16_to_f32(w).astype(np.float64)
    ref = wf * xf / np.sqrt(np.mean(xf * xf, axis=1, keepdims=True) + 1e-5)
    got = orc.bf16_to_f32(orc.rms_norm(x, w, 1e-5)).astype(np.float64)
    # two bf16 roundings: at most ~2^-8 relative each
    assert np.all(np.abs(got - ref) <= np.abs(ref) * 2 ** -7 + 1e-30)


def test_silu_mul_against_scipy_expit():
    from scipy.special import expit

    g = orc.f32_to_bf16(np.concatenate([orc.normal(8, 4000, 0.0, 4.0), [0.0, 1.0, -1.0, 30.0, -30.0, 88.0, -88.0]]).astype(np.float32))
    u = orc.f32_to_bf16(orc.normal(9, g.size, 0.0, 1.0))
    gf, uf = orc.bf16_to_f32(g), orc.bf16_to_f32(u)
    s = orc.bf16_to_f32(_torch_bf16(expit(gf.astype(np.float64)).astype(np.float32)))
    a = orc.bf16_to_f32(_torch_bf16(gf * s))
    want = _torch_bf16(a * uf)
    got = orc.silu_mul(g, u)
    # scipy's expit vs libm expf may differ in the last f32 bit, which can move a bf16 tie
    assert np.mean(got == want) > 0.999
    assert np.all(np.abs(orc.bf16_to_f32(got) - orc.bf16_to_f32(want)) <= np.abs(orc.bf16_to_f32(want)) * 2 ** -7)
    ones = orc.f32_to_bf16(np.ones(4, dtype=np.float32))
    # silu(0) = 0, silu(1) = sigmoid(1) = 0.7310585786.., silu(30) = 30, silu(-30) ~ -0
    v = orc.bf16_to_f32(orc.silu_mul(orc.f32_to_bf16(np.array([0.0, 1.0, 30.0, -30.0], dtype=np.float32)), ones))
    assert v[0] == 0.0 and v[2] == 30.0 and abs(v[3]) < 1e-10
    assert v[1] == orc.bf16_to_f32(_torch_bf16(np.array([0.7310585786300049], dtype=np.float32)))[0]


def test_add_matches_torch_bf16_add():
    import torch

    a = orc.f32_to_bf16(orc.normal(10, 5000, 0.0, 2.0))
    b = orc.f32_to_bf16(orc.normal(11, 5000, 0.0, 2.0))
    ta = torch.from_numpy(a.view(np.int16)).view(torch.bfloat16)
    tb = torch.from_numpy(b.view(np.int16)).view(torch.bfloat16)
    want = (ta + tb).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(orc.add(a, b), want)


def test_repeat_kv_reference_known_answer():
    # src/primitives/attention.rs:294-300: heads [0,1], [2,3] with 2 groups ->
    # head0, head0, head1, head1
    x = orc.f32_to_bf16(np.array([0.0, 1.0, 2.0, 3.0], dtype=np.float32)).reshape(1, 4)
    y = orc.bf16_to_f32(orc.repeat_kv(x, 2, 2, 2)).ravel()
    assert y.tolist() == [0.0, 1.0, 0.0, 1.0, 2.0, 3.0, 2.0, 3.0]
    # groups = 1 is the identity (attention.rs:281-285)
    assert np.array_equal(orc.repeat_kv(x, 2, 2, 1), x)


def test_permute_inverse_qk_reference_known_answer():
    # src/gguf/convert.rs:391-423: the llama.cpp forward interleave per head
    # (reshape(n_head, 2, hd/2).swapaxes(1, 2): GGUF row 2j+k <- HF row k*hd/2+j)
    # followed by the inverse must give back the HF rows, and is not the identity
    n_head, hd, in_dim = 2, 4, 3
    hf = np.arange(n_head * hd * in_dim, dtype=np.float32).reshape(n_head * hd, in_dim)
    gguf = np.empty_like(hf)
    half = hd // 2
    for h in range(n_head):
        for k in range(2):
            for j in range(half):
                gguf[h * hd + 2 * j + k] = hf[h * hd + k * half + j]
    assert not np.array_equal(gguf, hf)
    assert np.array_equal(orc.permute_inverse_qk(gguf, n_head), hf)
    # Llama-3 k_proj geometry: 8 heads x 128 rows, a permutation of the rows
    w = np.arange(1024, dtype=np.float32).reshape(1024, 1)
    p = orc.permute_inverse_qk(w, 8).ravel()
    assert sorted(p.tolist()) == w.ravel().tolist() and p[1] == 2.0 and p[64] == 1.0
