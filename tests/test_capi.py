"""The C ABI library loads, exports every symbol include/mlxq.h declares, and
rejects bad arguments with the reference's error classes -- all without a GPU
(every call here returns before anything is launched)."""
import ctypes
import re
from pathlib import Path

import pytest

import mlxq

ROOT = Path(__file__).resolve().parents[1]


def declared_symbols():
    text = (ROOT / "include" / "mlxq.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(mlxq_[a-z0-9_]+)\s*\(", text)))


def test_exports_every_declared_symbol():
    L = mlxq.lib()
    syms = declared_symbols()
    assert len(syms) >= 10
    for s in syms:
        assert hasattr(L, s), s
    assert set(syms) == set(mlxq.SIGNATURES), "ctypes signature table out of sync with the header"


def test_version():
    assert "gfx950" in mlxq.version()


def test_gguf_geometry_matches_reference_table():
    import json

    kat = json.loads((ROOT / "tests" / "golden" / "gguf_kat.json").read_text())
    for tag, (e, b) in kat["geometry"].items():
        assert mlxq.gguf_block(int(tag)) == (e, b)
    for tag in kat["supported_tags"]:
        mlxq.gguf_block(tag)
    for tag, n, nbytes in kat["byte_len"]:
        assert mlxq.gguf_tensor_byte_len(tag, n) == nbytes
    for tag in kat["unsupported_tags"]:  # dequant.rs:763-765
        with pytest.raises(mlxq.Unsupported):
            mlxq.gguf_block(tag)
        with pytest.raises(mlxq.Unsupported):
            mlxq.gguf_tensor_byte_len(tag, 256)


def _gguf(tag, data_len, n, out_dtype=mlxq.F32):
    fake = ctypes.c_void_p(0x1000)  # never dereferenced: the checks fail first
    return mlxq.lib().mlxq_gguf_dequantize(tag, fake, data_len, n, out_dtype, fake, None)


def test_gguf_error_paths():
    assert _gguf(2, 18, 31) == mlxq.ERR_SHAPE          # dequant.rs:159-163
    assert b"not a multiple of 32" in mlxq.lib().mlxq_last_error()
    assert _gguf(2, 17, 32) == mlxq.ERR_SHORT_BUFFER   # dequant.rs:166-171
    assert b"needs 18 bytes" in mlxq.lib().mlxq_last_error()
    assert _gguf(9, 64, 32) == mlxq.ERR_UNSUPPORTED    # dequant.rs:109-111
    assert _gguf(15, 292, 256) == mlxq.ERR_UNSUPPORTED  # dequant.rs:763-765 (Q8_K)
    assert _gguf(16, 65, 256) == mlxq.ERR_SHORT_BUFFER  # IQ2_XXS: 66 bytes per 256
    assert _gguf(2, 18, 32, out_dtype=mlxq.F16) == mlxq.ERR_UNSUPPORTED
    assert _gguf(2, 0, 0) == mlxq.OK                   # empty tensor


def test_quantize_and_qmatmul_argument_errors():
    L = mlxq.lib()
    p = ctypes.c_void_p(0x1000)
    assert L.mlxq_quantize(p, mlxq.BF16, 4, 100, 64, 4, p, p, p, None) == mlxq.ERR_SHAPE
    assert b"not divisible by group_size" in L.mlxq_last_error()
    assert L.mlxq_quantize(p, mlxq.BF16, 4, 128, 64, 3, p, p, p, None) == mlxq.ERR_UNSUPPORTED
    assert L.mlxq_quantize(p, mlxq.BF16, 4, 128, 48, 4, p, p, p, None) == mlxq.ERR_UNSUPPORTED
    assert L.mlxq_quantize(p, mlxq.F16, 4, 128, 64, 4, p, p, p, None) == mlxq.ERR_UNSUPPORTED
    assert L.mlxq_dequantize(p, p, p, mlxq.BF16, 4, 96, 64, 4, p, None) == mlxq.ERR_SHAPE
    assert L.mlxq_qmatmul(p, 1, p, p, p, None, 64, 100, 64, 4, p, None, 0, None) == mlxq.ERR_SHAPE
    assert L.mlxq_qmatmul(p, 1, p, p, p, None, 64, 128, 64, 2, p, None, 0, None) == mlxq.ERR_UNSUPPORTED
    # workspace: split-K partials of the batched-decode kernel (group 64,
    # 2 <= M <= 32: at most 16 slices of M x N f32) and of qmm shapes whose
    # 128-row tiles fill under 3/4 of the 256 CUs (slices chosen to fill
    # about one round)
    assert mlxq.workspace_size(1, 4096, 4096, 64, 4) == 0
    assert mlxq.workspace_size(32, 4096, 4096, 64, 4) == 16 * 32 * 4096 * 4
    assert mlxq.workspace_size(32, 4096, 4096, 32, 4) == 0
    # prefill routes: the library GEMM needs the whole weight as bf16 plus
    # 32 MiB for hipBLASLt; 33..64 rows run as 32-row decode calls
    lib = lambda n, k: n * k * 2 + (32 << 20)  # noqa: E731
    assert mlxq.workspace_size(2048, 4096, 4096, 64, 4) == lib(4096, 4096)          # square, M >= 1024: library
    assert mlxq.workspace_size(512, 4096, 4096, 64, 4) == 4 * 512 * 4096 * 4        # qmm, 128-row tiles, 4 slices
    # (arguments: M, N, K)
    assert mlxq.workspace_size(2048, 14336, 4096, 64, 4) == lib(14336, 4096)        # gate/up-like, M >= 1024
    assert mlxq.workspace_size(512, 14336, 4096, 64, 8) == 0                        # gate/up-like qmm: unsplit
    assert mlxq.workspace_size(2048, 4096, 14336, 64, 4) == 0                       # down-like qmm: unsplit
    assert mlxq.workspace_size(4096, 4096, 14336, 64, 4) == lib(4096, 14336)        # down-like, M = 4096
    assert mlxq.workspace_size(2048, 1024, 4096, 64, 4) == 4 * 2048 * 1024 * 4      # k/v-like qmm: 4 slices
    assert mlxq.workspace_size(64, 4096, 4096, 64, 4) == 16 * 32 * 4096 * 4      # decode chunks of 32
    assert L.mlxq_qmatmul_algo(p, 1, p, p, p, None, 64, 128, 64, 4, p, None, 0, 7, None) == mlxq.ERR_INVALID
    # M = 0 is a no-op
    assert L.mlxq_qmatmul(p, 0, p, p, p, None, 64, 128, 64, 4, p, None, 0, None) == mlxq.OK


def test_workspace_sizes_fused_prefill(monkeypatch):
    """MLXQ_QMM_FUSED=1: prefill always on the qmm kernel, which splits K
    (f32 partials in the workspace) only when even its 128-row tiles fill
    under 3/4 of the 256 CUs, into slices of whole 512-K periods."""
    monkeypatch.setenv("MLXQ_QMM_FUSED", "1")
    assert mlxq.workspace_size(2048, 4096, 4096, 64, 4) == 0                      # 256 128-row tiles: unsplit
    assert mlxq.workspace_size(2048, 4096, 14336, 64, 4) == 0
    assert mlxq.workspace_size(2048, 14336, 4096, 64, 4) == 0
    assert mlxq.workspace_size(2048, 1024, 4096, 64, 4) == 4 * 2048 * 1024 * 4    # 128-wide tiles, 4 slices


def test_workspace_sizes_cover_every_decode_shape():
    for k, n in [(4096, 4096), (4096, 1024), (4096, 14336), (14336, 4096)]:
        for m in (1, 4, 16, 32, 2048):
            for bits in (4, 8):
                mlxq.workspace_size(m, n, k, 64, bits)


def test_header_compiles_as_c99(tmp_path):
    """include/mlxq.h is a plain C header (the boundary binds from C / cgo /
    bindgen): it compiles alone under -std=c99 -pedantic with warnings as errors."""
    import shutil
    import subprocess

    if not shutil.which("gcc"):
        pytest.skip("no gcc")
    src = tmp_path / "h.c"
    src.write_text('#include "mlxq.h"\nint main(void) { return 0; }\n')
    r = subprocess.run(["gcc", "-std=c99", "-pedantic", "-Wall", "-Wextra", "-Werror", f"-I{ROOT / 'include'}",
                        "-c", str(src), "-o", str(tmp_path / "h.o")], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


def test_qmatmul_add_rms_norm_argument_errors():
    """Checked before any launch: shape, null and alignment, N % 8, eps."""
    L = mlxq.lib()
    p = ctypes.c_void_p(0x1000)
    f = L.mlxq_qmatmul_add_rms_norm
    ok = (p, 16, p, p, p, None, 4096, 4096, 64, 4)
    assert f(p, 16, p, p, p, None, 4096, 100, 64, 4, p, p, 1e-5, p, p, None, 0, None) == mlxq.ERR_SHAPE
    assert f(*ok, None, p, 1e-5, p, p, None, 0, None) == mlxq.ERR_INVALID
    assert f(*ok, p, p, 1e-5, ctypes.c_void_p(0x1002), p, None, 0, None) == mlxq.ERR_INVALID
    assert f(p, 16, p, p, p, None, 4100, 4096, 64, 4, p, p, 1e-5, p, p, None, 0, None) == mlxq.ERR_SHAPE
    assert f(*ok, p, p, -1.0, p, p, None, 0, None) == mlxq.ERR_INVALID
    assert f(p, 0, p, p, p, None, 4096, 4096, 64, 4, p, p, 1e-5, p, p, None, 0, None) == mlxq.OK
