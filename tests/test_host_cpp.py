"""The C++ host API (mlx-llm_amd/host/mlxq.hpp) and the C++ restatement of the
reference's own tests (tests/cpp/host_tests.cpp): the binary is built by
build() and lists its cases without touching a GPU; on a GPU every case
passes (the reference's inputs and expected values, run on the kernels)."""
import subprocess
from pathlib import Path

import pytest

BIN = Path(__file__).resolve().parents[1] / "mlx-llm_amd" / "bin" / "host_tests"
CASES = [
    "quantize_dequantize_roundtrip_q8", "quantized_matmul_approximates_linear_q8", "projection_load_and_dispatch",
    "type_geometry_matches_llama_cpp", "supported_and_unsupported_types", "iq4_nl_codebook_decode",
    "f32_f16_bf16_passthrough", "q8_0_block_dequant", "q4_0_zero_centered", "q2_k_scale_and_unpack",
    "q6_k_centered_is_zero", "dequantize_errors", "requantize_projection_undoes_qk_permute",
]


def test_host_tests_built_and_listed():
    assert BIN.is_file(), "run build() first"
    r = subprocess.run([str(BIN), "--list"], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stderr
    assert r.stdout.split() == CASES


@pytest.mark.gpu
def test_host_tests_pass_on_gpu():
    r = subprocess.run([str(BIN)], capture_output=True, text=True, timeout=120)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    for c in CASES:
        assert f"ok {c}" in r.stdout
