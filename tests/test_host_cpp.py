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
    "q6_k_centered_is_zero", "dequantize_errors", "iq2_xxs_grid_scale_and_offset", "iq2_xs_and_s_grid_zero_decode",
    "iq3_xxs_and_s_grid_zero_decode", "iq1_s_signed_grid_and_scale", "iq1_m_packed_f16_scale",
    "requantize_projection_undoes_qk_permute",
    "projection_predicate_selects_only_attn_mlp_projections", "dense_write_round_trips_bit_identical",
    "quantized_write_loads_through_prequantized_branch",
    "gguf_parse_minimal_roundtrip", "gguf_rejects_bad_magic_and_v1", "gguf_parses_int_float_array_metadata",
    "gguf_reader_errors_and_alignment", "gguf_remap_keys_and_ignorables", "gguf_convert_refuses_before_decoding",
    "safetensors_rejects_malformed_headers",
]


def test_host_only_cases_pass_on_cpu():
    """The host-only cases (GGUF reader and convert refusals, safetensors
    header checks, the projection predicate) run here without a GPU."""
    r = subprocess.run([str(BIN), "--cpu"], capture_output=True, text=True, timeout=120)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "8 cases, 0 failed" in r.stdout


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


@pytest.mark.gpu
def test_safetensors_interop(tmp_path):
    """A file the safetensors package writes (every dtype the snapshot uses,
    with metadata) loads through the C++ reader, and what the C++ writer
    saves loads back in the package bit-identical."""
    import torch
    from safetensors.torch import load_file, save_file

    g = torch.Generator().manual_seed(7)
    src = {
        "a.weight": torch.randint(0, 2**31 - 1, (6, 8), generator=g, dtype=torch.int64).to(torch.uint32),
        "a.scales": torch.randn(6, 2, generator=g).to(torch.bfloat16),
        "a.biases": torch.randn(6, 2, generator=g).to(torch.float16),
        "norm.weight": torch.randn(5, generator=g),
        "tok": torch.randint(0, 255, (3, 7), generator=g, dtype=torch.uint8),
        "scalar_row": torch.randn(1, 1, generator=g),
    }
    fin, fout = tmp_path / "in.safetensors", tmp_path / "out.safetensors"
    save_file(src, str(fin), metadata={"format": "pt", "note": "{\\\"x\\\": [1, 2]}"})
    r = subprocess.run([str(BIN), "--copy-safetensors", str(fin), str(fout)], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    back = load_file(str(fout))
    assert sorted(back) == sorted(src)
    for k, v in src.items():
        assert back[k].dtype == v.dtype and back[k].shape == v.shape, k
        assert torch.equal(back[k].view(torch.uint8), v.view(torch.uint8)), k
