"""GGUF container reader (mlxq::gguf::GgufFile, src/gguf/reader.rs:180-298)
on files written by an independent writer (tests/gguf_image.py), through
the converter's --inspect mode: no GPU."""
import json
import subprocess
from pathlib import Path

import numpy as np

import gguf_image as gi

CLI = Path(__file__).resolve().parents[1] / "mlx-llm_amd" / "bin" / "convert_gguf"


def inspect(path):
    r = subprocess.run([str(CLI), "--inspect", str(path)], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stderr
    return json.loads(r.stdout)


def test_inspect_shapes_types_offsets(tmp_path):
    meta = [("general.architecture", gi.STRING, "llama"), ("general.alignment", gi.U32, 64),
            ("llama.block_count", gi.U32, 1), ("tokenizer.ggml.tokens", gi.ARRAY, (gi.STRING, ["a", "b", "c"])),
            ("x.f64", gi.F64, 0.25), ("x.i8", gi.I8, -3), ("x.bool", gi.BOOL, True)]
    tensors = [("token_embd.weight", [5, 32], 0, np.zeros(5 * 32 * 4, np.uint8)),
               ("blk.0.attn_q.weight", [32, 32], 8, np.zeros(32 * 34, np.uint8)),   # Q8_0: 32 blocks x 34 B
               ("blk.0.ffn_up.weight", [2, 3, 4, 256], 12, np.zeros(24 * 144, np.uint8))]  # 4-D, Q4_K
    p = tmp_path / "m.gguf"
    gi.write(p, meta, tensors, alignment=64)
    h = inspect(p)
    assert h["alignment"] == 64 and h["data_start"] % 64 == 0
    assert sorted(h["metadata_keys"]) == sorted(k for k, _, _ in meta)
    got = [(t["name"], t["shape"], t["type"]) for t in h["tensors"]]
    assert got == [(n, s, t) for n, s, t, _ in tensors]  # ne reversed back to torch order
    offs = [t["offset"] for t in h["tensors"]]
    assert offs == [0, 640, (640 + 1088 + 63) // 64 * 64]


def test_inspect_rejects_v1_and_bad_magic(tmp_path):
    p = tmp_path / "v1.gguf"
    p.write_bytes((0x46554747).to_bytes(4, "little") + (1).to_bytes(4, "little") + bytes(16))
    r = subprocess.run([str(CLI), "--inspect", str(p)], capture_output=True, text=True, timeout=60)
    assert r.returncode == 1 and "only v2/v3" in r.stderr
    p.write_bytes(bytes(24))
    r = subprocess.run([str(CLI), "--inspect", str(p)], capture_output=True, text=True, timeout=60)
    assert r.returncode == 1 and "bad magic" in r.stderr
