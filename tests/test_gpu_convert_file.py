"""File-level GGUF -> MLX snapshot convert (mlxq::gguf::convert_file behind
bin/convert_gguf; the reference's gguf::convert, src/gguf/convert.rs:89-186,
and examples/convert_gguf.rs) on a small llama-shaped GGUF written by
tests/gguf_image.py.  Every stored tensor is compared bit for bit with the
oracle's restatement of the reference chain: dequantize (dequant.rs) ->
q/k un-permute (convert.rs:232-256) -> bf16 (convert.rs:156) -> MLX affine
quantize for projections (snapshot.rs:100-107)."""
import json
import subprocess
from pathlib import Path

import numpy as np
import pytest

import gguf_image as gi
import oracle as orc

pytestmark = pytest.mark.gpu

CLI = Path(__file__).resolve().parents[1] / "mlx-llm_amd" / "bin" / "convert_gguf"
H, HEADS, KV, FFN, VOCAB, LAYERS = 256, 4, 2, 512, 48, 2
# projection suffix -> (ggml type, torch shape); a mix of legacy, k-quant and IQ types
PROJ = {"attn_q": (12, (H, H)), "attn_k": (8, (KV * 64, H)), "attn_v": (20, (KV * 64, H)),
        "attn_output": (2, (H, H)), "ffn_gate": (23, (FFN, H)), "ffn_up": (14, (FFN, H)),
        "ffn_down": (12, (H, FFN))}
HF = {"attn_q": "self_attn.q_proj", "attn_k": "self_attn.k_proj", "attn_v": "self_attn.v_proj",
      "attn_output": "self_attn.o_proj", "ffn_gate": "mlp.gate_proj", "ffn_up": "mlp.up_proj",
      "ffn_down": "mlp.down_proj"}


def make_model(path, seed=0x6600, extra=()):
    tensors, src = [], {}
    w = orc.normal(seed, VOCAB * H, 0.0, 0.02)
    tensors.append(("token_embd.weight", [VOCAB, H], 1, w.astype(np.float16).view(np.uint8)))
    tensors.append(("output_norm.weight", [H], 0, orc.normal(seed + 1, H, 1.0, 0.1).view(np.uint8)))
    tensors.append(("output.weight", [VOCAB, H], 14, orc.gguf_quantize(14, orc.normal(seed + 2, VOCAB * H, 0, 0.02))))
    tensors.append(("rope_freqs.weight", [32], 0, np.ones(32, np.float32).view(np.uint8)))
    for i in range(LAYERS):
        for nm in ("attn_norm", "ffn_norm"):
            tensors.append((f"blk.{i}.{nm}.weight", [H], 0, orc.normal(seed + 10 * i + len(nm), H, 1, 0.1).view(np.uint8)))
        for j, (nm, (tag, shape)) in enumerate(PROJ.items()):
            data = orc.gguf_quantize(tag, orc.normal(seed + 100 * i + j + 50, shape[0] * shape[1], 0.0, 0.02))
            tensors.append((f"blk.{i}.{nm}.weight", list(shape), tag, data))
    for name, shape, tag, data in tensors:
        src[name] = (shape, tag, np.asarray(data, np.uint8))
    tensors += list(extra)
    meta = [("general.architecture", gi.STRING, "llama"), ("llama.embedding_length", gi.U32, H),
            ("llama.block_count", gi.U32, LAYERS), ("llama.attention.head_count", gi.U32, HEADS),
            ("llama.attention.head_count_kv", gi.U32, KV), ("llama.feed_forward_length", gi.U32, FFN),
            ("llama.attention.layer_norm_rms_epsilon", gi.F32, 1e-5), ("llama.rope.freq_base", gi.F32, 500000.0),
            ("llama.context_length", gi.U32, 8192), ("tokenizer.ggml.eos_token_id", gi.U32, 2),
            ("tokenizer.ggml.bos_token_id", gi.U32, 1)]
    gi.write(path, meta, tensors)
    return src


def load(out):
    from safetensors.torch import load_file

    import torch

    t = load_file(str(out / "model.safetensors"))
    res = {}
    for k, v in t.items():
        if v.dtype == torch.bfloat16:
            res[k] = v.view(torch.int16).numpy().view(np.uint16)
        elif v.dtype == torch.uint32:
            res[k] = v.numpy().view(np.uint32)
        else:
            res[k] = v.numpy()
    return res


def dense_bf16(shape, tag, data, heads=0):
    n = int(np.prod(shape))
    w = orc.gguf_dequantize(tag, data, n).reshape(shape)
    if heads:
        w = orc.permute_inverse_qk(w, heads)
    return orc.f32_to_bf16(w)


@pytest.mark.parametrize("quant", [None, "q4", "q8"])
def test_convert_file_matches_reference_chain(tmp_path, quant):
    gg = tmp_path / "m.gguf"
    src = make_model(gg)
    out = tmp_path / "snap"
    cmd = [str(CLI), str(gg), str(out)] + (["--quant", quant] if quant else [])
    print("convert:", " ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    cfg = json.loads((out / "config.json").read_text())
    assert cfg["model_type"] == "llama" and cfg["architectures"] == ["LlamaForCausalLM"]
    assert (cfg["hidden_size"], cfg["num_hidden_layers"], cfg["num_attention_heads"], cfg["num_key_value_heads"],
            cfg["intermediate_size"], cfg["head_dim"], cfg["vocab_size"]) == (H, LAYERS, HEADS, KV, FFN, 64, VOCAB)
    assert cfg["rms_norm_eps"] == float(np.float32(1e-5)) and cfg["rope_theta"] == 500000.0
    assert cfg["tie_word_embeddings"] is False and cfg["max_position_embeddings"] == 8192
    assert (cfg["eos_token_id"], cfg["bos_token_id"]) == (2, 1)
    bits = {"q4": 4, "q8": 8}.get(quant)
    if bits:
        assert cfg["quantization"] == {"group_size": 64, "bits": bits}
    else:
        assert "quantization" not in cfg
    st = load(out)
    want_keys = {"model.embed_tokens.weight", "model.norm.weight", "lm_head.weight"}
    for name, (shape, tag, data) in src.items():
        if name == "rope_freqs.weight":
            continue
        if name in ("token_embd.weight", "output_norm.weight", "output.weight"):
            key = {"token_embd.weight": "model.embed_tokens.weight", "output_norm.weight": "model.norm.weight",
                   "output.weight": "lm_head.weight"}[name]
            assert np.array_equal(st[key], dense_bf16(shape, tag, data)), key
            continue
        i, nm = name.split(".")[1], name.split(".")[2]
        if nm in ("attn_norm", "ffn_norm"):
            key = f"model.layers.{i}." + ("input_layernorm" if nm == "attn_norm" else "post_attention_layernorm") + ".weight"
            want_keys.add(key)
            assert np.array_equal(st[key], dense_bf16(shape, tag, data)), key
            continue
        base = f"model.layers.{i}.{HF[nm]}"
        heads = HEADS if nm == "attn_q" else KV if nm == "attn_k" else 0
        if bits:
            wq, s, b = orc.gguf_requantize(tag, data, shape[0], shape[1], heads, 64, bits)
            for suf, w in ((".weight", wq), (".scales", s), (".biases", b)):
                want_keys.add(base + suf)
                assert np.array_equal(st[base + suf].reshape(w.shape), w), base + suf
        else:
            want_keys.add(base + ".weight")
            assert np.array_equal(st[base + ".weight"], dense_bf16(shape, tag, data, heads)), base
    assert set(st) == want_keys


def test_convert_repeated_tensor_name_last_wins(tmp_path):
    """A GGUF naming one tensor twice: the snapshot holds the key once, with
    the later tensor's data (the reference collects the converted tensors
    by name, convert.rs:121-137)."""
    gg = tmp_path / "dup.gguf"
    tag, shape = PROJ["attn_q"]
    again = orc.gguf_quantize(tag, orc.normal(0x6677, shape[0] * shape[1], 0.0, 0.02))
    make_model(gg, extra=[("blk.0.attn_q.weight", list(shape), tag, again)])
    out = tmp_path / "snap"
    r = subprocess.run([str(CLI), str(gg), str(out), "--quant", "q4"], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    header_len = int.from_bytes((out / "model.safetensors").read_bytes()[:8], "little")
    header = json.loads((out / "model.safetensors").read_bytes()[8:8 + header_len])
    keys = [k for k in header if k != "__metadata__"]
    assert len(keys) == len(set(keys))
    st = load(out)
    wq, s, b = orc.gguf_requantize(tag, again, shape[0], shape[1], HEADS, 64, 4)
    base = "model.layers.0.self_attn.q_proj"
    for suf, w in ((".weight", wq), (".scales", s), (".biases", b)):
        assert np.array_equal(st[base + suf].reshape(w.shape), w), base + suf


def test_convert_rejects_oversized_tensor(tmp_path):
    """Dimensions whose product overflows 64 bits are refused by name, before
    anything is sized from the count."""
    gg = tmp_path / "big.gguf"
    meta = [("general.architecture", gi.STRING, "llama"), ("llama.embedding_length", gi.U32, 32),
            ("llama.block_count", gi.U32, 1), ("llama.attention.head_count", gi.U32, 1),
            ("llama.attention.head_count_kv", gi.U32, 1), ("llama.feed_forward_length", gi.U32, 32)]
    tensors = [("token_embd.weight", [1 << 40, 1 << 40], 0, np.zeros(64, np.uint8))]
    gi.write(gg, meta, tensors)
    r = subprocess.run([str(CLI), str(gg), str(tmp_path / "o")], capture_output=True, text=True, timeout=120)
    assert r.returncode != 0
    assert "tensor too large: token_embd.weight" in r.stderr, r.stderr
