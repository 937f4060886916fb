"""numpy/ctypes wrapper of liboracle.so -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may use
this module, as the checker or as the timed CPU baseline.  The product
(mlx-llm_amd/libmlxq.so) never calls it.
"""
from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"

_lib = None
_P = ctypes.c_void_p
_i64 = ctypes.c_int64


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        L = ctypes.CDLL(str(LIB_PATH))
        L.orc_splitmix64_next.restype = ctypes.c_uint64
        L.orc_splitmix64_next.argtypes = [ctypes.POINTER(ctypes.c_uint64)]
        L.orc_splitmix64_next_f32.restype = ctypes.c_float
        L.orc_splitmix64_next_f32.argtypes = [ctypes.POINTER(ctypes.c_uint64)]
        L.orc_gen_normal_f32.restype = None
        L.orc_gen_normal_f32.argtypes = [ctypes.c_uint64, ctypes.c_float, ctypes.c_float, _P, ctypes.c_size_t]
        L.orc_f16_to_f32.restype = ctypes.c_float
        L.orc_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.orc_f32_to_f16.restype = ctypes.c_uint16
        L.orc_f32_to_f16.argtypes = [ctypes.c_float]
        L.orc_f32_to_bf16.restype = ctypes.c_uint16
        L.orc_f32_to_bf16.argtypes = [ctypes.c_float]
        L.orc_bf16_to_f32.restype = ctypes.c_float
        L.orc_bf16_to_f32.argtypes = [ctypes.c_uint16]
        L.orc_gguf_block.argtypes = [ctypes.c_uint32, ctypes.POINTER(_i64), ctypes.POINTER(_i64)]
        L.orc_gguf_tensor_byte_len.argtypes = [ctypes.c_uint32, _i64, ctypes.POINTER(_i64)]
        L.orc_gguf_dequantize.argtypes = [ctypes.c_uint32, _P, _i64, _i64, _P]
        L.orc_gguf_dequantize_mt.argtypes = [ctypes.c_uint32, _P, _i64, _i64, _P, ctypes.c_int]
        L.orc_gguf_quantize.argtypes = [ctypes.c_uint32, _P, _i64, _P]
        L.orc_ksigns_iq2xs.restype = ctypes.c_uint8
        L.orc_ksigns_iq2xs.argtypes = [ctypes.c_int]
        L.orc_iq_grid.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.POINTER(ctypes.c_uint64)]
        L.orc_affine_quantize.argtypes = [ctypes.c_int, _P, _i64, _i64, ctypes.c_int, ctypes.c_int, _P, _P, _P]
        L.orc_affine_dequantize.argtypes = [ctypes.c_int, _P, _P, _P, _i64, _i64, ctypes.c_int, ctypes.c_int, _P]
        L.orc_qmatmul_f64.argtypes = [_P, _i64, _P, _P, _P, _i64, _i64, ctypes.c_int, ctypes.c_int, _P]
        L.orc_qmatmul_f32.argtypes = [_P, _i64, _P, _P, _P, _i64, _i64, ctypes.c_int, ctypes.c_int, _P, ctypes.c_int]
        L.orc_rms_norm_bf16.argtypes = [_P, _P, _i64, _i64, ctypes.c_float, _P]
        L.orc_silu_mul_bf16.argtypes = [_P, _P, _i64, _P]
        L.orc_add_bf16.argtypes = [_P, _P, _i64, _P]
        L.orc_repeat_kv.argtypes = [_P, _i64, ctypes.c_int, ctypes.c_int, ctypes.c_int, _P]
        _lib = L
    return _lib


class OracleError(RuntimeError):
    def __init__(self, rc):
        super().__init__(f"oracle status {rc}")
        self.status = rc


def _chk(rc):
    if rc:
        raise OracleError(rc)


def _p(a: np.ndarray):
    assert a.flags.c_contiguous
    return a.ctypes.data_as(ctypes.c_void_p)


# ---------------------------------------------------------------- generators
def splitmix64(seed: int, n: int) -> np.ndarray:
    st = ctypes.c_uint64(seed)
    return np.array([lib().orc_splitmix64_next(ctypes.byref(st)) for _ in range(n)], dtype=np.uint64)


def normal(seed: int, n: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    lib().orc_gen_normal_f32(seed, mean, std, _p(out), n)
    return out


# ---------------------------------------------------------------- conversions
def f32_to_bf16(a: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even f32 -> bf16 bits (vectorized; same rule as orc_f32_to_bf16)."""
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def bf16_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


# ---------------------------------------------------------------- GGUF
def gguf_block(tag: int):
    e, b = _i64(0), _i64(0)
    _chk(lib().orc_gguf_block(tag, ctypes.byref(e), ctypes.byref(b)))
    return e.value, b.value


def gguf_tensor_byte_len(tag: int, n: int) -> int:
    b = _i64(0)
    _chk(lib().orc_gguf_tensor_byte_len(tag, n, ctypes.byref(b)))
    return b.value


def gguf_dequantize(tag: int, data: np.ndarray, n: int, threads: int = 1) -> np.ndarray:
    data = np.ascontiguousarray(data, dtype=np.uint8)
    out = np.empty(n, dtype=np.float32)
    if threads > 1:
        _chk(lib().orc_gguf_dequantize_mt(tag, _p(data), data.size, n, _p(out), threads))
    else:
        _chk(lib().orc_gguf_dequantize(tag, _p(data), data.size, n, _p(out)))
    return out


IQ_GRIDS = {"iq2xxs": 0, "iq2xs": 1, "iq2s": 2, "iq3xxs": 3, "iq3s": 4, "iq1s": 5}


def iq_grid(name: str) -> np.ndarray:
    """A GGUF IQ codebook as stored (uint64 entries; the 4-byte grids in the
    low 32 bits)."""
    t = IQ_GRIDS[name]
    n = lib().orc_iq_grid(t, 0, None)
    out = np.empty(n, dtype=np.uint64)
    v = ctypes.c_uint64(0)
    for i in range(n):
        assert lib().orc_iq_grid(t, i, ctypes.byref(v)) == n
        out[i] = v.value
    return out


def ksigns_iq2xs() -> np.ndarray:
    return np.array([lib().orc_ksigns_iq2xs(i) for i in range(128)], dtype=np.uint8)


def gguf_quantize(tag: int, x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32).ravel()
    out = np.zeros(gguf_tensor_byte_len(tag, x.size), dtype=np.uint8)
    _chk(lib().orc_gguf_quantize(tag, _p(x), x.size, _p(out)))
    return out


# ---------------------------------------------------------------- affine
F32, BF16 = 0, 2


def affine_quantize(w: np.ndarray, group_size: int = 64, bits: int = 4, dtype: int = BF16):
    """w: [rows, cols] float32 (dtype F32) or uint16 bf16 bits (dtype BF16)."""
    w = np.ascontiguousarray(w)
    rows, cols = w.shape
    wq = np.empty((rows, cols * bits // 32), dtype=np.uint32)
    sd = np.float32 if dtype == F32 else np.uint16
    s = np.empty((rows, cols // group_size), dtype=sd)
    b = np.empty_like(s)
    _chk(lib().orc_affine_quantize(dtype, _p(w), rows, cols, group_size, bits, _p(wq), _p(s), _p(b)))
    return wq, s, b


def affine_dequantize(wq, s, b, group_size: int = 64, bits: int = 4, dtype: int = BF16):
    rows = wq.shape[0]
    cols = wq.shape[1] * 32 // bits
    out = np.empty((rows, cols), dtype=np.float32 if dtype == F32 else np.uint16)
    _chk(lib().orc_affine_dequantize(dtype, _p(np.ascontiguousarray(wq)), _p(np.ascontiguousarray(s)),
                                     _p(np.ascontiguousarray(b)), rows, cols, group_size, bits, _p(out)))
    return out


def qmatmul_f64(x_bf16, wq, s_bf16, b_bf16, group_size: int = 64, bits: int = 4) -> np.ndarray:
    x_bf16 = np.ascontiguousarray(x_bf16, dtype=np.uint16)
    m, k = x_bf16.shape
    n = wq.shape[0]
    y = np.empty((m, n), dtype=np.float64)
    _chk(lib().orc_qmatmul_f64(_p(x_bf16), m, _p(np.ascontiguousarray(wq)), _p(np.ascontiguousarray(s_bf16)),
                               _p(np.ascontiguousarray(b_bf16)), n, k, group_size, bits, _p(y)))
    return y


def qmatmul_f32(x_bf16, wq, s_bf16, b_bf16, group_size: int = 64, bits: int = 4, threads: int = 1) -> np.ndarray:
    x_bf16 = np.ascontiguousarray(x_bf16, dtype=np.uint16)
    m, k = x_bf16.shape
    n = wq.shape[0]
    y = np.empty((m, n), dtype=np.float32)
    _chk(lib().orc_qmatmul_f32(_p(x_bf16), m, _p(np.ascontiguousarray(wq)), _p(np.ascontiguousarray(s_bf16)),
                               _p(np.ascontiguousarray(b_bf16)), n, k, group_size, bits, _p(y), threads))
    return y


# ---------------------------------------------------------------- decode layer chain
def _u16(a):
    return np.ascontiguousarray(a, dtype=np.uint16)


def rms_norm(x_bf16, w_bf16, eps: float) -> np.ndarray:
    x = _u16(x_bf16)
    y = np.empty_like(x)
    d = x.shape[-1]
    _chk(lib().orc_rms_norm_bf16(_p(x), _p(_u16(w_bf16)), x.size // d, d, eps, _p(y)))
    return y


def silu_mul(g_bf16, u_bf16) -> np.ndarray:
    g, u = _u16(g_bf16), _u16(u_bf16)
    y = np.empty_like(g)
    _chk(lib().orc_silu_mul_bf16(_p(g), _p(u), g.size, _p(y)))
    return y


def add(a_bf16, b_bf16) -> np.ndarray:
    a, b = _u16(a_bf16), _u16(b_bf16)
    y = np.empty_like(a)
    _chk(lib().orc_add_bf16(_p(a), _p(b), a.size, _p(y)))
    return y


def repeat_kv(x_bf16, kv_heads: int, head_dim: int, groups: int) -> np.ndarray:
    x = _u16(x_bf16)
    rows = x.size // (kv_heads * head_dim)
    y = np.empty((rows, kv_heads * groups * head_dim), dtype=np.uint16)
    _chk(lib().orc_repeat_kv(_p(x), rows, kv_heads, head_dim, groups, _p(y)))
    return y


def qlinear_bf16(x_bf16, w, group_size: int, bits: int) -> np.ndarray:
    """A quantized projection with its bf16 output rounding (f64 sums -> f32 -> bf16)."""
    wq, s, b = w
    y = qmatmul_f64(x_bf16, wq, s, b, group_size, bits)
    return f32_to_bf16(y.astype(np.float32))


def decode_layer(x_bf16, L, cfg) -> np.ndarray:
    """One layer of the chain below (src/models/llama.rs:689-735 with the
    identity attention): bf16 hidden state [M, hidden] in and out."""
    gs, bits, eps = cfg["group_size"], cfg["bits"], cfg["eps"]
    groups = cfg["heads"] // cfg["kv_heads"]
    x = _u16(x_bf16)
    n1 = rms_norm(x, L["ln1"], eps)
    # q and k only feed attention, which the chain replaces: no effect on the output
    v = qlinear_bf16(n1, L["v"], gs, bits)
    attn = repeat_kv(v, cfg["kv_heads"], cfg["head_dim"], groups)
    h = add(x, qlinear_bf16(attn, L["o"], gs, bits))
    n2 = rms_norm(h, L["ln2"], eps)
    a = silu_mul(qlinear_bf16(n2, L["gate"], gs, bits), qlinear_bf16(n2, L["up"], gs, bits))
    return add(h, qlinear_bf16(a, L["down"], gs, bits))


def decode_head(x_bf16, final_norm, lm_head, cfg) -> np.ndarray:
    """Final norm and lm_head (src/models/llama.rs:595-603): bf16 logits."""
    return qlinear_bf16(rms_norm(_u16(x_bf16), final_norm, cfg["eps"]), lm_head, cfg["group_size"], cfg["bits"])


def decode_stack(x_bf16, layers, final_norm, lm_head, cfg) -> np.ndarray:
    """One decode step of the quantized Llama layer chain with attention replaced
    by the identity on v (GQA heads repeated): src/models/llama.rs:689-735
    (layer), :806-835 (q/k/v/o), :1040-1045 (MLP), :595-603 (final norm and
    lm_head).  layers: dicts with packed (wq, scales, biases) numpy triples
    under q, k, v, o, gate, up, down and bf16 norm weights ln1, ln2.
    Returns bf16 logits [M, vocab]."""
    x = _u16(x_bf16)
    for L in layers:
        x = decode_layer(x, L, cfg)
    return decode_head(x, final_norm, lm_head, cfg)


def permute_inverse_qk(w: np.ndarray, n_head: int) -> np.ndarray:
    """src/gguf/convert.rs:232-256: undo llama.cpp's q/k row interleave of a
    [out, in] weight: HF row r = k*(hd/2) + j of a head comes from GGUF row
    2*j + k."""
    out = w.shape[0]
    hd = out // n_head
    half = hd // 2
    r = np.arange(out)
    h, rr = r // hd, r % hd
    src = h * hd + 2 * (rr % half) + rr // half
    return w[src]


def gguf_requantize(tag: int, data: np.ndarray, rows: int, cols: int, permute_heads: int = 0,
                    group_size: int = 64, bits: int = 4):
    """The reference convert chain for one projection (convert.rs:131-176):
    dequantize -> q/k un-permute -> bf16 -> MLX affine quantize of the bf16 tensor."""
    w = gguf_dequantize(tag, data, rows * cols).reshape(rows, cols)
    if permute_heads:
        w = permute_inverse_qk(w, permute_heads)
    return affine_quantize(f32_to_bf16(w), group_size, bits, BF16)
