"""ctypes binding of libmlxq.so (the C ABI in include/mlxq.h).

This is test / benchmark plumbing: torch supplies device memory and the
current HIP stream, every computation runs in the HIP kernels of
libmlxq.so.  There is no fallback: if the library is missing, importing
`lib()` raises.

The function names mirror the reference crate's boundary:
  quantize            <- QuantizedLinear::quantize   (src/primitives/quant.rs:38-53)
  dequantize          <- QuantizedLinear::dequantize_weight (quant.rs:73-81)
  qmatmul             <- QuantizedLinear::forward    (quant.rs:56-70)
  gguf_dequantize     <- gguf::dequant::dequantize   (src/gguf/dequant.rs:156-211)
  gguf_block / gguf_tensor_byte_len <- GgmlType::block / tensor_byte_len (dequant.rs:116-153)
"""
from __future__ import annotations

import ctypes
import threading
from pathlib import Path

LIB_PATH = Path(__file__).resolve().with_name("libmlxq.so")

OK, ERR_INVALID, ERR_SHAPE, ERR_UNSUPPORTED, ERR_SHORT_BUFFER, ERR_WORKSPACE, ERR_DEVICE = range(7)
F32, F16, BF16 = 0, 1, 2
ALGO_AUTO, ALGO_QMV, ALGO_QMM, ALGO_QMM_LIB = 0, 1, 2, 3

# GGUF type tags (dequant.rs:85-108)
GGUF_TAGS = {
    "F32": 0, "F16": 1, "Q4_0": 2, "Q4_1": 3, "Q5_0": 6, "Q5_1": 7, "Q8_0": 8,
    "Q2_K": 10, "Q3_K": 11, "Q4_K": 12, "Q5_K": 13, "Q6_K": 14, "IQ2_XXS": 16,
    "IQ2_XS": 17, "IQ3_XXS": 18, "IQ1_S": 19, "IQ4_NL": 20, "IQ3_S": 21,
    "IQ2_S": 22, "IQ4_XS": 23, "IQ1_M": 29, "BF16": 30,
}

# Every symbol include/mlxq.h declares, with its ctypes signature.
_i64, _u32, _vp, _sz = ctypes.c_int64, ctypes.c_uint32, ctypes.c_void_p, ctypes.c_size_t
SIGNATURES = {
    "mlxq_last_error": (ctypes.c_char_p, []),
    "mlxq_version": (ctypes.c_char_p, []),
    "mlxq_reload_overrides": (ctypes.c_int, []),
    "mlxq_quantize": (ctypes.c_int, [_vp, ctypes.c_int, _i64, _i64, ctypes.c_int, ctypes.c_int, _vp, _vp, _vp, _vp]),
    "mlxq_dequantize": (ctypes.c_int, [_vp, _vp, _vp, ctypes.c_int, _i64, _i64, ctypes.c_int, ctypes.c_int, _vp, _vp]),
    "mlxq_qmatmul_workspace_size": (ctypes.c_int, [_i64, _i64, _i64, ctypes.c_int, ctypes.c_int, ctypes.POINTER(_sz)]),
    "mlxq_qmatmul": (ctypes.c_int, [_vp, _i64, _vp, _vp, _vp, _vp, _i64, _i64, ctypes.c_int, ctypes.c_int, _vp, _vp, _sz, _vp]),
    "mlxq_qmatmul_algo": (ctypes.c_int, [_vp, _i64, _vp, _vp, _vp, _vp, _i64, _i64, ctypes.c_int, ctypes.c_int, _vp, _vp, _sz, ctypes.c_int, _vp]),
    "mlxq_qmatmul_noalloc": (ctypes.c_int, [_vp, _i64, _vp, _vp, _vp, _vp, _i64, _i64, ctypes.c_int, ctypes.c_int,
                                            _vp, _vp]),
    "mlxq_qmatmul_noalloc_max_scratch": (_sz, []),
    "mlxq_qmatmul_route": (ctypes.c_int, [_i64, _i64, _i64, ctypes.c_int, ctypes.c_int, _sz, ctypes.c_int, ctypes.c_int,
                                          ctypes.c_char_p, _sz]),
    "mlxq_qmatmul_fused": (ctypes.c_int, [_vp, _i64, _i64, _vp, ctypes.c_float, ctypes.c_int, ctypes.c_int,
                                          ctypes.c_int, _vp, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                          ctypes.c_int, _vp]),
    "mlxq_qmatmul_add_rms_norm": (ctypes.c_int, [_vp, _i64, _vp, _vp, _vp, _vp, _i64, _i64, ctypes.c_int,
                                                 ctypes.c_int, _vp, _vp, ctypes.c_float, _vp, _vp, _vp, _sz, _vp]),
    "mlxq_rms_norm": (ctypes.c_int, [_vp, _vp, _i64, _i64, ctypes.c_float, _vp, _vp]),
    "mlxq_silu_mul": (ctypes.c_int, [_vp, _vp, _i64, _vp, _vp]),
    "mlxq_add": (ctypes.c_int, [_vp, _vp, _i64, _vp, _vp]),
    "mlxq_add_rms_norm": (ctypes.c_int, [_vp, _vp, _vp, _i64, _i64, ctypes.c_float, _vp, _vp, _vp]),
    "mlxq_repeat_kv": (ctypes.c_int, [_vp, _i64, ctypes.c_int, ctypes.c_int, ctypes.c_int, _vp, _vp]),
    "mlxq_gguf_requantize": (ctypes.c_int, [_u32, _vp, _i64, _i64, _i64, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                            _vp, _vp, _vp, _vp]),
    "mlxq_gguf_block": (ctypes.c_int, [_u32, ctypes.POINTER(_i64), ctypes.POINTER(_i64)]),
    "mlxq_gguf_tensor_byte_len": (ctypes.c_int, [_u32, _i64, ctypes.POINTER(_i64)]),
    "mlxq_gguf_dequantize": (ctypes.c_int, [_u32, _vp, _i64, _i64, ctypes.c_int, _vp, _vp]),
}


class Projection(ctypes.Structure):
    """mlxq_projection (include/mlxq.h)."""
    _fields_ = [("wq", _vp), ("scales", _vp), ("biases", _vp), ("bias", _vp), ("residual", _vp), ("y", _vp),
                ("N", _i64)]


class MlxqError(RuntimeError):
    """A failing mlxq call (the reference's Error::Msg / Error::Mlx)."""

    def __init__(self, status: int, msg: str):
        super().__init__(msg)
        self.status = status


class Unsupported(MlxqError):
    """MLXQ_ERR_UNSUPPORTED (the reference's Error::Unsupported)."""


_lib = None
_lock = threading.Lock()


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        with _lock:
            if _lib is None:
                if not LIB_PATH.exists():
                    raise ImportError(f"{LIB_PATH} is not built; run `python mlx-llm_amd/build.py`")
                L = ctypes.CDLL(str(LIB_PATH))
                for name, (res, args) in SIGNATURES.items():
                    f = getattr(L, name)
                    f.restype = res
                    f.argtypes = args
                _lib = L
    return _lib


def check(rc: int) -> None:
    if rc != OK:
        msg = lib().mlxq_last_error().decode()
        raise (Unsupported if rc == ERR_UNSUPPORTED else MlxqError)(rc, msg)


def version() -> str:
    return lib().mlxq_version().decode()


def check_build() -> None:
    """Refuse a libmlxq.so built from sources other than this tree's (a
    stale build pushed with newer sources): RuntimeError naming both hashes."""
    from provenance import library_hash, source_hash

    have, want = library_hash(version()), source_hash()
    if have != want:
        raise RuntimeError(f"{LIB_PATH} was built from other sources (library src={have}, tree src={want}); "
                           "rebuild with `python mlx-llm_amd/build.py`")


def reload_overrides() -> None:
    """Re-read the MLXQ_* kernel-override environment variables (read once otherwise)."""
    check(lib().mlxq_reload_overrides())


# ---------------------------------------------------------------- torch glue
def _torch():
    import torch

    return torch


def _stream():
    return _torch().cuda.current_stream().cuda_stream


def _ptr(t):
    return None if t is None else t.data_ptr()


def _dtype_code(dt) -> int:
    torch = _torch()
    if dt == torch.float32:
        return F32
    if dt == torch.bfloat16:
        return BF16
    if dt == torch.float16:
        return F16
    raise Unsupported(ERR_UNSUPPORTED, f"unsupported dtype {dt}")


def quantize(w, group_size: int = 64, bits: int = 4):
    """(wq uint32 [N, K*bits/32] as int32, scales, biases [N, K/group]) in w's dtype."""
    torch = _torch()
    assert w.is_cuda and w.is_contiguous() and w.dim() == 2
    n, k = w.shape
    wq = torch.empty((n, k * bits // 32), dtype=torch.int32, device=w.device)
    s = torch.empty((n, k // group_size), dtype=w.dtype, device=w.device)
    b = torch.empty_like(s)
    check(lib().mlxq_quantize(_ptr(w), _dtype_code(w.dtype), n, k, group_size, bits,
                              _ptr(wq), _ptr(s), _ptr(b), _stream()))
    return wq, s, b


def dequantize(wq, scales, biases, group_size: int = 64, bits: int = 4):
    torch = _torch()
    n = wq.shape[0]
    k = wq.shape[1] * 32 // bits
    out = torch.empty((n, k), dtype=scales.dtype, device=wq.device)
    check(lib().mlxq_dequantize(_ptr(wq), _ptr(scales), _ptr(biases), _dtype_code(scales.dtype), n, k,
                                group_size, bits, _ptr(out), _stream()))
    return out


def workspace_size(m: int, n: int, k: int, group_size: int = 64, bits: int = 4) -> int:
    out = ctypes.c_size_t(0)
    check(lib().mlxq_qmatmul_workspace_size(m, n, k, group_size, bits, ctypes.byref(out)))
    return out.value


_ws = {}
_ws_retired = []


def workspace(nbytes: int, device):
    """A per-device qmatmul workspace (scratch for split-K partial sums),
    grown on demand.  A workspace that is outgrown is kept alive, not freed:
    work already queued or captured in a HIP graph may still use it."""
    torch = _torch()
    key = str(device)
    cur = _ws.get(key)
    if cur is None or cur.numel() < nbytes:
        if cur is not None:
            _ws_retired.append(cur)
        cur = torch.zeros(max(nbytes, 1 << 20), dtype=torch.uint8, device=device)
        _ws[key] = cur
    return cur


def qmatmul(x, wq, scales, biases, group_size: int = 64, bits: int = 4, bias=None, algo: int = ALGO_AUTO,
            out=None):
    """y = x @ dequant(W).T (+ bias); x [..., K] bf16 -> y [..., N] bf16."""
    torch = _torch()
    k = x.shape[-1]
    n = wq.shape[0]
    x2 = x.reshape(-1, k)
    assert x2.is_contiguous()
    m = x2.shape[0]
    y = out if out is not None else torch.empty((m, n), dtype=torch.bfloat16, device=x.device)
    nbytes = workspace_size(m, n, k, group_size, bits)
    ws = workspace(nbytes, x.device) if nbytes else None
    check(lib().mlxq_qmatmul_algo(_ptr(x2), m, _ptr(wq), _ptr(scales), _ptr(biases), _ptr(bias), n, k,
                                  group_size, bits, _ptr(y), _ptr(ws), 0 if ws is None else ws.numel(),
                                  algo, _stream()))
    return y.reshape(*x.shape[:-1], n)


def qmatmul_route(m: int, n: int, k: int, group_size: int = 64, bits: int = 4, algo: int = ALGO_AUTO,
                  workspace_bytes=None, noalloc: bool = False) -> str:
    """The kernels a qmatmul call of this shape launches (the library's own
    dispatch, run with launches suppressed), e.g. "qmm_kernel<4, 64, 4, 2> +
    tile::split_reduce4_kernel<4>"; workspace_bytes defaults to what
    workspace_size() asks for."""
    if workspace_bytes is None:
        workspace_bytes = workspace_size(m, n, k, group_size, bits)
    buf = ctypes.create_string_buffer(1024)
    check(lib().mlxq_qmatmul_route(m, n, k, group_size, bits, workspace_bytes, algo, int(noalloc), buf, len(buf)))
    return buf.value.decode()


def bind_qmatmul(x, wq, scales, biases, group_size: int = 64, bits: int = 4, out=None, bias=None,
                 algo: int = ALGO_AUTO):
    """Pre-resolve every pointer of one qmatmul call and return a zero-argument
    callable that launches it on the then-current stream (for tight loops and
    HIP-graph capture; the workspace is allocated here, never in the call)."""
    torch = _torch()
    k = x.shape[-1]
    n = wq.shape[0]
    m = x.numel() // k
    y = out if out is not None else torch.empty((m, n), dtype=torch.bfloat16, device=x.device)
    nbytes = workspace_size(m, n, k, group_size, bits)
    ws = workspace(nbytes, x.device) if nbytes else None
    f = lib().mlxq_qmatmul_algo
    args = (_ptr(x), m, _ptr(wq), _ptr(scales), _ptr(biases), _ptr(bias), n, k, group_size, bits, _ptr(y),
            _ptr(ws), 0 if ws is None else ws.numel(), algo)
    cs = torch.cuda.current_stream

    def call():
        rc = f(*args, cs().cuda_stream)
        if rc:
            check(rc)
        return y

    call.out = y
    call.workspace = ws
    return call


def qmatmul_fused(x, projs, group_size: int = 64, bits: int = 4, norm_weight=None, eps: float = 0.0,
                  repeat=None, swiglu: bool = False):
    """One fused decode launch (mlxq_qmatmul_fused).  projs: list of dicts with
    wq, scales, biases, y and optional bias / residual (device tensors);
    repeat: (kv_heads, head_dim, groups) for a GQA head-repeated input.
    Raises Unsupported for shapes outside the fused decode kernel."""
    k = x.shape[-1] * (repeat[2] if repeat else 1)
    m = x.numel() // x.shape[-1]
    arr = (Projection * len(projs))()
    for i, p in enumerate(projs):
        arr[i] = Projection(_ptr(p["wq"]), _ptr(p["scales"]), _ptr(p["biases"]), _ptr(p.get("bias")),
                            _ptr(p.get("residual")), _ptr(p["y"]), p["wq"].shape[0])
    kvh, hd, groups = repeat if repeat else (0, 0, 1)
    check(lib().mlxq_qmatmul_fused(_ptr(x), m, k, _ptr(norm_weight), eps, kvh, hd, groups, arr, len(projs),
                                   int(swiglu), group_size, bits, _stream()))
    return projs[0]["y"]


def rms_norm(x, weight, eps: float, out=None):
    """MLX fast::rms_norm over the last axis (bf16)."""
    torch = _torch()
    d = x.shape[-1]
    y = out if out is not None else torch.empty_like(x)
    check(lib().mlxq_rms_norm(_ptr(x), _ptr(weight), x.numel() // d, d, eps, _ptr(y), _stream()))
    return y


def add_rms_norm(a, b, weight, eps: float, sum_out=None, out=None):
    """sum = a + b (bf16, as add), y = rms_norm(sum) (as rms_norm), one launch."""
    torch = _torch()
    d = a.shape[-1]
    s = sum_out if sum_out is not None else torch.empty_like(a)
    y = out if out is not None else torch.empty_like(a)
    check(lib().mlxq_add_rms_norm(_ptr(a), _ptr(b), _ptr(weight), a.numel() // d, d, eps, _ptr(s), _ptr(y),
                                  _stream()))
    return s, y


def qmatmul_add_rms_norm(x, wq, scales, biases, residual, weight, eps: float, group_size: int = 64, bits: int = 4,
                         bias=None, sum_out=None, out=None):
    """sum = residual + qmatmul(x) (bf16, as add), y = rms_norm(sum); the
    split-K sum, the add and the norm share one launch where K is split."""
    torch = _torch()
    k = x.shape[-1]
    n = wq.shape[0]
    x2 = x.reshape(-1, k)
    m = x2.shape[0]
    s = sum_out if sum_out is not None else torch.empty((m, n), dtype=torch.bfloat16, device=x.device)
    y = out if out is not None else torch.empty((m, n), dtype=torch.bfloat16, device=x.device)
    nbytes = workspace_size(m, n, k, group_size, bits)
    ws = workspace(nbytes, x.device) if nbytes else None
    check(lib().mlxq_qmatmul_add_rms_norm(_ptr(x2), m, _ptr(wq), _ptr(scales), _ptr(biases), _ptr(bias), n, k,
                                          group_size, bits, _ptr(residual), _ptr(weight), eps, _ptr(s), _ptr(y),
                                          _ptr(ws), 0 if ws is None else ws.numel(), _stream()))
    return s, y


def silu_mul(gate, up, out=None):
    """silu(gate) * up with MLX's bf16 rounding points."""
    torch = _torch()
    y = out if out is not None else torch.empty_like(gate)
    check(lib().mlxq_silu_mul(_ptr(gate), _ptr(up), gate.numel(), _ptr(y), _stream()))
    return y


def add(a, b, out=None):
    torch = _torch()
    y = out if out is not None else torch.empty_like(a)
    check(lib().mlxq_add(_ptr(a), _ptr(b), a.numel(), _ptr(y), _stream()))
    return y


def repeat_kv(x, kv_heads: int, head_dim: int, groups: int, out=None):
    """x [rows, kv_heads*head_dim] -> [rows, kv_heads*groups*head_dim] (heads repeated in place)."""
    torch = _torch()
    rows = x.numel() // (kv_heads * head_dim)
    y = out if out is not None else torch.empty((rows, kv_heads * groups * head_dim), dtype=x.dtype,
                                                device=x.device)
    check(lib().mlxq_repeat_kv(_ptr(x), rows, kv_heads, head_dim, groups, _ptr(y), _stream()))
    return y


def gguf_block(tag: int):
    e, b = ctypes.c_int64(0), ctypes.c_int64(0)
    check(lib().mlxq_gguf_block(tag, ctypes.byref(e), ctypes.byref(b)))
    return e.value, b.value


def gguf_tensor_byte_len(tag: int, n: int) -> int:
    b = ctypes.c_int64(0)
    check(lib().mlxq_gguf_tensor_byte_len(tag, n, ctypes.byref(b)))
    return b.value


def gguf_dequantize(tag: int, data, n: int, out_dtype=None, out=None):
    """Dequantize GGUF blocks held in a uint8 device tensor to f32 (or bf16)."""
    torch = _torch()
    out_dtype = out_dtype or torch.float32
    if out is None:
        out = torch.empty(n, dtype=out_dtype, device=data.device)
    check(lib().mlxq_gguf_dequantize(tag, _ptr(data), data.numel(), n, _dtype_code(out.dtype), _ptr(out),
                                     _stream()))
    return out


def gguf_requantize(tag: int, data, rows: int, cols: int, permute_heads: int = 0, group_size: int = 64,
                    bits: int = 4, out=None):
    """Fused GGUF blocks -> (un-permute) -> bf16 -> MLX affine (wq, scales, biases) on device.
    out: optional preallocated (wq, scales, biases)."""
    torch = _torch()
    if out is None:
        wq = torch.empty((rows, cols * bits // 32), dtype=torch.int32, device=data.device)
        s = torch.empty((rows, cols // group_size), dtype=torch.bfloat16, device=data.device)
        b = torch.empty_like(s)
    else:
        wq, s, b = out
    check(lib().mlxq_gguf_requantize(tag, _ptr(data), data.numel(), rows, cols, permute_heads, group_size, bits,
                                     _ptr(wq), _ptr(s), _ptr(b), _stream()))
    return wq, s, b
