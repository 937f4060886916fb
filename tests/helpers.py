"""Seeded inputs and numpy <-> device plumbing shared by the tests."""
import numpy as np

import oracle as orc


def bf16_weights(seed: int, n: int, k: int, std: float = 0.02) -> np.ndarray:
    """W ~ N(0, std) in f32, rounded to bf16 (the cast llama.rs:97 does before quantizing)."""
    return orc.f32_to_bf16(orc.normal(seed, n * k, 0.0, std)).reshape(n, k)


def bf16_acts(seed: int, m: int, k: int) -> np.ndarray:
    return orc.f32_to_bf16(orc.normal(seed, m * k, 0.0, 1.0)).reshape(m, k)


def dev(a: np.ndarray, bf16: bool = False):
    import torch

    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        t = torch.from_numpy(a.view(np.int16)).cuda()
        return t.view(torch.bfloat16) if bf16 else t
    if a.dtype == np.uint32:
        return torch.from_numpy(a.view(np.int32)).cuda()
    return torch.from_numpy(a).cuda()


def host(t) -> np.ndarray:
    import torch

    t = t.detach().cpu().contiguous()
    if t.dtype in (torch.bfloat16, torch.float16, torch.int16):
        return t.view(torch.int16).numpy().view(np.uint16)
    if t.dtype == torch.int32:
        return t.numpy().view(np.uint32)
    return t.numpy()


def rel_err(y: np.ndarray, ref: np.ndarray) -> float:
    """max |y - ref| / max |ref| (the max-relative-error figure the parity bar uses)."""
    return float(np.max(np.abs(y.astype(np.float64) - ref)) / max(np.max(np.abs(ref)), 1e-30))


def rel_err_elem(y: np.ndarray, ref: np.ndarray, floor: float = 1e-3) -> float:
    """max over elements of |y - ref| / |ref|, leaving out elements with
    |ref| < floor * max |ref| (near-zero references, where a relative error
    says nothing); reported beside rel_err."""
    ref = np.asarray(ref, dtype=np.float64)
    a = np.abs(ref)
    keep = a >= floor * max(a.max(), 1e-30)
    return float(np.max(np.abs(y.astype(np.float64)[keep] - ref[keep]) / a[keep]))
