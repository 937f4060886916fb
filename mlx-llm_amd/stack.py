"""Quantized Llama decode stack over the mlxq C ABI.

The layer chain of the reference's CausalLm decode step
(src/models/llama.rs:689-735 per layer, q/k/v/o at :806-835, the MLP at
:1040-1045, final norm + lm_head at :595-603) with every projection
quantized (Q4/Q8, MLX affine layout) and attention replaced by the identity
on v, its 8 KV heads repeated to the 32 query heads (the attention of a
single cached position).  Only the quantized GEMV/GEMM path and the bf16
ops around it run:

    n1 = rms_norm(x, ln1);  q, k, v = n1 Wq^T, n1 Wk^T, n1 Wv^T
    h  = x + repeat_kv(v) Wo^T
    n2 = rms_norm(h, ln2);  x' = h + (silu(n2 Wg^T) * (n2 Wu^T)) Wd^T
    logits = rms_norm(x_L, norm) Wlm^T

Every op is a libmlxq kernel; torch provides device memory, streams and
graph capture.  The lm_head is quantized too (the reference keeps it dense,
src/models/llama.rs:122-128; the benchmark configuration asks for Q4).
"""
from __future__ import annotations

from dataclasses import dataclass, field

import mlxq
import seeded

PROJ = ("q", "k", "v", "o", "gate", "up", "down")


@dataclass
class StackConfig:
    layers: int = 32
    hidden: int = 4096
    intermediate: int = 14336
    heads: int = 32
    kv_heads: int = 8
    head_dim: int = 128
    vocab: int = 128256
    eps: float = 1e-5
    group_size: int = 64
    bits: int = 4

    @property
    def groups(self) -> int:
        return self.heads // self.kv_heads

    def proj_shape(self, name: str) -> tuple[int, int]:
        """(out N, in K) of a projection (Hugging Face [out, in] layout)."""
        h, i, q, kv = self.hidden, self.intermediate, self.heads * self.head_dim, self.kv_heads * self.head_dim
        return {"q": (q, h), "k": (kv, h), "v": (kv, h), "o": (h, q), "gate": (i, h), "up": (i, h),
                "down": (h, i), "lm_head": (self.vocab, h)}[name]

    def as_dict(self) -> dict:
        return dict(layers=self.layers, hidden=self.hidden, intermediate=self.intermediate, heads=self.heads,
                    kv_heads=self.kv_heads, head_dim=self.head_dim, vocab=self.vocab, eps=self.eps,
                    group_size=self.group_size, bits=self.bits)


def llama3_8b(**kw) -> StackConfig:
    return StackConfig(**kw)


@dataclass
class QLinear:
    """A quantized projection in MLX's packed layout (all device tensors)."""
    wq: object
    scales: object
    biases: object
    n: int
    k: int

    def bytes(self) -> int:
        return self.wq.numel() * 4 + self.scales.numel() * 2 + self.biases.numel() * 2


@dataclass
class Layer:
    proj: dict = field(default_factory=dict)
    ln1: object = None
    ln2: object = None


class DecodeStack:
    """Random-init quantized Llama stack (seeded N(0, 0.02) weights quantized on
    device) with activations preallocated for up to `batch` rows, so a decode
    step of any batch b <= batch can be captured in a HIP graph and replayed
    (the step works on the first b rows of every buffer)."""

    def __init__(self, cfg: StackConfig, batch: int = 1, seed: int = 0, device="cuda", norm_noise: float = 0.0):
        import torch
        self.cfg, self.batch, self.device = cfg, batch, torch.device(device)

        def qlin(name, idx):
            n, k = cfg.proj_shape(name)
            # N(0, 0.02) f32 from the tensor's SplitMix64 stream, cast to bf16
            w = seeded.normal(0x5EED0000 + seed * 1_000_003 + idx, n * k, 0.0, 0.02, device=self.device)
            w = w.view(n, k).to(torch.bfloat16)
            wq, s, b = mlxq.quantize(w, cfg.group_size, cfg.bits)
            del w
            return QLinear(wq, s, b, n, k)

        def norm_w(idx):
            w = torch.ones(cfg.hidden, device=self.device)
            if norm_noise:
                w = w + seeded.normal(0x5EED0000 + seed * 1_000_003 + idx, cfg.hidden, 0.0, norm_noise,
                                      device=self.device)
            return w.to(torch.bfloat16)

        self.layers = []
        idx = 0
        for _ in range(cfg.layers):
            L = Layer()
            for p in PROJ:
                L.proj[p] = qlin(p, idx)
                idx += 1
            L.ln1, L.ln2 = norm_w(idx), norm_w(idx + 1)
            idx += 2
            self.layers.append(L)
        self.norm = norm_w(idx)
        self.lm_head = qlin("lm_head", idx + 1)

        M, bf = batch, torch.bfloat16
        e = lambda n: torch.empty((M, n), dtype=bf, device=self.device)  # noqa: E731
        q_dim, kv_dim = cfg.heads * cfg.head_dim, cfg.kv_heads * cfg.head_dim
        self.x = e(cfg.hidden)          # step input (hidden state entering layer 0)
        self.xa, self.xb = e(cfg.hidden), e(cfg.hidden)  # residual stream ping-pong
        self.n = e(cfg.hidden)
        self.h = e(cfg.hidden)
        self.q, self.k, self.v = e(q_dim), e(kv_dim), e(kv_dim)
        self.attn = e(q_dim)
        self.o = e(cfg.hidden)
        self.g, self.u, self.a = e(cfg.intermediate), e(cfg.intermediate), e(cfg.intermediate)
        self.d = e(cfg.hidden)
        self.logits = e(cfg.vocab)
        # the qmatmul workspace for the largest projection call of any batch
        # <= batch, reserved now so that no call grows it inside a capture
        shapes = [(p.n, p.k) for p in [*self.layers[0].proj.values(), self.lm_head]]
        need = max(mlxq.workspace_size(b, n, k, cfg.group_size, cfg.bits)
                   for b in range(1, batch + 1) for n, k in shapes)
        if need:
            mlxq.workspace(need, self.device)

    def weight_bytes(self) -> int:
        """Packed weight bytes one decode step streams (codes + scales + biases)."""
        return sum(p.bytes() for L in self.layers for p in L.proj.values()) + self.lm_head.bytes()

    def _lin(self, x, p: QLinear, out):
        return mlxq.qmatmul(x, p.wq, p.scales, p.biases, self.cfg.group_size, self.cfg.bits, out=out)

    def forward(self, b: int | None = None, fused: bool = True, layers=None, head: bool = True):
        """One decode step of b rows on the current stream: self.x[:b] -> self.logits[:b].
        fused: per layer, four launches of the fused decode kernel (norm + q/k/v,
        head repeat + o + residual, norm + gate/up + SwiGLU, down + residual)
        wherever it covers the shape; a call it does not cover (it rejects the
        shape before launching anything) runs as the op-by-op chain.
        layers (an iterable of layer indices, default all) and head=False run
        part of the chain, for checking it layer by layer: without the head
        the hidden state after the last layer run is returned."""
        if not fused:
            return self._forward_ops(b, layers, head)
        c = self.cfg
        b = self.batch if b is None else b
        gs, bits = c.group_size, c.bits
        n, h, q, k, v, attn, o = (t[:b] for t in (self.n, self.h, self.q, self.k, self.v, self.attn, self.o))
        g, u, a, d = (t[:b] for t in (self.g, self.u, self.a, self.d))
        lin = self._lin

        def fz(x, projs, fallback, **kw):
            try:
                mlxq.qmatmul_fused(x, projs, gs, bits, **kw)
            except mlxq.Unsupported:
                fallback()

        x = self.x[:b]
        # b > 4 (no fused norm / SwiGLU forms): gate, up and down as plain
        # qmatmul calls (the LDS-shared tile kernel) measured faster than the
        # streaming matrix-core multi-projection and residual forms (batch 16:
        # 3.01 -> 2.85 ms per step); q/k/v and o keep the fused forms (plain
        # calls there: 3.24 / 2.98 ms)
        split = {"mlp", "down"} if b > 4 else set()
        order = list(range(len(self.layers)) if layers is None else layers)
        # b > 4: the residual add that ends a layer and the norm that starts
        # the next (or the final norm) run as one launch; `normed` says that
        # n already holds the next norm's output
        normed = [False]
        for j, i in enumerate(order):
            L = self.layers[i]
            P = L.proj
            xn = (self.xa if j % 2 == 0 else self.xb)[:b]

            # where the single fused launch does not cover the shape (b > 4),
            # the norm / head repeat / SwiGLU run as their own kernels and the
            # projections still share launches with their residual adds
            def qkv(x=x, P=P, L=L):
                if not normed[0]:
                    mlxq.rms_norm(x, L.ln1, c.eps, out=n)
                fz(n, [self._proj(P["q"], q), self._proj(P["k"], k), self._proj(P["v"], v)],
                   lambda: (lin(n, P["q"], q), lin(n, P["k"], k), lin(n, P["v"], v)))

            def oproj(x=x, P=P):
                mlxq.repeat_kv(v, c.kv_heads, c.head_dim, c.groups, out=attn)
                fz(attn, [self._proj(P["o"], h, res=x)], lambda: (lin(attn, P["o"], o), mlxq.add(x, o, out=h)))

            def mlp_in(P=P, L=L, split=split):
                mlxq.rms_norm(h, L.ln2, c.eps, out=n)

                def plain():
                    lin(n, P["gate"], g)
                    lin(n, P["up"], u)
                    mlxq.silu_mul(g, u, out=a)

                if "mlp" in split:  # gate/up pairs and SwiGLU in one streaming launch where covered
                    fz(n, [self._proj(P["gate"], a), self._proj(P["up"], u)], plain, swiglu=True)
                else:
                    fz(n, [self._proj(P["gate"], g), self._proj(P["up"], u)],
                       lambda: (lin(n, P["gate"], g), lin(n, P["up"], u)))
                    mlxq.silu_mul(g, u, out=a)

            nxt = self.layers[order[j + 1]].ln1 if j + 1 < len(order) else (self.norm if head else None)

            def down(P=P, xn=xn, nxt=nxt):
                if nxt is not None:  # down + residual + the next norm (split-K sum, add and norm in one launch)
                    pd = P["down"]
                    mlxq.qmatmul_add_rms_norm(a, pd.wq, pd.scales, pd.biases, h, nxt, c.eps, gs, bits,
                                              sum_out=xn, out=n)
                else:
                    lin(a, P["down"], d)
                    mlxq.add(h, d, out=xn)

            fz(x, [self._proj(P["q"], q), self._proj(P["k"], k), self._proj(P["v"], v)], qkv,
               norm_weight=L.ln1, eps=c.eps)
            normed[0] = False
            fz(v, [self._proj(P["o"], h, res=x)], oproj, repeat=(c.kv_heads, c.head_dim, c.groups))
            fz(h, [self._proj(P["gate"], a), self._proj(P["up"], u)], mlp_in, norm_weight=L.ln2, eps=c.eps,
               swiglu=True)
            if "down" in split:
                down()
                normed[0] = nxt is not None
            else:
                fz(a, [self._proj(P["down"], xn, res=h)], down)
            x = xn
        if not head:
            return x

        def head_ops(x=x):
            if not normed[0]:
                mlxq.rms_norm(x, self.norm, c.eps, out=n)
            lin(n, self.lm_head, self.logits[:b])

        fz(x, [self._proj(self.lm_head, self.logits[:b])], head_ops, norm_weight=self.norm, eps=c.eps)
        return self.logits[:b]

    def _proj(self, p: QLinear, y, res=None):
        d = {"wq": p.wq, "scales": p.scales, "biases": p.biases, "y": y}
        if res is not None:
            d["residual"] = res
        return d

    def _forward_ops(self, b: int | None = None, layers=None, head: bool = True):
        c = self.cfg
        b = self.batch if b is None else b
        assert 1 <= b <= self.batch
        n, h, q, k, v, attn, o = (t[:b] for t in (self.n, self.h, self.q, self.k, self.v, self.attn, self.o))
        g, u, a, d = (t[:b] for t in (self.g, self.u, self.a, self.d))
        x = self.x[:b]
        for j, i in enumerate(range(len(self.layers)) if layers is None else layers):
            L = self.layers[i]
            P = L.proj
            mlxq.rms_norm(x, L.ln1, c.eps, out=n)
            self._lin(n, P["q"], q)
            self._lin(n, P["k"], k)
            self._lin(n, P["v"], v)
            mlxq.repeat_kv(v, c.kv_heads, c.head_dim, c.groups, out=attn)
            self._lin(attn, P["o"], o)
            mlxq.add(x, o, out=h)
            mlxq.rms_norm(h, L.ln2, c.eps, out=n)
            self._lin(n, P["gate"], g)
            self._lin(n, P["up"], u)
            mlxq.silu_mul(g, u, out=a)
            self._lin(a, P["down"], d)
            x = (self.xa if j % 2 == 0 else self.xb)[:b]
            mlxq.add(h, d, out=x)
        if not head:
            return x
        mlxq.rms_norm(x, self.norm, c.eps, out=n)
        self._lin(n, self.lm_head, self.logits[:b])
        return self.logits[:b]

    def capture(self, b: int | None = None, fused: bool = True):
        """Capture forward(b) in a HIP graph; returns the graph (replay() runs one step)."""
        import torch
        s = torch.cuda.Stream(device=self.device)
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            self.forward(b, fused)  # warm-up outside the capture (kernel attributes)
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=s):
            self.forward(b, fused)
        torch.cuda.synchronize()
        return graph

    def host_weights(self):
        """Packed weights as numpy (uint32 codes, bf16 bits) for a CPU checker."""
        import numpy as np
        import torch

        def h16(t):
            return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)

        def hq(p: QLinear):
            return (p.wq.cpu().numpy().view(np.uint32), h16(p.scales), h16(p.biases))

        layers = [dict({k: hq(v) for k, v in L.proj.items()}, ln1=h16(L.ln1), ln2=h16(L.ln2)) for L in self.layers]
        return layers, h16(self.norm), hq(self.lm_head)
