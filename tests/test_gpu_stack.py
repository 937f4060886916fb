"""Quantized decode stack (the Llama layer chain with attention replaced by
the identity on v) on the GPU against the CPU oracle's chain of the same
ops, same packed weights and same bf16 rounding points.

The oracle sums each projection in f64; the GPU in f32 in another order.
Rounding differences then propagate through the chain, so the logits are
compared by max |y - ref| / max |ref| <= 1e-2 (the qmatmul parity bar).
"""
import numpy as np
import pytest

import oracle as orc
from helpers import dev, host, rel_err
from stack import DecodeStack, StackConfig

pytestmark = pytest.mark.gpu

TOL = 1e-2

SMALL = dict(layers=3, hidden=512, intermediate=1536, heads=8, kv_heads=2, head_dim=64, vocab=1000)


def _run(cfg: StackConfig, batch: int, graph: bool, fused: bool = True):
    st = DecodeStack(cfg, batch=batch, seed=7, norm_noise=0.1)
    x = orc.f32_to_bf16(orc.normal(1234 + batch, batch * cfg.hidden, 0.0, 1.0)).reshape(batch, cfg.hidden)
    st.x.copy_(dev(x, True))
    if graph:
        g = st.capture(fused=fused)
        g.replay()
        g.replay()  # a replay must give the same result as the first
    else:
        st.forward(fused=fused)
    got = host(st.logits)
    layers, norm, lm = st.host_weights()
    want = orc.decode_stack(x, layers, norm, lm, cfg.as_dict())
    return got, want


@pytest.mark.parametrize("fused", [True, False])
@pytest.mark.parametrize("batch", [1, 4, 16])
def test_small_stack(torch_gpu, batch, fused):
    got, want = _run(StackConfig(**SMALL), batch, graph=False, fused=fused)
    assert rel_err(orc.bf16_to_f32(got), orc.bf16_to_f32(want).astype(np.float64)) <= TOL


@pytest.mark.parametrize("bits", [4, 8])
def test_small_stack_graph(torch_gpu, bits):
    got, want = _run(StackConfig(bits=bits, **SMALL), 2, graph=True)
    assert rel_err(orc.bf16_to_f32(got), orc.bf16_to_f32(want).astype(np.float64)) <= TOL


@pytest.mark.parametrize("batch", [1, 3, 16])
def test_llama3_8b_width_two_layers(torch_gpu, batch):
    """Config-5 widths (hidden 4096, intermediate 14336, 32/8 heads x 128,
    vocab 128256, Q4 g64) with two layers, so the f64 CPU chain stays short."""
    got, want = _run(StackConfig(layers=2), batch, graph=True)
    print("rel_err", rel_err(orc.bf16_to_f32(got), orc.bf16_to_f32(want).astype(np.float64)))
    assert rel_err(orc.bf16_to_f32(got), orc.bf16_to_f32(want).astype(np.float64)) <= TOL


# ---- persistent single-launch decode step (mlxq_decode_plan / mlxq_decode_step)

def _persistent(cfg: StackConfig, seeds, graph: bool):
    """Logits of the persistent step and of the oracle chain for each input
    seed, on one plan (and one graph when graph=True): later calls must see
    the new input, not activations left by an earlier call."""
    st = DecodeStack(cfg, batch=1, seed=11, norm_noise=0.1)
    layers, norm, lm = st.host_weights()
    g = None
    out = []
    for sd in seeds:
        x = orc.f32_to_bf16(orc.normal(sd, cfg.hidden, 0.0, 1.0)).reshape(1, cfg.hidden)
        st.x.copy_(dev(x, True))
        if graph:
            if g is None:
                g = st.capture(1, persistent=True)
            g.replay()
        else:
            st.forward(1, persistent=True)
        got = host(st.logits).copy()
        want = orc.decode_stack(x, layers, norm, lm, cfg.as_dict())
        out.append((got, want))
    assert not st.persistent_plan().timed_out()
    return st, out


@pytest.mark.parametrize("graph", [False, True])
def test_persistent_small(torch_gpu, graph):
    _, res = _persistent(StackConfig(**SMALL), [501, 502, 503], graph)
    for got, want in res:
        assert rel_err(orc.bf16_to_f32(got), orc.bf16_to_f32(want).astype(np.float64)) <= TOL


def test_persistent_llama3_8b_width_two_layers(torch_gpu):
    """Config-5 widths, two layers, three inputs through one captured graph;
    also against the fused multi-launch chain on the same weights."""
    st, res = _persistent(StackConfig(layers=2), [601, 602, 603], graph=True)
    for got, want in res:
        e = rel_err(orc.bf16_to_f32(got), orc.bf16_to_f32(want).astype(np.float64))
        print("rel_err", e)
        assert e <= TOL
    pers = orc.bf16_to_f32(res[-1][0]).astype(np.float64)
    st.forward(1, fused=True)
    fused = orc.bf16_to_f32(host(st.logits))
    assert rel_err(pers, fused.astype(np.float64)) <= TOL


def test_persistent_unsupported(torch_gpu):
    import mlxq
    st = DecodeStack(StackConfig(bits=8, **SMALL), batch=1, seed=3)
    with pytest.raises(mlxq.Unsupported):
        st.persistent_plan()


def test_persistent_barrier_timeout_path(torch_gpu, monkeypatch):
    """Failure handling forced from the host: a 1-tick barrier wait limit
    makes the grid barriers give up.  Every wave leaves the launch (the
    bounded waits end it; nothing hangs), the plan reports the time-out, and a
    fresh plan on the same weights computes the step correctly again."""
    import torch
    cfg = StackConfig(**SMALL)
    st = DecodeStack(cfg, batch=1, seed=13, norm_noise=0.1)
    x = orc.f32_to_bf16(orc.normal(777, cfg.hidden, 0.0, 1.0)).reshape(1, cfg.hidden)
    st.x.copy_(dev(x, True))
    monkeypatch.setenv("MLXQ_DECODE_TIMEOUT_TICKS", "1")
    st.forward(1, persistent=True)
    torch.cuda.synchronize()
    assert st.persistent_plan().timed_out()
    monkeypatch.delenv("MLXQ_DECODE_TIMEOUT_TICKS")
    st._plan = None  # a new plan: the barrier state starts over
    st.forward(1, persistent=True)
    torch.cuda.synchronize()
    assert not st.persistent_plan().timed_out()
    layers, norm, lm = st.host_weights()
    want = orc.decode_stack(x, layers, norm, lm, cfg.as_dict())
    assert rel_err(orc.bf16_to_f32(host(st.logits)), orc.bf16_to_f32(want).astype(np.float64)) <= TOL
