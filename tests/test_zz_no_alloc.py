"""mlxq_qmatmul_noalloc (split-K partials in the library's fixed scratch
array) against mlxq_qmatmul with a caller workspace: bit-identical, on two
calls in a row with the second smaller, at shapes that split K (batched
decode, prefill) and one that does not; oversize shapes are refused before
any launch."""
import ctypes

import numpy as np
import pytest

import mlxq
import oracle as orc
from helpers import bf16_acts, bf16_weights, dev, host

pytestmark = pytest.mark.gpu


def noalloc(x, wq, s, b, n, k, bits, bias=None):
    import torch

    m = x.shape[0]
    y = torch.empty((m, n), dtype=torch.bfloat16, device="cuda:0")
    mlxq.check(mlxq.lib().mlxq_qmatmul_noalloc(mlxq._ptr(x), m, mlxq._ptr(wq), mlxq._ptr(s), mlxq._ptr(b),
                                               mlxq._ptr(bias), n, k, 64, bits, mlxq._ptr(y),
                                               torch.cuda.current_stream().cuda_stream))
    return y


def layer(seed, n, k, bits):
    w = bf16_weights(seed, n, k)
    wq, s, b = orc.affine_quantize(w, 64, bits, orc.BF16)
    return dev(wq), dev(s, bf16=True), dev(b, bf16=True)


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("n,k,m1,m2", [(14336, 4096, 32, 16), (4096, 14336, 16, 5), (1024, 4096, 32, 1),
                                       (4096, 14336, 2048, 512), (14336, 4096, 96, 48), (14336, 4096, 2048, 96)])
def test_noalloc_matches_workspace_path(torch_gpu, bits, n, k, m1, m2):
    torch = torch_gpu
    print(f"noalloc bits={bits} n={n} k={k} m={m1},{m2}", flush=True)
    wq, s, b = layer(0x7000 + n + bits, n, k, bits)
    bias = dev(orc.f32_to_bf16(np.random.default_rng(n).normal(0, 1, n).astype(np.float32)), bf16=True)
    for m in (m1, m2):
        x = dev(bf16_acts(0x7100 + m, m, k), bf16=True)
        # the no-alloc route is mlxq_qmatmul's except where that takes the
        # library GEMM (the qmm kernel runs there): 33..64 rows in 32-row
        # decode calls, gate/up-like 65..128 rows on the 64-row streaming form
        lib = "hipBLASLt" in mlxq.qmatmul_route(m, n, k, 64, bits)
        want = mlxq.qmatmul(x, wq, s, b, 64, bits, bias=bias, algo=mlxq.ALGO_QMM if lib else mlxq.ALGO_AUTO)
        got = noalloc(x, wq, s, b, n, k, bits, bias)
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), m


def test_noalloc_rejects_oversize_before_launch(torch_gpu):
    torch = torch_gpu
    cap = mlxq.lib().mlxq_qmatmul_noalloc_max_scratch()
    assert cap == 64 << 20
    need = mlxq.workspace_size(32, 128256, 4096, 64, 4)  # a Llama-3 lm_head at batch 32
    assert need > cap
    rc = mlxq.lib().mlxq_qmatmul_noalloc(None, 32, None, None, None, None, 128256, 4096, 64, 4, None, None)
    assert rc == mlxq.ERR_WORKSPACE
    assert b"scratch" in mlxq.lib().mlxq_last_error()


def test_noalloc_route_query_refuses_what_the_call_refuses(torch_gpu):
    """The route query of the no-alloc call refuses the shapes the call itself
    refuses (scratch beyond the fixed array), and names the kernels otherwise."""
    with pytest.raises(mlxq.MlxqError) as e:
        mlxq.qmatmul_route(32, 128256, 4096, 64, 4, noalloc=True)
    assert e.value.status == mlxq.ERR_WORKSPACE
    assert mlxq.qmatmul_route(2048, 4096, 14336, 64, 4, noalloc=True).startswith("qmm_kernel<4, 64")
