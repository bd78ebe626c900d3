"""GPU: my_int4.chain.make_chain / graphed -- eager results against the oracle
and graph replays against eager (reference tests/test_p13.py:45-66, with
bit-identical replays instead of its 0.5 tolerance: every op here is
deterministic)."""
import numpy as np
import pytest

import oracle
from _util import f16_tensor_f64, f32_to_bf16_bits, outlier_activations, rel_fro, rng, to_dev_bf16, to_dev_u8

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("M", [1, 3, 4, 5, 8, 16, 32, 33, 64, 300])
def test_make_chain_eager_and_replays(M):
    import torch
    from my_int4.chain import graphed, make_chain
    g = rng(6000 + M)
    N, K = 384, 1024
    xb = outlier_activations(g, M, K)
    tb = f32_to_bf16_bits(g.standard_normal((K // 32, 32, 32)) * 0.25)
    wq, ws = oracle.quant(f32_to_bf16_bits(g.standard_normal((N, K)) * 0.02), "bf16")
    X, T = to_dev_bf16(xb), to_dev_bf16(tb)
    step = make_chain(X, T, to_dev_u8(wq), to_dev_bf16(ws), M)
    y0 = step().clone()
    assert y0.shape == ((N,) if M == 1 else (M, N))
    qo, so = oracle.fused_tq(xb, tb)
    ref = oracle.gemm_f64(qo, so, wq, ws)
    assert rel_fro(f16_tensor_f64(y0).reshape(M, N), ref) < 2e-3
    graph, out = graphed(step)
    for r in range(3):
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, y0), (M, r)
        step()                                # eager work between replays
        torch.cuda.synchronize()
