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


# Larger layer steps under graph replay: (2048, 8192, 4096) runs the two-tile
# transform and the 256-row fp16 tiles on activations converted into the
# workspace; (128, 24576, 4096) the small-M transform and the 128-row fp16
# tiles with K split over 2 slices (partials and their sum in the graph).
# Eager against the fp64 oracle on sampled outputs; every replay equal to
# eager bit for bit.
@pytest.mark.parametrize("M,N,K", [(2048, 8192, 4096), (128, 24576, 4096)])
def test_make_chain_replays_large(M, N, K):
    import torch
    from my_int4.chain import graphed, make_chain
    g = rng(6100 + M)
    xb = outlier_activations(g, M, K)
    tb = f32_to_bf16_bits(g.standard_normal((K // 32, 32, 32)) * 0.25)
    wq, ws = oracle.quant(f32_to_bf16_bits(g.standard_normal((N, K)) * 0.02), "bf16")
    X, T = to_dev_bf16(xb), to_dev_bf16(tb)
    step = make_chain(X, T, to_dev_u8(wq), to_dev_bf16(ws), M)
    y0 = step().clone()
    rows = np.unique(np.concatenate([[0, M - 1], g.choice(M, 30, replace=False)]))
    cols = np.unique(np.concatenate([[0, N - 1], g.choice(N, 600, replace=False)]))
    qo, so = oracle.fused_tq(xb[rows], tb)
    ref = oracle.gemm_f64(qo, so, wq[cols], ws[cols])
    assert rel_fro(f16_tensor_f64(y0)[np.ix_(rows, cols)], ref) < 2e-3
    graph, out = graphed(step)
    for r in range(3):
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, y0), (M, N, K, r)
        step()
        torch.cuda.synchronize()
