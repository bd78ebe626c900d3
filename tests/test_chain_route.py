"""CPU: the M dispatch of my_int4.chain follows the reference's make_chain
(bench/exp_p13_official.py:31-39)."""
import pytest


def test_route_table():
    from my_int4.chain import route
    smallm, v3 = "fused_transform_quant_int4_smallm", "fused_transform_quant_int4_v3"
    assert route(1) == (smallm, "w4a4_gemv")
    for M in (2, 3, 4):
        assert route(M) == (smallm, "w4a4_gemv_multi")
    for M in (5, 8, 16, 32):
        assert route(M) == (smallm, "w4a4_gemm_s4")
    for M in (33, 64, 4096):
        assert route(M) == (v3, "w4a4_gemm_s4")
    with pytest.raises(ValueError):
        route(0)


def test_routes_name_existing_ops():
    from my_int4 import _C
    from my_int4.chain import route
    for M in (1, 2, 8, 64):
        for name in route(M):
            assert callable(getattr(_C, name))
