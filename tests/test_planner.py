"""Host-only checks of the sparse planner (forge_sparse_int8_gemm_plan), mirroring the
reference's plan invariants (tests/test_int8_sparse_gemm.cu:132-137, :302-311):
forced tiles and splits are honoured, no split without a workspace, and automatic
plans are valid. The MI355X planner has its own coefficients, so numeric plan parity
with the RTX-4090 model is not a goal."""
import ctypes

import pytest


@pytest.fixture(scope="module")
def plan():
    import forge_amd
    lib = forge_amd.load()

    def f(M, K, N, split_k=0, have_ws=True, tile=-1):
        t, s = ctypes.c_int(), ctypes.c_int()
        assert lib.forge_sparse_int8_gemm_plan(M, K, N, split_k, 1 if have_ws else 0, tile,
                                               ctypes.byref(t), ctypes.byref(s)) == 0
        return t.value, s.value
    return f


SHAPES = [(1, 64, 16), (32, 128, 64), (37, 192, 208), (100, 640, 272), (300, 1280, 384), (1000, 1536, 512),
          (2050, 512, 400), (129, 4096, 96), (4096, 4096, 11008), (16, 8192, 8192)]


@pytest.mark.parametrize("M,K,N", SHAPES)
def test_forced_plans_honoured(plan, M, K, N):
    for tile in range(3):
        for split in (1, 2, 3, 4, 6, 7):
            t, s = plan(M, K, N, split, True, tile)
            assert t == tile and s == split
            t, s = plan(M, K, N, split, False, tile)
            assert t == tile and s == 1


@pytest.mark.parametrize("M,K,N", SHAPES)
def test_auto_plans_valid(plan, M, K, N):
    for have_ws in (True, False):
        t, s = plan(M, K, N, 0, have_ws, -1)
        assert 0 <= t < 3 and s >= 1
        if not have_ws:
            assert s == 1
        assert s in (1, 2, 3, 4, 6)
        steps = (K + 127) // 128
        assert s == 1 or s <= steps // 2


def test_out_of_range_tile_means_auto(plan):
    assert plan(4096, 4096, 11008, 1, True, 7) == plan(4096, 4096, 11008, 1, True, -1)


def test_headline_plan_is_unsplit(plan):
    # 4096 x 11008 x 4096 has 1376 128x128 tiles: splitting cannot pay
    assert plan(4096, 4096, 11008, 0, True)[1] == 1


# The automatic fused/two-pass choice of the sparse linear (the role of the reference's
# sp_use_fused, src/gemm/int8_sparse.cu:926-938), host-only: the MI355X rule follows
# measured timings of both paths, not the RTX-4090 model.
FUSED_CHOICE = [
    ((147456, 1280, 320), True),     # the reference's example layer (int8_sparse.cuh:82)
    ((147456, 1280, 160), True), ((147456, 1536, 384), True), ((147456, 2048, 256), True),
    ((147456, 1024, 128), True), ((98304, 1280, 320), True), ((262144, 1280, 320), True),
    ((65536, 1280, 320), True), ((147456, 1024, 256), True), ((147456, 640, 160), True),
    ((147456, 1280, 640), True), ((147456, 1024, 1024), True),
    ((4096, 1280, 320), False),      # small M: the INT8 copy stays on chip
    ((65536, 640, 320), False),      # M*K below 50M
    ((98304, 1280, 1024), False),    # N over 640 needs M*K >= 150M
    ((147456, 2048, 1024), False),   # ... and K <= 1536
    ((147456, 1024, 2048), False),   # N over 1024
    ((147456, 2176, 256), False),    # K beyond the fused kernel's 2048
    ((147456, 1280, 328), False),    # N not a multiple of 16
    ((1, 8192, 8192), True),         # decode: the decode kernel with its quantize prologue
    ((2, 512, 96), True), ((2, 384, 96), False),   # ... needs K % 256 == 0
    ((3, 8192, 8192), False),        # more tokens than the prologue quantizes
    ((2, 8448, 8192), False),        # K beyond the decode kernel's 8192
]


@pytest.mark.parametrize("shape,fused", FUSED_CHOICE)
def test_sparse_linear_auto_path_choice(shape, fused):
    import forge_amd
    lib = forge_amd.load()
    f = ctypes.c_int(-1)
    assert lib.forge_sparse_int8_linear_fused(*shape, ctypes.byref(f)) == 0
    assert f.value == (1 if fused else 0)
