"""GPU parity: the wide-tile 2:4 sparse engine (INT32 out; 256 tokens x 8-11 32-row weight
blocks per tile, every CU the same weight blocks of a 256-token block as T tiles).

Bar: every INT32 output bit-exact against the oracle (the reference's sparse GEMM sums,
src/gemm/int8_sparse.cu:116-120, over the decompressed 2:4 weights), output poisoned first.
The shapes cover 1 to 4 tiles per CU, tiles of 8, 9, 10 and 11 blocks, ragged token blocks,
a half last weight block (N % 32 == 16), the shortest K (4 stages), the XCD grouping and the
plain slot mapping (CU slots fewer than the CUs)."""
import numpy as np
import pytest

from helpers import int8_uniform, poison, say, to_dev, to_host

pytestmark = pytest.mark.gpu


def _prep(dev, W):
    import torch
    from forge_amd import ops
    N, K = W.shape
    comp = torch.empty((N, K // 2), dtype=torch.int8, device=dev)
    raw = torch.empty((N * K // 4,), dtype=torch.uint8, device=dev)
    meta = torch.empty((N * K // 32,), dtype=torch.int32, device=dev)
    ops.prune_compress_24(to_dev(W, dev), comp, raw, N, K)
    ops.pack_metadata(raw, meta, N, K)
    return comp, meta


# (M, K, N, tiles per CU): plan on 256 CUs -- token blocks TB = ceil(M / 256), c = 256 // TB CUs
# each, weight 32-blocks ceil(N / 32) over them (q or q + 1 per CU), T = ceil((q + 1) / 11); the
# engine is taken where 256 x 256 tiles leave a partial last wave (sparse_wide_pays).
WIDE_SHAPES = [
    (1000, 4096, 17904, 1),   # TB 4, tiles of 8 and 9 blocks, ragged tokens, half last block
    (512, 4096, 35008, 1),    # TB 2, 8/9 blocks, half last block
    (4096, 2048, 11008, 2),   # configs[2]'s N: 21/22 blocks as 11 + 10 / 11 + 11
    (8192, 512, 7936, 3),     # TB 32, c 8, K = 512 (four stages): 31 blocks as 11 + 10 + 10
    (8192, 512, 11008, 4),    # 43 blocks as 11 + 11 + 11 + 10
    (3000, 4096, 6720, 1),    # TB 12, c 21: 252 CU slots, no XCD grouping; 10 blocks
]


@pytest.mark.parametrize("M,K,N,T", WIDE_SHAPES)
def test_sparse_wide_int32(dev, orc, M, K, N, T):
    import torch
    from forge_amd import ops
    rng = np.random.default_rng(M + 5 * K + 11 * N)
    W = int8_uniform(rng, (N, K))
    x = int8_uniform(rng, (M, K))
    cr, mr = orc.prune_compress_24(W)
    ref = orc.sparse_gemm_s32(cr, x, mr, N, K, threads=orc.cpu_threads())
    comp, meta = _prep(dev, W)
    say(f"sparse wide INT32 M={M} K={K} N={N}")
    C = torch.empty((M, N), dtype=torch.int32, device=dev)
    poison(C, 0x7B)
    got = to_host(ops.sparse_int8_gemm_s32(comp, to_dev(x, dev), meta, out=C))
    assert ops.last_route() == f"wide256 tile{T}"
    bad = int((got != ref).sum())
    assert bad == 0, f"{bad} of {got.size} outputs differ"
    # a second call on the same buffers gives the same bits (no state carried between launches)
    poison(C, 0x5A)
    again = to_host(ops.sparse_int8_gemm_s32(comp, to_dev(x, dev), meta, out=C))
    assert np.array_equal(again, got)

