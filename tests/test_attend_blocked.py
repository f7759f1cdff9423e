"""``attend``'s eager branch (the reference's ``vesper/attention.py:384-407``, taken for float32
activations): blocks of ``window`` queries over the keys they can still see, masked by position.

The blocked computation runs on the CPU here, against two forms of the oracle that block
differently: the index-space ``window_attention`` (consecutive positions, another block size) and
one masked softmax over every key of the cache and the chunk at once (positions with gaps, where
the blocks' key ranges and the cache's cut-off must still hold every visible key). Float32 against
float64, so the bound is float32's (``rtol = atol = 1e-5``).
"""

from __future__ import annotations

import pytest
import torch

from oracle import attention as oa


def _case(b, m, n, h, hkv, dk, seed, gaps=False):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(b, n, h, dk, generator=g)
    k, v = (torch.randn(b, n, hkv, dk, generator=g) for _ in range(2))
    ck, cv = (torch.randn(b, m, hkv, dk, generator=g) for _ in range(2))
    if gaps:  # strictly increasing positions with steps of 1 to 3, each batch row its own
        steps = torch.randint(1, 4, (b, m + n), generator=g)
        allpos = 50 + torch.cumsum(steps, dim=1)
    else:
        allpos = torch.arange(50, 50 + m + n).expand(b, m + n).contiguous()
    return q, k, v, allpos[:, m:].contiguous(), ck, cv, allpos[:, :m].contiguous()


@pytest.mark.parametrize(("m", "n", "w"), [(0, 1, 8), (0, 30, 8), (5, 30, 8), (8, 8, 8), (3, 17, 16), (7, 5, 8)])
@pytest.mark.parametrize(("h", "hkv"), [(4, 2), (2, 2)])
def test_consecutive_positions_equal_the_index_space_window(m, n, w, h, hkv):
    from vesper.attention import KVCache, _attend_blocked

    q, k, v, pos, ck, cv, cpos = _case(2, m, n, h, hkv, 16, m * 100 + n + w + h)
    got = _attend_blocked(q, k, v, pos, KVCache(ck, cv, cpos, w))
    keys, vals = torch.cat([ck, k], 1).double(), torch.cat([cv, v], 1).double()
    want = oa.window_attention(q.double(), keys, vals, w, block=5)
    assert got.dtype == torch.float32 and got.shape == q.shape
    torch.testing.assert_close(got.double(), want, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize(("m", "n", "w"), [(0, 40, 8), (6, 40, 8), (8, 23, 8), (2, 9, 4)])
def test_positions_with_gaps_equal_one_masked_softmax_over_every_key(m, n, w):
    from vesper.attention import KVCache, _attend_blocked

    q, k, v, pos, ck, cv, cpos = _case(2, m, n, 4, 2, 16, 7 * m + n, gaps=True)
    got = _attend_blocked(q, k, v, pos, KVCache(ck, cv, cpos, w))
    keys, vals = torch.cat([ck, k], 1).double(), torch.cat([cv, v], 1).double()
    want = oa.attention_full_mask(q.double(), keys, vals, pos, torch.cat([cpos, pos], 1), w)
    torch.testing.assert_close(got.double(), want, rtol=1e-5, atol=1e-5)


def test_a_mistake_in_the_window_edge_is_caught():
    # the same comparison fails for a window one wider: the check above is sensitive to the edge
    from vesper.attention import KVCache, _attend_blocked

    q, k, v, pos, ck, cv, cpos = _case(1, 6, 40, 2, 2, 16, 11, gaps=True)
    got = _attend_blocked(q, k, v, pos, KVCache(ck, cv, cpos, 8))
    keys, vals = torch.cat([ck, k], 1).double(), torch.cat([cv, v], 1).double()
    wrong = oa.attention_full_mask(q.double(), keys, vals, pos, torch.cat([cpos, pos], 1), 9)
    assert (got.double() - wrong).abs().max() > 1e-3
