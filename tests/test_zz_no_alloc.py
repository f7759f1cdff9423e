"""The allocation-free ring attention entry (``vsp_ring_attn_noalloc_bf16``) against the entry it
varies (``vsp_ring_attn_bf16`` with a caller's workspace), through the C ABI.

Both run the same kernel on the same inputs, so outputs and the written rings must agree bitwise;
two calls in a row, the second with fewer rows, show the static counters are left zero between
calls. A request beyond the static scratch is refused on the host, before any launch.
"""

from __future__ import annotations

import math

import pytest
import torch

from conftest import needs_gpu

pytestmark = [pytest.mark.gpu, needs_gpu]

GPU = torch.device("cuda")
BF16 = torch.bfloat16


def _case(b, h, hkv, dk, w, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(b, h, dk, generator=g).to(GPU, BF16)
    k = torch.randn(b, hkv, dk, generator=g).to(GPU, BF16)
    v = torch.randn(b, hkv, dk, generator=g).to(GPU, BF16)
    pos = torch.randint(w // 2, 3 * w, (b,), generator=g).to(GPU)
    ring_k = torch.randn(b, w, hkv, dk, generator=g).to(GPU, BF16)
    ring_v = torch.randn(b, w, hkv, dk, generator=g).to(GPU, BF16)
    ring_pos = (pos[:, None].cpu() - 1 - torch.randperm(w, generator=g)[None, :]).to(GPU)
    ring_valid = (torch.rand(b, w, generator=g) < 0.9).to(GPU, torch.uint8)
    return q, k, v, pos, [ring_k, ring_v, ring_pos, ring_valid]


def _run(entry, q, k, v, pos, ring, h, hkv, dk, w, workspace=None):
    from vesper.kernels import _lib

    b = q.shape[0]
    o = torch.empty_like(q)
    stream = _lib.stream_of(q.device)
    args = [q.data_ptr(), k.data_ptr(), v.data_ptr(), pos.data_ptr(), *(t.data_ptr() for t in ring), o.data_ptr(), None]
    if workspace is not None:
        args += [workspace.data_ptr(), workspace.numel() * 4]
    _lib.call(entry, *args, b, h, hkv, dk, w, 1.0 / math.sqrt(dk), 1, stream)
    return o


@pytest.mark.parametrize(("b1", "b2"), [(64, 5)])
def test_the_allocation_free_entry_equals_the_workspace_entry_on_two_calls(b1, b2):
    h, hkv, dk, w = 8, 2, 64, 512
    for b, seed in ((b1, 1), (b2, 2)):  # the second call with fewer rows
        q, k, v, pos, ring = _case(b, h, hkv, dk, w, seed)
        ring_ws = [t.clone() for t in ring]
        workspace = torch.zeros(b, dtype=torch.int32, device=GPU)
        want = _run("vsp_ring_attn_bf16", q, k, v, pos, ring_ws, h, hkv, dk, w, workspace)
        got = _run("vsp_ring_attn_noalloc_bf16", q, k, v, pos, ring, h, hkv, dk, w)
        torch.cuda.synchronize()
        assert torch.equal(got, want), b
        for mine, theirs in zip(ring, ring_ws):
            assert torch.equal(mine, theirs), b
        assert not bool(workspace.any())  # the workspace entry leaves its counters zero


def test_rows_beyond_the_static_scratch_are_refused_before_any_launch():
    from vesper.kernels import _lib

    lib = _lib.library()
    status = lib.vsp_ring_attn_noalloc_bf16(None, None, None, None, None, None, None, None, None, None,
                                            65537, 8, 8, 64, 512, 0.125, 1, None)
    assert status != 0
    assert "static scratch" in lib.vsp_last_error().decode()
