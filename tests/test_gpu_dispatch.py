"""Dispatch proofs: the product entry points reach the HIP library's kernels, and the reference scan
does not.

Like the reference's spy on its CUDA call (tests/test_window_attn.py:91-123) and its check that a
sublayer switched to "fused" reaches the kernel (tests/test_delta_scan_fused.py:169-178), each test
wraps the one function through which Python calls the C ABI (``vesper.kernels._lib.call``) and
records the entry points a call reaches.
"""

from __future__ import annotations

import pytest
import torch

from conftest import needs_gpu, scan_inputs

pytestmark = [pytest.mark.gpu, needs_gpu]

GPU = torch.device("cuda")


@pytest.fixture
def calls(monkeypatch: pytest.MonkeyPatch) -> list[str]:
    from vesper.kernels import _lib

    seen: list[str] = []
    real = _lib.call

    def spy(name: str, *args: object) -> None:
        seen.append(name)
        real(name, *args)

    monkeypatch.setattr(_lib, "call", spy)
    return seen


def test_the_scan_switch_reaches_the_kernels_and_the_reference_does_not(calls):
    from vesper.column import recurrent_scan

    q, k, v, beta, h0 = (t.to(GPU) for t in scan_inputs(1, 130, 2, 64, seed=5))
    recurrent_scan("fused", q, k, v, beta, h0)
    assert calls == ["vsp_delta_scan_bf16"], calls
    calls.clear()
    recurrent_scan("fused-fp32", q, k, v, beta, h0)
    assert calls == ["vsp_delta_scan_f32"], calls
    calls.clear()
    recurrent_scan("reference", q, k, v, beta, h0)
    assert calls == [], calls


def test_the_scan_gradient_runs_the_backward_kernel(calls):
    from vesper.kernels.delta_scan import delta_scan_fused

    q, k, v, beta, h0 = (t.to(GPU) for t in scan_inputs(1, 130, 2, 64, seed=6))
    leaves = [t.to(torch.bfloat16).requires_grad_() for t in (q, k, v, beta)]
    o, s = delta_scan_fused(*leaves, h0)
    (o.float().sum() + s.sum()).backward()
    assert calls == ["vsp_delta_scan_record_bf16", "vsp_delta_scan_backward_recorded_bf16"], calls


def test_attend_reaches_the_window_kernels_and_the_cache_push(calls):
    from vesper.attention import attend, kv_cache_empty

    g = torch.Generator().manual_seed(7)
    b, n, h, hkv, dk, w = 2, 96, 4, 2, 64, 64
    q = torch.randn(b, n, h, dk, generator=g).to(GPU, torch.bfloat16)
    k = torch.randn(b, n, hkv, dk, generator=g).to(GPU, torch.bfloat16)
    v = torch.randn(b, n, hkv, dk, generator=g).to(GPU, torch.bfloat16)
    cache = kv_cache_empty(b, hkv, dk, w, torch.bfloat16, GPU)
    pos = torch.arange(n, device=GPU).expand(b, n).contiguous()
    _, cache = attend(q, k, v, pos, cache)  # an empty cache: the chunk alone, the plain kernel
    assert calls == ["vsp_window_attn_bf16", "vsp_kv_cache_push"], calls
    calls.clear()
    _, cache = attend(q, k, v, pos + n, cache)  # a second chunk over the 64-row cache
    assert calls == ["vsp_window_attn_cached_bf16", "vsp_kv_cache_push"], calls


def test_ring_attention_reaches_the_ring_kernel(calls):
    from vesper.kernels.ring_attn import kv_ring_empty, ring_attention

    g = torch.Generator().manual_seed(8)
    b, h, hkv, dk, w = 3, 4, 2, 64, 32
    ring = kv_ring_empty(b, hkv, dk, w, torch.bfloat16, GPU)
    for p in range(3):
        q = torch.randn(b, 1, h, dk, generator=g).to(GPU, torch.bfloat16)
        k = torch.randn(b, 1, hkv, dk, generator=g).to(GPU, torch.bfloat16)
        v = torch.randn(b, 1, hkv, dk, generator=g).to(GPU, torch.bfloat16)
        _, ring = ring_attention(q, k, v, torch.full((b, 1), p, dtype=torch.long, device=GPU), ring)
    assert calls and all(name.startswith("vsp_ring_attn") for name in calls), calls
