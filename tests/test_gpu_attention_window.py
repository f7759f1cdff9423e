"""The attention sublayer's pieces around the window kernel (``vesper.attention``) on the GPU:
the rotary embedding (``vsp_rotary_qk_*``), the window carried across chunks
(``vsp_kv_cache_push``) and ``attend`` over a cache, against the CPU oracle.

Parity: the rotary kernel computes the phases in float64 and the rotation in the activations'
dtype as the reference does, so it equals the oracle's ``rotary`` bitwise (the reference's own
known answers and precision cases included); the cache push is a selection, bitwise; attention
over a cache at the reference's bound (relative Frobenius 1e-2, elementwise ``rtol = atol =
3e-2``, ``tests/test_window_attn.py:67-78``) against the oracle over the whole sequence.
"""

from __future__ import annotations

import pytest
import torch

from conftest import needs_gpu, reference_vectors
from oracle import attention as oa
from oracle.delta import relative_error

pytestmark = [pytest.mark.gpu, needs_gpu]

GPU = torch.device("cuda")
BF16 = torch.bfloat16


@pytest.mark.parametrize("dtype", [BF16, torch.float16, torch.float32])
@pytest.mark.parametrize("dk", [2, 16, 64, 128])
def test_rotary_equals_the_oracle_bitwise(dtype, dk):
    from vesper.attention import rotary, rotary_qk

    g = torch.Generator().manual_seed(dk)
    b, n, h, hkv = 2, 37, 4, 2
    q = torch.randn(b, n, h, dk, generator=g).to(dtype)
    k = torch.randn(b, n, hkv, dk, generator=g).to(dtype)
    pos = torch.randint(0, 70000 if dtype != torch.float16 else 60000, (b, n), generator=g)
    pos[0] = torch.arange(n)  # including position 0: the identity
    want_q, want_k = oa.rotary(q, pos, 10000.0), oa.rotary(k, pos, 10000.0)
    got_q, got_k = rotary_qk(q.to(GPU), k.to(GPU), pos.to(GPU), 10000.0)
    assert torch.equal(got_q.cpu(), want_q) and torch.equal(got_k.cpu(), want_k)
    assert torch.equal(rotary(q.to(GPU), pos.to(GPU), 10000.0).cpu(), want_q)
    assert torch.equal(got_q[0, 0].cpu(), q[0, 0])


def test_rotary_known_answers_and_precision_cases():
    from vesper.attention import rotary

    c = reference_vectors()["rotary"]
    base = float(c["base"])
    pos = torch.full((1, 1), c["position"], dtype=torch.long, device=GPU)
    for case in c["pairs"]:  # float32 here: the known answers within float32's rounding
        x = torch.tensor([[[[float(v) for v in case["x"]]]]], device=GPU)
        want = torch.tensor([float(v) for v in case["want"]], dtype=torch.float64)
        assert torch.allclose(rotary(x, pos, base)[0, 0, 0].cpu().double(), want, rtol=0, atol=1e-7)
    import math

    for dtype_name, position, atol in c["precision"]:
        dtype = getattr(torch, dtype_name)
        x = torch.zeros(1, 2, 1, 2, dtype=dtype)
        x[..., 0] = 1.0
        r = rotary(x.to(GPU), torch.tensor([[position, position + 1]], device=GPU), base).cpu()
        want = torch.tensor([[math.cos(position), math.sin(position)],
                             [math.cos(position + 1), math.sin(position + 1)]], dtype=torch.float64)
        assert r.dtype == dtype and not torch.equal(r[0, 0], r[0, 1])
        assert torch.allclose(r[0, :, 0, :].double(), want, rtol=0, atol=float(atol)), dtype_name


def test_rotary_gradients_and_refusals():
    from vesper.attention import rotary, rotary_qk
    from vesper.contracts import ContractError

    g = torch.Generator().manual_seed(5)
    q = torch.randn(2, 9, 4, 16, generator=g, dtype=torch.float64)
    k = torch.randn(2, 9, 2, 16, generator=g, dtype=torch.float64)
    pos = torch.randint(0, 5000, (2, 9), generator=g)
    uq, uk = torch.randn(q.shape, generator=g, dtype=torch.float64), torch.randn(k.shape, generator=g, dtype=torch.float64)
    qr, kr = q.clone().requires_grad_(), k.clone().requires_grad_()
    ((oa.rotary(qr, pos, 10000.0) * uq).sum() + (oa.rotary(kr, pos, 10000.0) * uk).sum()).backward()
    qg, kg = q.float().to(GPU).requires_grad_(), k.float().to(GPU).requires_grad_()
    a, b_ = rotary_qk(qg, kg, pos.to(GPU), 10000.0)
    ((a * uq.float().to(GPU)).sum() + (b_ * uk.float().to(GPU)).sum()).backward()
    torch.testing.assert_close(qg.grad.cpu().double(), qr.grad, rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(kg.grad.cpu().double(), kr.grad, rtol=1e-5, atol=1e-5)
    x = torch.zeros(1, 2, 1, 4, device=GPU)
    with pytest.raises(ContractError, match="axis"):
        rotary(x, torch.zeros(2, 2, dtype=torch.long, device=GPU), 10000.0)
    with pytest.raises(ValueError, match="even"):
        rotary(torch.zeros(1, 2, 1, 3, device=GPU), torch.zeros(1, 2, dtype=torch.long, device=GPU), 10000.0)
    with pytest.raises(ValueError, match="above 1"):
        rotary(x, torch.zeros(1, 2, dtype=torch.long, device=GPU), 1.0)


@pytest.mark.parametrize(("m", "n"), [(0, 5), (3, 2), (8, 0), (8, 3), (2, 13), (0, 20)])
def test_the_cache_push_equals_the_oracle(m, n):
    from vesper.attention import KVCache, kv_cache_push

    w = 8
    g = torch.Generator().manual_seed(10 * m + n)
    ck, cv = (torch.randn(2, m, 2, 16, generator=g).to(BF16) for _ in range(2))
    cp = torch.arange(100, 100 + m).expand(2, m).contiguous()
    k, v = (torch.randn(2, n, 2, 16, generator=g).to(BF16) for _ in range(2))
    pos = torch.arange(100 + m, 100 + m + n).expand(2, n).contiguous()
    cache = KVCache(ck.to(GPU), cv.to(GPU), cp.to(GPU), w)
    got = kv_cache_push(cache, k.to(GPU), v.to(GPU), pos.to(GPU))
    wk, wv, wp = oa.kv_cache_push(ck, cv, cp, k, v, pos, w)
    assert torch.equal(got.k.cpu(), wk) and torch.equal(got.v.cpu(), wv) and torch.equal(got.pos.cpu(), wp)
    assert got.window == w and (n > 0 or got is cache)


def test_two_chunks_through_the_cache_equal_the_whole_sequence():
    # the window carried across chunks (attention.py:340-407 with kv_cache_push): chunk 2 sees the
    # last w rows of chunk 1 through the cache (m = w), as the whole sequence would
    from vesper.attention import attend, kv_cache_empty

    b, h, hkv, dk, w = 2, 4, 2, 64, 64
    g = torch.Generator().manual_seed(3)
    n1, n2 = 150, 97
    q = torch.randn(b, n1 + n2, h, dk, generator=g).to(BF16)
    k = torch.randn(b, n1 + n2, hkv, dk, generator=g).to(BF16)
    v = torch.randn(b, n1 + n2, hkv, dk, generator=g).to(BF16)
    pos = torch.arange(n1 + n2).expand(b, n1 + n2).contiguous()
    cache = kv_cache_empty(b, hkv, dk, w, BF16, GPU)
    o1, cache = attend(q[:, :n1].to(GPU), k[:, :n1].to(GPU), v[:, :n1].to(GPU), pos[:, :n1].to(GPU), cache)
    assert cache.k.shape[1] == w and torch.equal(cache.pos.cpu(), pos[:, n1 - w:n1])
    o2, cache = attend(q[:, n1:].to(GPU), k[:, n1:].to(GPU), v[:, n1:].to(GPU), pos[:, n1:].to(GPU), cache)
    want = oa.window_attention(q.double(), k.double(), v.double(), w)
    got = torch.cat([o1, o2], dim=1)
    assert relative_error(got, want) < 1e-2
    torch.testing.assert_close(got.cpu().double(), want, rtol=3e-2, atol=3e-2)
    assert torch.equal(cache.k.cpu(), k[:, -w:])


def test_float32_attend_takes_the_blocked_branch_and_chunks_equal_the_whole_sequence():
    # float32 activations (attention.py:384-407): two chunks through the cache against the oracle
    # over the whole sequence, and the gradients of q, k, v (float32 against float64 on the CPU)
    from vesper.attention import attend, kv_cache_empty

    b, h, hkv, dk, w = 2, 4, 2, 32, 48
    g = torch.Generator().manual_seed(5)
    n1, n2 = 70, 131
    q = torch.randn(b, n1 + n2, h, dk, generator=g)
    k, v = (torch.randn(b, n1 + n2, hkv, dk, generator=g) for _ in range(2))
    dout = torch.randn(b, n1 + n2, h, dk, generator=g)
    pos = torch.arange(n1 + n2).expand(b, n1 + n2).contiguous()
    qg, kg, vg = (t.to(GPU).requires_grad_() for t in (q, k, v))
    cache = kv_cache_empty(b, hkv, dk, w, torch.float32, GPU)
    o1, cache = attend(qg[:, :n1], kg[:, :n1], vg[:, :n1], pos[:, :n1].to(GPU), cache)
    o2, cache = attend(qg[:, n1:], kg[:, n1:], vg[:, n1:], pos[:, n1:].to(GPU), cache)
    got = torch.cat([o1, o2], dim=1)
    (got * dout.to(GPU)).sum().backward()
    qd, kd, vd = (t.double().requires_grad_() for t in (q, k, v))
    want = oa.window_attention(qd, kd, vd, w)
    (want * dout.double()).sum().backward()
    assert got.dtype == torch.float32 and cache.k.shape[1] == w
    torch.testing.assert_close(got.detach().cpu().double(), want.detach(), rtol=1e-5, atol=1e-5)
    for name, a, e in (("q", qg, qd), ("k", kg, kd), ("v", vg, vd)):
        torch.testing.assert_close(a.grad.cpu().double(), e.grad, rtol=1e-4, atol=1e-4, msg=name)
    assert torch.equal(cache.k.detach().cpu(), k[:, -w:]) and torch.equal(cache.pos.cpu(), pos[:, -w:])


def test_a_second_4096_token_chunk_with_a_full_window_cache_at_b4_h8_d64_w512():
    # the prefill attention config's shape, continued: chunk 2 of 4096 tokens over the 512-entry
    # cache chunk 1 left, against the oracle over the 8192-token sequence (float32 on the CPU)
    from vesper.attention import attend, kv_cache_empty

    b, h, dk, w, n = 4, 8, 64, 512, 4096
    g = torch.Generator().manual_seed(4)
    q, k, v = (torch.randn(b, 2 * n, h, dk, generator=g).to(BF16) for _ in range(3))
    pos = torch.arange(2 * n).expand(b, 2 * n).contiguous()
    cache = kv_cache_empty(b, h, dk, w, BF16, GPU)
    _, cache = attend(q[:, :n].to(GPU), k[:, :n].to(GPU), v[:, :n].to(GPU), pos[:, :n].to(GPU), cache)
    o2, cache = attend(q[:, n:].to(GPU), k[:, n:].to(GPU), v[:, n:].to(GPU), pos[:, n:].to(GPU), cache)
    keys, vals = k[:, n - w:].float(), v[:, n - w:].float()
    want = oa.window_attention(q[:, n:].float(), keys, vals, w)
    assert relative_error(o2, want) < 1e-2
    assert torch.equal(cache.pos.cpu(), pos[:, -w:])


@pytest.mark.parametrize("dtype", [BF16, torch.float16])
@pytest.mark.parametrize("dk", [16, 32, 64, 128, 256])
@pytest.mark.parametrize(("m", "n", "w"), [(1, 70, 64), (37, 130, 64), (64, 200, 64), (100, 64, 128), (300, 700, 512),
                                            (512, 300, 512), (511, 1, 512)])
def test_the_cache_and_the_chunk_as_two_sources_equal_their_concatenation_bitwise(dtype, dk, m, n, w):
    """vsp_window_attn_cached_*: key rows below m from the cache, the rest from the chunk, with the
    tile across row m (m not a multiple of 64, or straddling the window) read row by row; outputs
    equal the one-tensor kernel over the concatenated keys bit for bit, GQA included."""
    from vesper.kernels.window_attn import window_attention, window_attention_cached

    b, h, hkv = 2, 4, 2
    g = torch.Generator().manual_seed(m + n + dk)
    q = torch.randn(b, n, h, dk, generator=g).to(dtype).to(GPU)
    ck, cv = (torch.randn(b, m, hkv, dk, generator=g).to(dtype).to(GPU) for _ in range(2))
    k, v = (torch.randn(b, n, hkv, dk, generator=g).to(dtype).to(GPU) for _ in range(2))
    with torch.no_grad():
        got = window_attention_cached(q, ck, cv, k, v, w)
        want = window_attention(q, torch.cat([ck, k], 1), torch.cat([cv, v], 1), w)
    torch.cuda.synchronize()
    assert torch.equal(got, want)


def test_attend_refuses_positions_that_are_not_consecutive():
    from vesper.attention import attend, kv_cache_empty
    from vesper.contracts import ContractError

    q = torch.zeros(1, 4, 2, 16, dtype=BF16, device=GPU)
    k = torch.zeros(1, 4, 2, 16, dtype=BF16, device=GPU)
    with pytest.raises(ContractError, match="consecutive"):
        attend(q, k, k, torch.tensor([[0, 1, 3, 4]], device=GPU), kv_cache_empty(1, 2, 16, 8, BF16, GPU))
