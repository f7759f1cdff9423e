"""The HIP window attention (``vesper.kernels.window_attn``) against the CPU oracle, through the C ABI.

The oracle runs in float64 (float32 at the full headline size) on the same bf16/fp16-valued inputs.
Bound: relative Frobenius error below 1e-2, and elementwise within the reference's
``rtol = atol = 3e-2`` (``tests/test_window_attn.py:78``), for the outputs and for the gradients of
q, keys and values (the oracle's by autograd, pinned by finite differences in
``tests/test_oracle_attention.py``).
"""

from __future__ import annotations

import pytest
import torch

from conftest import needs_gpu
from oracle.attention import window_attention as oracle_window
from oracle.delta import relative_error

pytestmark = [pytest.mark.gpu, needs_gpu]

GPU = torch.device("cuda")
BF16 = torch.bfloat16


def _inputs(b, n, m, h, hkv, dk, seed=0, dtype=BF16):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(b, n, h, dk, generator=g).to(dtype)
    keys = torch.randn(b, m + n, hkv, dk, generator=g).to(dtype)
    values = torch.randn(b, m + n, hkv, dk, generator=g).to(dtype)
    return q, keys, values


def _check(got, want, rel=1e-2):
    assert relative_error(got, want) < rel
    torch.testing.assert_close(got.float().cpu(), want.float(), rtol=3e-2, atol=3e-2)


# the reference's shapes: h 4, 2 KV heads, dk 64, window 16; chunks shorter and longer than the
# window with an empty, a partial and a full cache (tests/test_window_attn.py:67-78)
@pytest.mark.parametrize(("n", "m"), [(8, 0), (40, 0), (8, 5), (40, 5), (8, 16), (40, 16)])
def test_the_kernel_equals_the_oracle_window(n, m):
    from vesper.kernels.window_attn import window_attention

    q, keys, values = _inputs(3, n, m, 4, 2, 64, seed=n * 100 + m)
    want = oracle_window(q.double(), keys.double(), values.double(), 16)
    got = window_attention(q.to(GPU), keys.to(GPU), values.to(GPU), 16)
    assert got.dtype == BF16 and got.shape == q.shape
    _check(got, want)


@pytest.mark.parametrize("dtype", [BF16, torch.float16])
@pytest.mark.parametrize("dk", [16, 32, 64, 128, 256])
@pytest.mark.parametrize(("n", "m", "w"), [(1, 0, 1), (70, 3, 7), (130, 64, 64), (300, 100, 100), (200, 40, 600)])
def test_widths_windows_and_offsets(dtype, dk, n, m, w):
    from vesper.kernels.window_attn import window_attention

    q, keys, values = _inputs(2, n, m, 4, 1, dk, seed=dk + n + w, dtype=dtype)
    want = oracle_window(q.double(), keys.double(), values.double(), w)
    got = window_attention(q.to(GPU), keys.to(GPU), values.to(GPU), w)
    assert got.dtype == dtype
    _check(got, want)


@pytest.mark.parametrize(("h", "hkv"), [(8, 8), (8, 2), (12, 3), (4, 1)])
def test_grouped_kv_heads(h, hkv):
    from vesper.kernels.window_attn import window_attention

    q, keys, values = _inputs(2, 100, 20, h, hkv, 64, seed=h * 10 + hkv)
    want = oracle_window(q.double(), keys.double(), values.double(), 32)
    _check(window_attention(q.to(GPU), keys.to(GPU), values.to(GPU), 32), want)


def test_headline_config_b4_t4096_h8_d64_w512():
    from vesper.kernels.window_attn import window_attention

    q, keys, values = _inputs(4, 4096, 0, 8, 8, 64, seed=0)
    got = window_attention(q.to(GPU), keys.to(GPU), values.to(GPU), 512)
    want = oracle_window(q.float(), keys.float(), values.float(), 512)
    _check(got, want)


def test_causality_and_the_window_edge_hold_bitwise_at_b4_t4096_h8_d64_w512():
    # the reference's causality and window-boundary properties (tests/test_attention.py:58-147) at
    # the attention config: keys and values changed from position p on leave every earlier query's
    # output unchanged bit for bit, and changed before position p leave every query from p + w - 1 on
    from vesper.kernels.window_attn import window_attention

    q, keys, values = (t.to(GPU) for t in _inputs(4, 4096, 0, 8, 8, 64, seed=59))
    base = window_attention(q, keys, values, 512)
    p, w = 2000, 512
    noise = torch.randn(keys.shape, generator=torch.Generator().manual_seed(60)).to(GPU, BF16)
    late_k, late_v = keys.clone(), values.clone()
    late_k[:, p:] += noise[:, p:]
    late_v[:, p:] -= noise[:, p:]
    after = window_attention(q, late_k, late_v, w)
    assert torch.equal(after[:, :p], base[:, :p]) and not torch.equal(after[:, p:], base[:, p:])
    early_k, early_v = keys.clone(), values.clone()
    early_k[:, :p] += noise[:, :p]
    early_v[:, :p] -= noise[:, :p]
    after = window_attention(q, early_k, early_v, w)
    assert torch.equal(after[:, p + w - 1:], base[:, p + w - 1:])
    assert not torch.equal(after[:, p + w - 2], base[:, p + w - 2])


def test_active_mask_skips_inactive_queries_only():
    from vesper.kernels.window_attn import window_attention

    q, keys, values = _inputs(2, 300, 10, 4, 2, 64, seed=4)
    act = torch.rand(2, 300, generator=torch.Generator().manual_seed(1)) < 0.4
    act[0, 64:128] = False  # a whole tile of 64 queries inactive
    dev = [t.to(GPU) for t in (q, keys, values)]
    full = window_attention(*dev, 48)
    got = window_attention(*dev, 48, active=act.to(GPU))
    a = act.to(GPU)
    assert torch.equal(got[a], full[a])
    assert bool((got[~a] == 0).all())
    want = oracle_window(q.double(), keys.double(), values.double(), 48, active=act)
    _check(got, want)


def test_large_logits_stay_finite_and_match():
    # logits with a standard deviation near 100: exp2 overflows unless every tile's running maximum
    # is the true maximum over the four lane groups of its query (the lazy rescale relies on it)
    from vesper.kernels.window_attn import window_attention

    q, keys, values = _inputs(2, 300, 20, 4, 2, 64, seed=31)
    q, keys = (10 * q.float()).to(BF16), (10 * keys.float()).to(BF16)
    want = oracle_window(q.double(), keys.double(), values.double(), 100)
    got = window_attention(q.to(GPU), keys.to(GPU), values.to(GPU), 100)
    assert bool(torch.isfinite(got).all())
    _check(got, want)


def test_refusals():
    from vesper.contracts import ContractError
    from vesper.kernels.window_attn import window_attention

    q, keys, values = _inputs(1, 8, 0, 4, 2, 64)
    with pytest.raises(ContractError, match="CUDA only"):
        window_attention(q, keys, values, 4)
    dq, dk_, dv = (t.to(GPU) for t in (q, keys, values))
    with pytest.raises(ContractError, match="dtype"):
        window_attention(dq.float(), dk_.float(), dv.float(), 4)
    with pytest.raises(ContractError, match="dtype"):
        window_attention(dq, dk_.half(), dv, 4)
    with pytest.raises(ContractError, match="multiple"):
        window_attention(dq[:, :, :3], dk_, dv, 4)
    with pytest.raises(ContractError, match="fewer"):
        window_attention(dq, dk_[:, :4], dv[:, :4], 4)
    with pytest.raises(ValueError, match="window"):
        window_attention(dq, dk_, dv, 0)
    wide = torch.zeros(1, 8, 4, 264, dtype=BF16, device=GPU)
    with pytest.raises(ContractError, match="exceeds"):
        window_attention(wide, wide[:, :, :2], wide[:, :, :2], 4)


@pytest.mark.parametrize("dk", [8, 24, 48, 96, 192])
def test_widths_between_the_kernels_run_zero_padded(dk):
    """A head width the kernels do not tile runs with zero features up to the next one (scale
    1 / sqrt(dk) kept): outputs and gradients against the oracle at that width, with a cache, grouped
    KV heads and an active mask, and with carried keys and values."""
    from vesper.kernels.window_attn import window_attention

    n, m, w, h, hkv = 150, 30, 48, 4, 2
    q, keys, values = _inputs(2, n, m, h, hkv, dk, seed=dk + 3)
    active = torch.rand(2, n, generator=torch.Generator().manual_seed(dk)) < 0.7
    want = oracle_window(q.double(), keys.double(), values.double(), w, active=active)
    got = window_attention(q.to(GPU), keys.to(GPU), values.to(GPU), w, active=active.to(GPU))
    assert got.shape == q.shape
    _check(got, want)
    up = torch.randn(2, n, h, dk, generator=torch.Generator().manual_seed(dk + 1)).to(BF16)
    g_got = _grads(q, keys, values, w, up)
    g_want = _oracle_grads(q, keys, values, w, up)
    for a, b, name in zip(g_got, g_want, ("o", "dq", "dk", "dv")):
        assert relative_error(a, b) < 1e-2, name
    # carried keys and values: equal to the where-merged inputs
    g = torch.Generator().manual_seed(dk + 2)
    ck = torch.randn(2, n, hkv, dk, generator=g).to(BF16)
    cv = torch.randn(2, n, hkv, dk, generator=g).to(BF16)
    keep = active.reshape(2, n, 1, 1)
    mk = torch.cat([keys[:, :m], torch.where(keep, keys[:, m:], ck)], dim=1)
    mv = torch.cat([values[:, :m], torch.where(keep, values[:, m:], cv)], dim=1)
    with torch.no_grad():
        fused = window_attention(q.to(GPU), keys.to(GPU), values.to(GPU), w, active=active.to(GPU),
                                 carried=(ck.to(GPU), cv.to(GPU)))
        merged = window_attention(q.to(GPU), mk.to(GPU), mv.to(GPU), w, active=active.to(GPU))
    assert torch.equal(fused, merged)


def test_repeatable_and_captured_replays_equal_eager():
    from vesper.kernels.window_attn import window_attention

    q, keys, values = (t.to(GPU) for t in _inputs(2, 500, 16, 8, 2, 64, seed=7))
    eager = window_attention(q, keys, values, 64)
    assert torch.equal(window_attention(q, keys, values, 64), eager)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        window_attention(q, keys, values, 64)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = window_attention(q, keys, values, 64)
    for i in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), i
        window_attention(q, keys, values, 64)
        torch.cuda.synchronize()


def _grads(q, keys, values, w, up, active=None):
    from vesper.kernels.window_attn import window_attention

    qs, ks, vs = (t.to(GPU).requires_grad_() for t in (q, keys, values))
    out = window_attention(qs, ks, vs, w, active=None if active is None else active.to(GPU))
    out.backward(up.to(GPU))
    return out.detach(), qs.grad, ks.grad, vs.grad


def _oracle_grads(q, keys, values, w, up, active=None, dtype=torch.float64):
    qs, ks, vs = (t.to(dtype).requires_grad_() for t in (q, keys, values))
    out = oracle_window(qs, ks, vs, w, active=active)
    out.backward(up.to(dtype))
    return out.detach(), qs.grad, ks.grad, vs.grad


# the reference's gradient cases (tests/test_window_attn.py:67-78): h 4, 2 KV heads, dk 64, window
# 16, chunks shorter and longer than the window, with no cache, a short one and a full one
@pytest.mark.parametrize(("n", "m"), [(8, 0), (40, 0), (8, 5), (40, 5), (8, 16), (40, 16)])
def test_the_gradients_match_the_oracle(n, m):
    q, keys, values = _inputs(3, n, m, 4, 2, 64, seed=40 + n + m)
    up = torch.randn(3, n, 4, 64, generator=torch.Generator().manual_seed(n * m + 1)).to(BF16)
    got = _grads(q, keys, values, 16, up)
    want = _oracle_grads(q, keys, values, 16, up)
    for a, b, name in zip(got, want, ("o", "dq", "dk", "dv")):
        assert relative_error(a, b) < 1e-2, name
        torch.testing.assert_close(a.float().cpu(), b.float(), rtol=3e-2, atol=3e-2, msg=name)


@pytest.mark.parametrize("dk", [16, 32, 64, 128, 256])
@pytest.mark.parametrize(("h", "hkv"), [(2, 2), (8, 1), (8, 4)])
@pytest.mark.parametrize("dtype", [BF16, torch.float16])
def test_the_gradients_for_every_width_and_group(dk, h, hkv, dtype):
    n, m, w = 150, 30, 48
    q, keys, values = _inputs(2, n, m, h, hkv, dk, seed=dk + h, dtype=dtype)
    up = torch.randn(2, n, h, dk, generator=torch.Generator().manual_seed(dk)).to(dtype)
    got = _grads(q, keys, values, w, up)
    want = _oracle_grads(q, keys, values, w, up)
    for a, b, name in zip(got[1:], want[1:], ("dq", "dk", "dv")):
        assert relative_error(a, b) < 1e-2, name


def test_inactive_queries_pass_no_gradient():
    n = 100
    q, keys, values = _inputs(2, n, 10, 4, 2, 64, seed=50)
    active = torch.rand(2, n, generator=torch.Generator().manual_seed(51)) < 0.6
    up = torch.randn(2, n, 4, 64, generator=torch.Generator().manual_seed(52)).to(BF16)
    got = _grads(q, keys, values, 32, up, active)
    want = _oracle_grads(q, keys, values, 32, up, active)
    assert torch.equal(got[1][~active.to(GPU)], torch.zeros_like(got[1][~active.to(GPU)]))
    for a, b, name in zip(got[1:], want[1:], ("dq", "dk", "dv")):
        assert relative_error(a, b) < 1e-2, name


def test_the_gradients_at_t4096_w512_against_the_fp32_oracle_and_they_repeat():
    q, keys, values = _inputs(1, 4096, 0, 8, 8, 64, seed=53)
    up = torch.randn(1, 4096, 8, 64, generator=torch.Generator().manual_seed(54)).to(BF16)
    got = _grads(q, keys, values, 512, up)
    again = _grads(q, keys, values, 512, up)
    for a, b in zip(got, again):
        assert torch.equal(a, b)  # deterministic: no atomics
    want = _oracle_grads(q, keys, values, 512, up, dtype=torch.float32)
    for a, b, name in zip(got[1:], want[1:], ("dq", "dk", "dv")):
        assert relative_error(a, b) < 1e-2, name


# the shape the reference quotes its kernel at (kernels/window_attn.py:10-13: b 16, a 1024-token
# chunk after a 512-row cache, 8 query heads over 2 KV heads, dk 64, window 512), forward and
# every gradient against the float32 oracle (the reference reports 2-4e-3 relative for its kernel)
def test_the_reference_benchmark_shape_b16_n1024_m512_h8_hkv2_d64():
    q, keys, values = _inputs(16, 1024, 512, 8, 2, 64, seed=57)
    up = torch.randn(16, 1024, 8, 64, generator=torch.Generator().manual_seed(58)).to(BF16)
    got = _grads(q, keys, values, 512, up)
    want = _oracle_grads(q, keys, values, 512, up, dtype=torch.float32)
    for a, b, name in zip(got, want, ("o", "dq", "dk", "dv")):
        assert relative_error(a, b) < 1e-2, (name, relative_error(a, b))


def test_captured_forward_and_backward_equal_eager():
    from vesper.kernels.window_attn import window_attention

    q, keys, values = (t.to(GPU).requires_grad_() for t in _inputs(2, 300, 16, 8, 2, 64, seed=55))
    up = torch.randn(2, 300, 8, 64, generator=torch.Generator().manual_seed(56)).to(GPU, BF16)

    def step():
        out = window_attention(q, keys, values, 64)
        return (out.detach(), *torch.autograd.grad(out, (q, keys, values), up))

    eager = [t.clone() for t in step()]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        static = step()
    for _ in range(3):
        for t in static:
            t.zero_()
        graph.replay()
        torch.cuda.synchronize()
        for a, b in zip(static, eager):
            assert torch.equal(a, b)


# ---- copy-forward read inside the tile loads (carried keys and values of inactive tokens) ----

def _carry_case(b, n, m, h, hkv, dk, seed, dtype=BF16, frac=0.4):
    q, keys, values = (t.to(GPU) for t in _inputs(b, n, m, h, hkv, dk, seed, dtype))
    g = torch.Generator().manual_seed(seed + 1)
    kc = torch.randn(b, n, hkv, dk, generator=g).to(GPU, dtype)
    vc = torch.randn(b, n, hkv, dk, generator=g).to(GPU, dtype)
    active = (torch.rand(b, n, generator=g) >= frac).to(GPU)
    return q, keys, values, (kc, vc), active


def _merged_kv(keys, values, carried, active):
    m = keys.shape[1] - active.shape[1]
    keep = active[..., None, None]
    return (torch.cat([keys[:, :m], torch.where(keep, keys[:, m:], carried[0])], dim=1),
            torch.cat([values[:, :m], torch.where(keep, values[:, m:], carried[1])], dim=1))


@pytest.mark.parametrize("dtype", [BF16, torch.float16])
@pytest.mark.parametrize("dk", [16, 32, 64, 128, 256])
@pytest.mark.parametrize(("n", "m", "w", "h", "hkv"), [(70, 0, 16, 4, 2), (200, 40, 64, 8, 2), (300, 100, 600, 4, 4)])
def test_carried_keys_and_values_equal_the_merged_ones_bitwise(dtype, dk, n, m, w, h, hkv):
    from vesper.kernels.window_attn import window_attention

    q, keys, values, carried, active = _carry_case(2, n, m, h, hkv, dk, seed=dk + n, dtype=dtype)
    # the fresh rows of inactive tokens must never be read: poison them
    hold = torch.cat([torch.zeros(2, m, dtype=torch.bool, device=GPU), ~active], dim=1)[..., None, None]
    keys, values = keys.masked_fill(hold, float("nan")), values.masked_fill(hold, float("nan"))
    got = window_attention(q, keys, values, w, active=active, carried=carried)
    want = window_attention(q, *_merged_kv(keys, values, carried, active), w, active=active)
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    assert bool(torch.isfinite(got).all())


@pytest.mark.parametrize("pattern", ["all_active", "all_held", "alternating", "tail_held"])
def test_carried_keys_on_every_flag_pattern(pattern):
    from vesper.kernels.window_attn import window_attention

    b, n, m = 2, 260, 30
    q, keys, values, carried, _ = _carry_case(b, n, m, 4, 2, 64, seed=4)
    t = torch.arange(n, device=GPU).expand(b, n)
    active = {"all_active": t >= 0, "all_held": t < 0, "alternating": t % 2 == 0, "tail_held": t < 200}[pattern]
    got = window_attention(q, keys, values, 100, active=active, carried=carried)
    mk, mv = _merged_kv(keys, values, carried, active)
    want = window_attention(q, mk, mv, 100, active=active)
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    ref = oracle_window(q.double().cpu(), mk.double().cpu(), mv.double().cpu(), 100) * active[..., None, None].cpu()
    _check(got, ref)


def test_carried_keys_at_b4_t4096_h8_d64_w512():
    from vesper.kernels.window_attn import window_attention

    q, keys, values, carried, active = _carry_case(4, 4096, 0, 8, 8, 64, seed=6, frac=0.3)
    got = window_attention(q, keys, values, 512, active=active, carried=carried)
    want = window_attention(q, *_merged_kv(keys, values, carried, active), 512, active=active)
    torch.cuda.synchronize()
    assert torch.equal(got, want)


def test_carried_keys_under_autograd_route_gradients_to_the_carried_tensors():
    from vesper.kernels.window_attn import window_attention

    q, keys, values, carried, active = _carry_case(2, 80, 10, 4, 2, 32, seed=8)
    leaves = [t.clone().requires_grad_() for t in (keys, values, *carried)]
    window_attention(q, leaves[0], leaves[1], 16, active=active, carried=tuple(leaves[2:])).float().square().sum().backward()
    ref = [t.clone().requires_grad_() for t in (keys, values, *carried)]
    window_attention(q, *_merged_kv(ref[0], ref[1], tuple(ref[2:]), active), 16, active=active).float().square().sum().backward()
    for got, want in zip(leaves, ref):
        assert torch.equal(got.grad, want.grad)
    assert not bool(leaves[2].grad[active].any())


def test_carried_refusals():
    from vesper.contracts import ContractError
    from vesper.kernels.window_attn import window_attention

    q, keys, values, carried, active = _carry_case(1, 20, 4, 2, 2, 16, seed=2)
    with pytest.raises(ContractError, match="active"):
        window_attention(q, keys, values, 8, carried=carried)
    with pytest.raises(ContractError, match="carried keys"):
        window_attention(q, keys, values, 8, active=active, carried=(keys, carried[1]))
    with pytest.raises(ContractError, match="carried holds"):
        window_attention(q, keys, values, 8, active=active, carried=carried[:1])
