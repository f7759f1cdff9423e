"""Pins of the CPU attention oracle (``oracle/attention.py``) against what the mathematics fixes.

Expected values come from scalar arithmetic (the reference's two-token and GQA cases), the ring
example with positions out of slot order, equality of three independent formulations (index
window, blocked position window, ring decoding), and window-edge / causality probes.
"""

from __future__ import annotations

import math

import pytest
import torch

from conftest import frac_tensor, reference_vectors
from oracle import attention as oa

F64 = torch.float64


def test_two_tokens_match_scalar_arithmetic() -> None:
    s1, c1 = math.sin(1.0), math.cos(1.0)
    q = torch.tensor([[[1.0, 0.0]], [[-s1, c1]]], dtype=F64).reshape(1, 2, 1, 2)
    v = torch.tensor([[[2.0, 0.0]], [[0.0, 3.0]]], dtype=F64).reshape(1, 2, 1, 2)
    out = oa.window_attention(q, q, v, window=reference_vectors()["attention_two_token"]["window"])
    z0, z1 = -s1 / math.sqrt(2.0), 1.0 / math.sqrt(2.0)
    a = math.exp(z0) / (math.exp(z0) + math.exp(z1))
    want = torch.tensor([[2.0, 0.0], [2 * a, 3 * (1 - a)]], dtype=F64)
    assert torch.allclose(out[0, :, 0], want, rtol=0, atol=1e-12)


def test_gqa_query_heads_read_their_group() -> None:
    c = reference_vectors()["attention_gqa"]
    kv = frac_tensor(c["kv_values"]).reshape(1, 1, 2, 2)
    q = torch.randn(1, 1, 4, 2, dtype=F64)
    out = oa.window_attention(q, torch.zeros_like(kv), kv, window=1)
    assert torch.allclose(out[0, 0], frac_tensor(c["want_heads"]), rtol=0, atol=1e-12)


def test_a_ring_attends_by_position_not_by_slot_order() -> None:
    c = reference_vectors()["ring_by_position"]
    w = c["window"]
    vals = frac_tensor(c["ring_values"]).reshape(1, w, 1, 1).expand(1, w, 1, 2).contiguous()
    ring_pos = torch.tensor([c["ring_pos"]])
    valid = torch.ones(1, w, dtype=torch.bool)
    q = torch.zeros(1, 1, 1, 2, dtype=F64)
    k = torch.zeros(1, 1, 1, 2, dtype=F64)
    v = torch.full((1, 1, 1, 2), float(frac_tensor([c["new_value"]])[0]), dtype=F64)
    pos = torch.tensor([[c["new_pos"]]])
    out = oa.ring_attend(q, k, v, pos, torch.zeros_like(vals), vals, ring_pos, valid, w)
    want = float(frac_tensor([c["want"]])[0])
    assert torch.allclose(out, torch.full_like(out, want), rtol=0, atol=1e-12)
    wrong = float(frac_tensor([c["wrong_if_slot_order"]])[0])
    assert abs(float(out[0, 0, 0, 0]) - wrong) > 1.0
    _, nv, npos, nvalid = oa.kv_ring_write(torch.zeros_like(vals), vals, ring_pos, valid, k, v, pos)
    assert npos.tolist() == [c["pos_after_write"]]
    assert float(nv[0, c["new_pos"] % w, 0, 0]) == float(frac_tensor([c["new_value"]])[0])
    assert bool(nvalid.all())


def test_ring_rows_write_their_own_slots() -> None:
    c = reference_vectors()["ring_rows_write_own_slots"]
    ring = torch.zeros(2, 4, 1, 2, dtype=F64)
    pos = torch.tensor([[p] for p in c["positions"]])
    _, _, npos, nvalid = oa.kv_ring_write(
        ring, ring, torch.zeros(2, 4, dtype=torch.long), torch.zeros(2, 4, dtype=torch.bool),
        torch.ones(2, 1, 1, 2, dtype=F64), torch.ones(2, 1, 1, 2, dtype=F64), pos,
    )
    assert nvalid.tolist() == c["valid_after"]
    assert int(npos[0, 1]) == c["positions"][0]


def _qkv(b: int, n: int, h: int, hkv: int, dk: int, seed: int = 0):
    g = torch.Generator().manual_seed(seed)
    return (
        torch.randn(b, n, h, dk, generator=g, dtype=F64),
        torch.randn(b, n, hkv, dk, generator=g, dtype=F64),
        torch.randn(b, n, hkv, dk, generator=g, dtype=F64),
    )


def test_blocked_positions_equal_the_full_mask_with_a_prefilled_cache() -> None:
    b, m, n, h, hkv, dk, w = 2, 20, 130, 4, 2, 8, 16
    cq, ck, cv = _qkv(b, m, h, hkv, dk, seed=2)
    q, k, v = _qkv(b, n, h, hkv, dk, seed=3)
    cpos = torch.arange(m).expand(b, m)
    pos = torch.arange(m, m + n).expand(b, n)
    kk, vv, kp = oa.kv_cache_push(ck[:, :0], cv[:, :0], cpos[:, :0], ck, cv, cpos, w)
    blocked = oa.attend_positions(q, k, v, pos, kk, vv, kp, w)
    full = oa.attention_full_mask(q, torch.cat([kk, k], 1), torch.cat([vv, v], 1), pos, torch.cat([kp, pos], 1), w)
    assert (blocked - full).abs().max().item() < 1e-10
    # the index-space form over the same consecutive keys
    index = oa.window_attention(q, torch.cat([kk, k], 1), torch.cat([vv, v], 1), w, block=7)
    assert (index - full).abs().max().item() < 1e-10


def test_ring_decoding_equals_the_growing_cache_and_the_whole_chunk() -> None:
    b, h, hkv, dk, w, start = 2, 4, 2, 8, 16, 7
    steps = 3 * w + 5
    q, k, v = _qkv(b, steps, h, hkv, dk, seed=4)
    pos = torch.arange(start, start + steps).expand(b, steps)
    whole = oa.window_attention(q, k, v, w)
    rk, rv = torch.zeros(b, w, hkv, dk, dtype=F64), torch.zeros(b, w, hkv, dk, dtype=F64)
    rpos, rvalid = torch.zeros(b, w, dtype=torch.long), torch.zeros(b, w, dtype=torch.bool)
    ck, cv, cp = k[:, :0], v[:, :0], pos[:, :0]
    for i in range(steps):
        sl = slice(i, i + 1)
        y_ring = oa.ring_attend(q[:, sl], k[:, sl], v[:, sl], pos[:, sl], rk, rv, rpos, rvalid, w)
        y_grow = oa.attend_positions(q[:, sl], k[:, sl], v[:, sl], pos[:, sl], ck, cv, cp, w)
        assert torch.allclose(y_ring, y_grow, rtol=0, atol=1e-12)
        assert torch.allclose(y_ring, whole[:, sl], rtol=0, atol=1e-12)
        rk, rv, rpos, rvalid = oa.kv_ring_write(rk, rv, rpos, rvalid, k[:, sl], v[:, sl], pos[:, sl])
        ck, cv, cp = oa.kv_cache_push(ck, cv, cp, k[:, sl], v[:, sl], pos[:, sl], w)
        assert torch.equal(rpos[0][rvalid[0]].sort().values, cp[0])


def test_window_edge_is_exact_and_nothing_leaks_from_the_future() -> None:
    w, n = 16, 48
    q, k, v = _qkv(1, n, 2, 2, 8, seed=5)
    base = oa.window_attention(q, k, v, w)
    i = 2 * w + 3
    far = v.clone()
    far[:, i - w] += 1.0  # one index past the window's oldest key
    assert (oa.window_attention(q, k, far, w)[:, i] - base[:, i]).abs().max().item() < 1e-12
    near = v.clone()
    near[:, i - w + 1] += 1.0  # the oldest key inside the window
    assert (oa.window_attention(q, k, near, w)[:, i] - base[:, i]).abs().max().item() > 1e-6
    j = 17
    bumped = k.clone()
    bumped[:, j] += 1.0
    moved = oa.window_attention(q, bumped, v, w)
    assert (moved[:, :j] - base[:, :j]).abs().max().item() < 1e-12
    assert (moved[:, j:] - base[:, j:]).abs().max().item() > 1e-6


def test_window_one_copies_the_own_value() -> None:
    q, k, v = _qkv(2, 9, 4, 4, 8, seed=6)
    assert torch.allclose(oa.window_attention(q, k, v, 1), v, rtol=0, atol=1e-12)


def test_cache_push_keeps_the_newest_window() -> None:
    c = reference_vectors()["cache_push"]
    w = c["window"]
    k = torch.randn(1, 4096, 1, 2, dtype=F64)
    ck, cv, cp = oa.kv_cache_push(k[:, :0], k[:, :0], torch.zeros(1, 0, dtype=torch.long), k, k, torch.arange(4096)[None], w)
    assert torch.equal(ck, k[:, -w:])
    for step in range(4096, 4096 + 40):
        ck, cv, cp = oa.kv_cache_push(ck, cv, cp, k[:, :1], k[:, :1], torch.tensor([[step]]), w)
    assert int(cp[0, 0]) == c["first_pos_after"] and int(cp[0, -1]) == c["last_pos_after"]


def test_active_mask_zeroes_inactive_queries_only() -> None:
    q, k, v = _qkv(2, 30, 4, 2, 8, seed=7)
    active = torch.rand(2, 30, generator=torch.Generator().manual_seed(8)) < 0.5
    full = oa.window_attention(q, k, v, 8)
    got = oa.window_attention(q, k, v, 8, active=active)
    assert torch.equal(got[active], full[active])
    assert bool((got[~active] == 0).all())


@pytest.mark.parametrize("kind", ["off_by_one", "no_scale", "gqa_modulo"])
def test_planted_mistakes_are_caught(kind: str, monkeypatch: pytest.MonkeyPatch) -> None:
    original_full = oa.attention_full_mask
    original_expand = oa._expand_kv

    def wrong_full(q, keys, values, qpos, kpos, window):
        if kind == "off_by_one":
            return original_full(q, keys, values, qpos, kpos, window + 1)
        if kind == "no_scale":
            return original_full(q * math.sqrt(q.shape[-1]), keys, values, qpos, kpos, window)
        return original_full(q, keys, values, qpos, kpos, window)

    def wrong_expand(x, heads):
        if kind == "gqa_modulo":
            return x.repeat(1, 1, heads // x.shape[2], 1)
        return original_expand(x, heads)

    monkeypatch.setattr(oa, "attention_full_mask", wrong_full)
    monkeypatch.setattr(oa, "_expand_kv", wrong_expand)
    caught = []
    try:
        test_two_tokens_match_scalar_arithmetic()
        test_gqa_query_heads_read_their_group()
        test_window_edge_is_exact_and_nothing_leaks_from_the_future()
        caught.append(False)
    except AssertionError:
        caught.append(True)
    assert caught == [True]


def test_the_window_attention_gradients_match_finite_differences() -> None:
    # the oracle of the backward is autograd through the forward above; finite differences pin it
    # (grouped heads, a cache in front of the chunk, a window shorter than the keys, an inactive query)
    g = torch.Generator().manual_seed(31)
    b, n, m, h, hkv, dk, w = 1, 5, 2, 2, 1, 3, 3
    q = torch.randn(b, n, h, dk, generator=g, dtype=torch.float64, requires_grad=True)
    k = torch.randn(b, m + n, hkv, dk, generator=g, dtype=torch.float64, requires_grad=True)
    v = torch.randn(b, m + n, hkv, dk, generator=g, dtype=torch.float64, requires_grad=True)
    active = torch.tensor([[True, True, False, True, True]])
    assert torch.autograd.gradcheck(lambda a, c, e: oa.window_attention(a, c, e, w, active=active), (q, k, v))
    # an inactive query passes no gradient
    out = oa.window_attention(q, k, v, w, active=active)
    gq, _, _ = torch.autograd.grad(out.sum(), (q, k, v))
    assert torch.equal(gq[:, 2], torch.zeros_like(gq[:, 2]))


def test_a_planted_scale_mistake_changes_the_gradients() -> None:
    g = torch.Generator().manual_seed(32)
    q = torch.randn(1, 4, 1, 4, generator=g, dtype=torch.float64, requires_grad=True)
    k = torch.randn(1, 4, 1, 4, generator=g, dtype=torch.float64, requires_grad=True)
    v = torch.randn(1, 4, 1, 4, generator=g, dtype=torch.float64)
    (gq,) = torch.autograd.grad(oa.window_attention(q, k, v, 4).sum(), (q,))
    (wrong,) = torch.autograd.grad(oa.window_attention(2 * q, k, v, 4).sum(), (q,))  # a doubled score scale
    assert not torch.allclose(gq, wrong, rtol=1e-3)


def test_rotary_pairs_match_the_reference_scalar_trig():
    # tests/test_attention_independent.py:66-79: at position 2, pair 0 turns by 2 rad, pair 1 by
    # 2 / sqrt(base) (base^(-2/4)); a planted mistake (the pair's partner of the wrong sign, or
    # base^(-j/dk)) fails it
    from conftest import reference_vectors

    c = reference_vectors()["rotary"]
    base = float(c["base"])
    pos = torch.full((1, 1), c["position"], dtype=torch.long)
    for case in c["pairs"]:
        x = torch.tensor([[[[float(v) for v in case["x"]]]]], dtype=torch.float64)
        want = torch.tensor([float(v) for v in case["want"]], dtype=torch.float64)
        assert torch.allclose(oa.rotary(x, pos, base)[0, 0, 0], want, rtol=0, atol=1e-12)
    x = torch.tensor([[[[1.0, 0.0, 1.0, 0.0]]]], dtype=torch.float64)
    wrong = torch.stack([x[..., 0::2], x[..., 1::2]], dim=-1).flatten(-2)  # no rotation at all
    assert not torch.allclose(oa.rotary(x, pos, base), wrong, atol=1e-3)


def test_rotary_keeps_norms_is_the_identity_at_zero_and_keeps_phases_in_float64():
    from conftest import reference_vectors

    g = torch.Generator().manual_seed(4)
    x = torch.randn(1, 5, 2, 16, generator=g, dtype=torch.float64)
    pos = torch.arange(5).expand(1, 5)
    r = oa.rotary(x, pos, 10000.0)
    assert (r.square().sum(-1) - x.square().sum(-1)).abs().max().item() < 1e-12
    assert torch.equal(oa.rotary(x, torch.zeros(1, 5, dtype=torch.long), 10000.0), x)
    # scores depend on position differences only (tests/test_attention.py:106-111)
    q, k = torch.randn(1, 6, 1, 16, generator=g, dtype=torch.float64), torch.randn(1, 6, 1, 16, generator=g,
                                                                                    dtype=torch.float64)
    p0 = torch.arange(6).expand(1, 6)
    s0 = oa.rotary(q, p0, 10000.0)[0, :, 0] @ oa.rotary(k, p0, 10000.0)[0, :, 0].T
    s1 = oa.rotary(q, p0 + 1000, 10000.0)[0, :, 0] @ oa.rotary(k, p0 + 1000, 10000.0)[0, :, 0].T
    assert (s1 - s0).abs().max().item() < 1e-9
    for dtype_name, position, atol in reference_vectors()["rotary"]["precision"]:
        dtype = getattr(torch, dtype_name)
        x = torch.zeros(1, 2, 1, 2, dtype=dtype)
        x[..., 0] = 1.0
        r = oa.rotary(x, torch.tensor([[position, position + 1]]), 10000.0)
        want = torch.tensor([[math.cos(position), math.sin(position)], [math.cos(position + 1), math.sin(position + 1)]],
                            dtype=torch.float64)
        assert r.dtype == dtype and not torch.equal(r[0, 0], r[0, 1])
        assert torch.allclose(r[0, :, 0, :].double(), want, rtol=0, atol=float(atol)), dtype_name


def test_rotary_refusals():
    x = torch.zeros(1, 2, 1, 4)
    with pytest.raises(ValueError, match="int64"):
        oa.rotary(x, torch.zeros(2, 2, dtype=torch.long), 10000.0)
    with pytest.raises(ValueError, match="even"):
        oa.rotary(torch.zeros(1, 2, 1, 3), torch.zeros(1, 2, dtype=torch.long), 10000.0)
    with pytest.raises(ValueError, match="above 1"):
        oa.rotary(x, torch.zeros(1, 2, dtype=torch.long), float("nan"))
