"""Pins of the key-filter oracle (``oracle/keys.py``) against what the operator's definition fixes.

Expected values come from outside the vectorized oracle: answers worked by hand (one-feature heads,
whose normalized key is the sign of the filtered input, and a 3-4-5 row), the operator applied one
position and tap at a time, and the properties the reference's own tests state
(``tests/test_key_conv.py:72-128``): an asymmetric filter tells a reversed one apart, the history
carries exactly the newest inputs, streaming equals one pass, no filter is the plain normalization.
"""

from __future__ import annotations

import torch

from oracle import keys as ok
from oracle.delta import normalize_keys

F64 = torch.float64
K = 4


def _taps(d: int) -> torch.Tensor:
    # every tap and channel differ (the reference's asymmetric pattern, tests/test_key_conv.py:51-55)
    r = torch.arange(K, dtype=F64)[:, None]
    j = torch.arange(d, dtype=F64)[None, :]
    return (r + 1) * 0.5 - 0.3 * j + 0.1 * r * j


def test_one_feature_heads_give_the_sign_of_the_hand_filtered_input():
    # d = 2 features, 2 heads of width one: a normalized one-element key is the sign of u
    taps = torch.tensor([[1.0, 1.0], [-2.0, 0.5], [0.0, -4.0], [1.0, 0.0]], dtype=F64)
    history = torch.tensor([[[1.0, 0.0], [0.0, 2.0], [3.0, 0.0]]], dtype=F64)  # rows t = -3, -2, -1
    z = torch.tensor([[[1.0, -1.0], [2.0, 1.0]]], dtype=F64)  # t = 0, 1
    # t = 0: u0 = 1*1 + (-2)*3 + 0*0 + 1*1 = -4;  u1 = 1*(-1) + 0.5*0 + (-4)*2 + 0*0 = -9
    # t = 1: u0 = 1*2 + (-2)*1 + 0*3 + 1*0 = 0;   u1 = 1*1 + 0.5*(-1) + (-4)*0 + 0*2 = 0.5
    keys, after = ok.filter_keys(z, history, taps, heads=2)
    assert keys.shape == (1, 2, 2, 1)
    assert keys.flatten().tolist() == [-1.0, -1.0, 0.0, 1.0]
    assert torch.equal(after, torch.cat([history[:, 2:], z], dim=1))


def test_a_three_four_five_row():
    taps = torch.tensor([[1.0, 1.0], [0.0, 0.0]], dtype=F64)  # K = 2: the current token only
    z = torch.tensor([[[3.0, 4.0], [0.0, 0.0]]], dtype=F64)
    keys, _ = ok.filter_keys(z, torch.zeros(1, 1, 2, dtype=F64), taps, heads=1)
    assert torch.allclose(keys[0, 0, 0], torch.tensor([0.6, 0.8], dtype=F64), rtol=0, atol=1e-15)
    assert torch.equal(keys[0, 1, 0], torch.zeros(2, dtype=F64))  # a zero row stays zero (the floor)


def test_the_vectorized_filter_equals_the_literal_operator_and_a_reversed_one_differs():
    g = torch.Generator().manual_seed(1)
    z = torch.randn(2, 6, 8, generator=g, dtype=F64)
    history = torch.randn(2, K - 1, 8, generator=g, dtype=F64)
    keys, after = ok.filter_keys(z, history, _taps(8), heads=2)
    want, want_after = ok.filter_keys_literal(z, history, _taps(8), heads=2)
    assert torch.allclose(keys, want, rtol=0, atol=1e-12)
    assert torch.equal(after, want_after)
    reversed_keys, _ = ok.filter_keys_literal(z, history, _taps(8).flip(0), heads=2)
    assert not torch.allclose(keys, reversed_keys, rtol=0, atol=1e-6)


def test_a_planted_shift_is_caught_by_the_hand_case():
    taps = torch.tensor([[1.0, 1.0], [-2.0, 0.5], [0.0, -4.0], [1.0, 0.0]], dtype=F64)
    history = torch.tensor([[[1.0, 0.0], [0.0, 2.0], [3.0, 0.0]]], dtype=F64)
    z = torch.tensor([[[1.0, -1.0], [2.0, 1.0]]], dtype=F64)
    # the filter one position late (taps[r] on z[t - r - 1]): what an off-by-one kernel would do
    full = torch.cat([history, z], dim=1)
    shifted = torch.zeros(1, 2, 2, dtype=F64)
    for t in range(2):
        for r in range(K):
            shifted[:, t] += taps[r] * full[:, K - 2 + t - r] if K - 2 + t - r >= 0 else 0.0
    bad = normalize_keys(shifted.view(1, 2, 2, 1))
    good, _ = ok.filter_keys(z, history, taps, heads=2)
    assert not torch.equal(bad, good)


def test_the_history_carries_exactly_the_newest_inputs():
    g = torch.Generator().manual_seed(2)
    history = torch.randn(1, K - 1, 8, generator=g, dtype=F64)
    empty = torch.zeros(1, 0, 8, dtype=F64)
    keys, after = ok.filter_keys(empty, history, _taps(8), heads=2)
    assert keys.shape == (1, 0, 2, 4) and after is history
    for n in (1, 2):
        z = torch.randn(1, n, 8, generator=g, dtype=F64)
        _, after = ok.filter_keys(z, history, _taps(8), heads=2)
        assert torch.equal(after, torch.cat([history[:, n:], z], dim=1))
    z = torch.randn(1, 50, 8, generator=g, dtype=F64)
    _, after = ok.filter_keys(z, history, _taps(8), heads=2)
    assert torch.equal(after, z[:, -(K - 1):])


def test_streaming_equals_one_pass_over_the_whole_sequence():
    g = torch.Generator().manual_seed(3)
    z = torch.randn(1, 11, 8, generator=g, dtype=F64)
    cold = torch.zeros(1, K - 1, 8, dtype=F64)
    whole, _ = ok.filter_keys(z, cold, _taps(8), heads=2)
    for sizes in ((1,) * 11, (2, 0, 3, 1, 5), (11,), (0, 4, 7)):
        history, start, parts = cold, 0, []
        for size in sizes:
            keys, history = ok.filter_keys(z[:, start:start + size], history, _taps(8), heads=2)
            parts.append(keys)
            start += size
        assert torch.allclose(torch.cat(parts, dim=1), whole, rtol=0, atol=1e-12), sizes


def test_no_filter_is_the_plain_normalization():
    g = torch.Generator().manual_seed(4)
    z = torch.randn(2, 5, 8, generator=g, dtype=F64)
    none = torch.zeros(2, 0, 8, dtype=F64)
    keys, after = ok.filter_keys(z, none, None, heads=2)
    assert torch.equal(keys, normalize_keys(z.view(2, 5, 2, 4)))
    assert after is none


def test_low_precision_inputs_filter_in_float32_and_return_their_dtype():
    g = torch.Generator().manual_seed(5)
    z = torch.randn(1, 7, 8, generator=g).to(torch.bfloat16)
    history = torch.randn(1, K - 1, 8, generator=g)
    keys, after = ok.filter_keys(z, history, _taps(8).float(), heads=2)
    assert keys.dtype == torch.bfloat16 and after.dtype == torch.float32
    wide, _ = ok.filter_keys_literal(z.double(), history.double(), _taps(8), heads=2)
    assert torch.allclose(keys.double(), wide, rtol=0, atol=8e-3)


def test_the_gradients_match_finite_differences():
    g = torch.Generator().manual_seed(21)
    z = torch.randn(2, 5, 8, generator=g, dtype=torch.float64)
    hist = torch.randn(2, 2, 8, generator=g, dtype=torch.float64)
    taps = torch.randn(3, 8, generator=g, dtype=torch.float64)
    up = torch.randn(2, 5, 2, 4, generator=g, dtype=torch.float64)

    def loss(zz, hh, tt):
        keys, _ = ok.filter_keys(zz, hh, tt, 2)
        return (keys * up).sum()

    assert torch.autograd.gradcheck(loss, (z.requires_grad_(), hist.requires_grad_(), taps.requires_grad_()))
    dz, dh, dt = ok.filter_keys_grads(z, hist, taps, 2, up)
    lz, lh, lt = ok.filter_keys_grads_literal(z.detach(), hist.detach(), taps.detach(), 2, up)
    for a, b in ((dz, lz), (dh, lh), (dt, lt)):
        torch.testing.assert_close(a, b, rtol=1e-10, atol=1e-12)


def test_the_gradients_below_the_unit_norm_and_under_the_floor():
    # a head whose scaled norm is exactly one (one nonzero component) and a row under the floor
    z = torch.zeros(1, 3, 4, dtype=torch.float64)
    z[0, 0, 1] = 2.0
    z[0, 2] = 1e-8
    hist = torch.zeros(1, 1, 4, dtype=torch.float64)
    taps = torch.ones(2, 4, dtype=torch.float64)
    up = torch.arange(12, dtype=torch.float64).view(1, 3, 1, 4) - 5.0
    dz, dh, dt = ok.filter_keys_grads(z, hist, taps, 1, up)
    lz, lh, lt = ok.filter_keys_grads_literal(z, hist, taps, 1, up)
    for a, b in ((dz, lz), (dh, lh), (dt, lt)):
        torch.testing.assert_close(a, b, rtol=1e-12, atol=1e-12)
    # under the floor the key is u / 1e-6 (norm below one): its gradient is up / 1e-6 through the filter
    want_row2 = up[0, 2, 0] / 1e-6
    torch.testing.assert_close(dz[0, 2], want_row2, rtol=1e-12, atol=0)  # dz[2] = taps[0] du[2]


def test_a_planted_mistake_in_the_literal_gradients_is_caught():
    g = torch.Generator().manual_seed(22)
    z = torch.randn(1, 4, 8, generator=g, dtype=torch.float64)
    hist = torch.randn(1, 2, 8, generator=g, dtype=torch.float64)
    taps = torch.randn(3, 8, generator=g, dtype=torch.float64)
    up = torch.randn(1, 4, 2, 4, generator=g, dtype=torch.float64)
    dz, _, dt = ok.filter_keys_grads(z, hist, taps, 2, up)
    # the taps' gradient with the input shifted by one token (a plausible indexing slip)
    full = torch.cat([hist, z], dim=1)
    _, _, lt = ok.filter_keys_grads_literal(z, hist, taps, 2, up)
    assert torch.allclose(dt, lt)
    shifted = torch.cat([hist[:, :1], full[:, :-1]], dim=1)
    _, _, wrong = ok.filter_keys_grads_literal(shifted[:, 2:], shifted[:, :2], taps, 2, up)
    assert not torch.allclose(dt, wrong, rtol=1e-3, atol=1e-6)
