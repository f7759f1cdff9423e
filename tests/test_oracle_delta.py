"""Pins of the CPU delta-rule oracle (``oracle/delta.py``) against what the mathematics fixes.

Every expected value here comes from outside the oracle: the reference's exact two-token
rational answers (``tests/golden/reference_vectors.json``), the serial recurrence on tiny inputs,
the delta rule's defining overwrite, the contraction bound on the state, and planted mistakes that
each of these must catch.
"""

from __future__ import annotations

import pytest
import torch

from conftest import frac_tensor, reference_vectors, scan_inputs
from oracle import delta as od
from oracle.delta import delta_scan_chunked, delta_scan_chunked_backward, normalize_keys

F64 = torch.float64


def _two_token():
    c = reference_vectors()["delta_two_token"]
    q = frac_tensor(c["q"]).reshape(1, 2, 1, 2)
    k = frac_tensor(c["k"]).reshape(1, 2, 1, 2)
    v = frac_tensor(c["v"]).reshape(1, 2, 1, 2)
    beta = frac_tensor(c["beta"]).reshape(1, 2, 1)
    h0 = frac_tensor(c["h0"]).reshape(1, 1, 2, 2)
    h1 = frac_tensor(c["h1"]).reshape(1, 1, 2, 2)
    h2 = frac_tensor(c["h2"]).reshape(1, 1, 2, 2)
    o = frac_tensor(c["o"]).reshape(1, 2, 1, 2)
    return q, k, v, beta, h0, h1, h2, o, c["blocks"]


def test_two_token_rational_answers_step_by_step() -> None:
    q, k, v, beta, h0, h1, h2, o, _ = _two_token()
    first, s1 = od.delta_scan_step(q[:, 0], k[:, 0], v[:, 0], beta[:, 0], h0)
    assert torch.allclose(first, o[:, 0], rtol=0, atol=1e-12)
    assert torch.allclose(s1, h1, rtol=0, atol=1e-12)
    second, s2 = od.delta_scan_step(q[:, 1], k[:, 1], v[:, 1], beta[:, 1], s1)
    assert torch.allclose(second, o[:, 1], rtol=0, atol=1e-12)
    assert torch.allclose(s2, h2, rtol=0, atol=1e-12)


@pytest.mark.parametrize("block", [1, 2, 3, 64])
def test_two_token_rational_answers_blocked(block: int) -> None:
    q, k, v, beta, h0, _, h2, o, blocks = _two_token()
    assert block in blocks
    out, state = od.delta_scan_chunked(q, k, v, beta, h0, block)
    assert torch.allclose(out, o, rtol=0, atol=1e-12)
    assert torch.allclose(state, h2, rtol=0, atol=1e-12)
    out_s, state_s = od.delta_scan_serial(q, k, v, beta, h0)
    assert torch.allclose(out_s, o, rtol=0, atol=1e-12)
    assert torch.allclose(state_s, h2, rtol=0, atol=1e-12)


def test_the_update_equation_written_out_by_hand() -> None:
    # the first token of the rational case, expanded entry by entry with Python floats:
    # H1[i][j] = H0[i][j] - beta k_i sum_l k_l H0[l][j] + beta k_i v_j
    q, k, v, beta, h0, h1, *_ = _two_token()
    kk = [0.6, 0.8]
    vv = [5.0, -2.0]
    hh = [[1.0, 2.0], [3.0, 4.0]]
    b = 0.5
    read = [kk[0] * hh[0][j] + kk[1] * hh[1][j] for j in range(2)]
    want = [[hh[i][j] + b * kk[i] * (vv[j] - read[j]) for j in range(2)] for i in range(2)]
    got = od.delta_update(k[:, 0], v[:, 0], beta[:, 0], h0)
    assert torch.allclose(got[0, 0], torch.tensor(want, dtype=F64), rtol=0, atol=1e-12)
    assert torch.allclose(got, h1, rtol=0, atol=1e-12)


@pytest.mark.parametrize("block", [1, 7, 64])
def test_blocked_equals_serial(block: int) -> None:
    # 130 tokens: two full 64-blocks and a partial one (tests/test_recurrence.py:30-37)
    q, k, v, beta, h0 = (t.double() for t in scan_inputs(2, 130, 3, 16, state_scale=0.1))
    o_ref, h_ref = od.delta_scan_serial(q, k, v, beta, h0)
    o, h_n = od.delta_scan_chunked(q, k, v, beta, h0, block)
    assert (o - o_ref).abs().max().item() < 1e-10
    assert (h_n - h_ref).abs().max().item() < 1e-10


def test_blocked_equals_serial_in_float32() -> None:
    q, k, v, beta, h0 = scan_inputs(2, 130, 3, 16, state_scale=0.1)
    o_ref, h_ref = od.delta_scan_serial(q, k, v, beta, h0)
    o, h_n = od.delta_scan_chunked(q, k, v, beta, h0, 64)
    assert (o - o_ref).abs().max().item() < 1e-4
    assert (h_n - h_ref).abs().max().item() < 1e-4


def test_beta_one_overwrites_exactly() -> None:
    # the delta rule's defining property: reading k right after writing (k, v) at beta 1 gives v
    g = torch.Generator().manual_seed(1)
    state = torch.randn(1, 2, 8, 8, generator=g, dtype=F64)
    k = od.normalize_keys(torch.randn(1, 2, 8, generator=g, dtype=F64))
    v = torch.randn(1, 2, 8, generator=g, dtype=F64)
    o, _ = od.delta_scan_step(k, k, v, torch.ones(1, 2, dtype=F64), state)
    assert (o - v).abs().max().item() < 1e-12


def test_zero_beta_leaves_the_state_and_reads_it() -> None:
    q, k, v, _, h0 = (t.double() for t in scan_inputs(1, 5, 2, 4))
    beta = torch.zeros(1, 5, 2, dtype=F64)
    o, h_n = od.delta_scan_chunked(q, k, v, beta, h0, 4)
    assert torch.equal(h_n, h0)
    assert torch.allclose(o, torch.einsum("bhij,bnhi->bnhj", h0, q), rtol=0, atol=1e-12)


def test_state_norm_is_bounded_by_the_writes() -> None:
    # ||(I - b k k^T) H|| <= ||H|| for unit k and b in [0, 1] (tests/test_recurrence.py:86-92)
    q, k, v, beta, h0 = scan_inputs(1, 2000, 2, 16, state_scale=0.1)
    _, h_n = od.delta_scan_chunked(q, k, v, beta, h0, 64)
    bound = h0.flatten(1).norm(dim=1) + (beta * v.norm(dim=-1)).sum(dim=(1, 2))
    assert torch.isfinite(h_n).all()
    assert (h_n.flatten(1).norm(dim=1) <= bound + 1e-3).all()


def test_linear_in_values_and_state_jointly() -> None:
    q, k, v, beta, h0 = (t.double() for t in scan_inputs(1, 70, 2, 8))
    o1, s1 = od.delta_scan_chunked(q, k, v, beta, h0, 64)
    o2, s2 = od.delta_scan_chunked(q, k, -2.5 * v, beta, -2.5 * h0, 64)
    assert torch.allclose(o2, -2.5 * o1, rtol=1e-12, atol=1e-12)
    assert torch.allclose(s2, -2.5 * s1, rtol=1e-12, atol=1e-12)


def test_a_carried_state_continues_the_sequence() -> None:
    q, k, v, beta, h0 = (t.double() for t in scan_inputs(2, 130, 3, 16))
    o, s = od.delta_scan_chunked(q, k, v, beta, h0, 64)
    oa, sa = od.delta_scan_chunked(q[:, :50], k[:, :50], v[:, :50], beta[:, :50], h0, 64)
    ob, sb = od.delta_scan_chunked(q[:, 50:], k[:, 50:], v[:, 50:], beta[:, 50:], sa, 64)
    assert torch.allclose(torch.cat([oa, ob], 1), o, rtol=0, atol=1e-10)
    assert torch.allclose(sb, s, rtol=0, atol=1e-10)


def test_active_mask_zeroes_outputs_but_keeps_every_write() -> None:
    q, k, v, beta, h0 = (t.double() for t in scan_inputs(2, 40, 2, 8))
    active = torch.rand(2, 40, generator=torch.Generator().manual_seed(3)) < 0.6
    o_all, s_all = od.delta_scan_chunked(q, k, v, beta, h0, 16)
    o, s = od.delta_scan_chunked(q, k, v, beta, h0, 16, active=active)
    assert torch.equal(s, s_all)
    assert torch.equal(o[active], o_all[active])
    assert bool((o[~active] == 0).all())


def test_no_tokens_return_the_same_objects() -> None:
    q = torch.empty(2, 0, 3, 4, dtype=F64)
    beta = torch.empty(2, 0, 3, dtype=F64)
    state = torch.ones(2, 3, 4, 4, dtype=F64)
    o, s = od.delta_scan_chunked(q, q, q, beta, state, 64)
    assert o is q and s is state
    with pytest.raises(ValueError, match="block must be at least 1"):
        od.delta_scan_chunked(q, q, q, beta, state, 0)


def test_shape_mismatches_are_refused() -> None:
    q, k, v, beta, h0 = scan_inputs(1, 4, 2, 4)
    with pytest.raises(ValueError, match="state"):
        od.delta_scan_chunked(q, k, v, beta, h0[:, :1], 2)
    with pytest.raises(ValueError, match="beta"):
        od.delta_scan_chunked(q, k, v, beta[:, :3], h0, 2)


def test_normalize_keys_known_answers() -> None:
    c = reference_vectors()["normalize_keys"]
    for case in ("small_floor", "large", "zero"):
        k = frac_tensor(c[case]["k"])
        want = frac_tensor(c[case]["want"])
        assert torch.allclose(od.normalize_keys(k), want, rtol=1e-12, atol=0), case
    wide = torch.ones(1, c["wide_ones_fp16"]["n"], dtype=torch.float16)
    assert torch.equal(od.normalize_keys(wide), torch.full_like(wide, 1 / 256))
    for dtype_name, magnitude in c["magnitudes_by_dtype"]["rows"]:
        dtype = getattr(torch, dtype_name)
        k = torch.tensor([[float(magnitude), 0.0]], dtype=dtype)
        assert torch.equal(od.normalize_keys(k), torch.tensor([[1.0, 0.0]], dtype=dtype)), dtype_name


def test_write_strength_known_answers() -> None:
    c = reference_vectors()["write_strength"]
    got = od.write_strength(frac_tensor(c["logits"], torch.float32))
    assert torch.equal(got, frac_tensor(c["want"], torch.float32))
    o = c["odds_case"]
    beta = float(frac_tensor([o["beta"]])[0])
    logits = torch.full((1, 1, 1), float(torch.logit(torch.tensor(beta, dtype=F64))), dtype=F64)
    m = torch.full((1, 1), float(frac_tensor([o["m"]])[0]), dtype=F64)
    got = od.write_strength(logits, m, float(frac_tensor([o["alpha"]])[0]))
    assert abs(float(got) - float(frac_tensor([o["want"]])[0])) < 1e-12


# --- planted mistakes: each pin above must catch a plausible slip in the oracle ----------------


def _planted(kind: str):
    def step(q, k, v, beta, state):
        if kind == "reversed_erase":  # H (I - b k k^T) + b k v^T
            eye = torch.eye(k.shape[-1], dtype=state.dtype)
            erase = eye - beta[..., None, None] * k[..., :, None] * k[..., None, :]
            new = state @ erase + beta[..., None, None] * k[..., :, None] * v[..., None, :]
        elif kind == "beta_squared":
            new = od.delta_update(k, v, beta * beta, state)
        elif kind == "read_before_write":
            new = od.delta_update(k, v, beta, state)
            return torch.einsum("bhij,bhi->bhj", state, q), new
        else:
            raise AssertionError(kind)
        return torch.einsum("bhij,bhi->bhj", new, q), new

    return step


@pytest.mark.parametrize("kind", ["reversed_erase", "beta_squared", "read_before_write"])
def test_the_rational_case_catches_planted_mistakes(kind: str) -> None:
    q, k, v, beta, h0, _, h2, o, _ = _two_token()
    step = _planted(kind)
    s = h0
    outs = []
    for t in range(2):
        ot, s = step(q[:, t], k[:, t], v[:, t], beta[:, t], s)
        outs.append(ot)
    got = torch.stack(outs, 1)
    assert (got - o).abs().max().item() > 1e-3 or (s - h2).abs().max().item() > 1e-3


@pytest.mark.parametrize(("b", "n", "h", "dk", "block"), [(2, 1, 2, 4, 64), (2, 63, 3, 8, 64), (1, 130, 2, 8, 64),
                                                          (2, 70, 2, 4, 16)])
def test_the_chunked_backward_equals_autograd(b, n, h, dk, block):
    # the WY-form backward (what the scan's backward kernels compute) against autograd through the
    # chunked forward: partial blocks, a zero write strength, inactive tokens, a state gradient
    g = torch.Generator().manual_seed(b * 100 + n)
    q = torch.randn(b, n, h, dk, generator=g, dtype=torch.float64)
    k = normalize_keys(torch.randn(b, n, h, dk, generator=g, dtype=torch.float64))
    v = torch.randn(b, n, h, dk, generator=g, dtype=torch.float64)
    beta = torch.sigmoid(torch.randn(b, n, h, generator=g, dtype=torch.float64))
    beta[0, 0, 0] = 0.0
    h0 = 0.3 * torch.randn(b, h, dk, dk, generator=g, dtype=torch.float64)
    d_o = torch.randn(b, n, h, dk, generator=g, dtype=torch.float64)
    d_s = torch.randn(b, h, dk, dk, generator=g, dtype=torch.float64)
    active = torch.rand(b, n, generator=g) < 0.7
    ins = [t.clone().requires_grad_() for t in (q, k, v, beta, h0)]
    o, s = delta_scan_chunked(*ins, block, active=active)
    ((o * d_o).sum() + (s * d_s).sum()).backward()
    got = delta_scan_chunked_backward(q, k, v, beta, h0, d_o, d_s, block, active=active)
    for a, t, name in zip(got, ins, ("q", "k", "v", "beta", "state")):
        torch.testing.assert_close(a, t.grad, rtol=1e-11, atol=1e-12, msg=name)


def test_the_chunked_scan_gradients_match_finite_differences():
    g = torch.Generator().manual_seed(77)
    b, n, h, dk = 1, 7, 1, 3
    q = torch.randn(b, n, h, dk, generator=g, dtype=torch.float64, requires_grad=True)
    k = normalize_keys(torch.randn(b, n, h, dk, generator=g, dtype=torch.float64)).requires_grad_()
    v = torch.randn(b, n, h, dk, generator=g, dtype=torch.float64, requires_grad=True)
    beta = torch.sigmoid(torch.randn(b, n, h, generator=g, dtype=torch.float64)).requires_grad_()
    h0 = torch.randn(b, h, dk, dk, generator=g, dtype=torch.float64, requires_grad=True)
    assert torch.autograd.gradcheck(lambda *a: delta_scan_chunked(*a, 3), (q, k, v, beta, h0))


def test_a_planted_transpose_in_the_backward_is_caught(monkeypatch):
    import oracle.delta as od

    g = torch.Generator().manual_seed(78)
    args = [torch.randn(1, 9, 1, 4, generator=g, dtype=torch.float64) for _ in range(3)]
    args[1] = normalize_keys(args[1])
    beta = torch.sigmoid(torch.randn(1, 9, 1, generator=g, dtype=torch.float64))
    h0 = torch.randn(1, 1, 4, 4, generator=g, dtype=torch.float64)
    d_o = torch.randn(1, 9, 1, 4, generator=g, dtype=torch.float64)
    right = od.delta_scan_chunked_backward(*args, beta, h0, d_o, None, 4)
    real = torch.linalg.solve_triangular
    monkeypatch.setattr(torch.linalg, "solve_triangular", lambda a, b_, **kw: real(a, b_, **kw).transpose(-1, -2))
    wrong = od.delta_scan_chunked_backward(*args, beta, h0, d_o, None, 4)
    assert not torch.allclose(right[1], wrong[1], rtol=1e-3)


def test_write_strength_is_the_scaled_odds_closed_form() -> None:
    # sigmoid(l + ln(1 + a m)) = s (1 + a m) / (1 + s a m) with s = sigmoid(l): the write odds
    # s / (1 - s) multiplied by 1 + a m; 1 + a m = 0 gives an exact zero, m = 0 the plain sigmoid
    g = torch.Generator().manual_seed(11)
    logits = torch.randn(3, 5, 4, generator=g, dtype=F64) * 3
    m = torch.rand(3, 5, generator=g, dtype=F64) * 4
    alpha = 0.75
    s = torch.sigmoid(logits)
    am = (alpha * m)[..., None]
    want = s * (1 + am) / (1 + s * am)
    assert (od.write_strength(logits, m, alpha) - want).abs().max().item() < 1e-14
    assert torch.equal(od.write_strength(logits, torch.zeros(3, 5, dtype=F64), alpha), s)
    edge = torch.full((3, 5), -1.0 / alpha, dtype=F64)
    assert not bool(od.write_strength(logits, edge, alpha).any())
    more = od.write_strength(logits, m + 0.5, alpha)
    assert bool((more > od.write_strength(logits, m, alpha)).all())
    # a planted mistake: the factor added to the probability instead of scaling the odds
    wrong = torch.sigmoid(logits) * (1 + am)
    assert not torch.allclose(wrong, want, atol=1e-3)
