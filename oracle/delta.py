"""CPU oracle of the delta-rule scan (test infrastructure only; see ``oracle/__init__.py``).

Per head the state ``H`` is ``[dk, dk]`` (key rows, value columns) and is read as ``H^T q``. One
token applies

    H' = (I - beta k k^T) H + beta k v^T,        o = H'^T q

(reference ``vesper/recurrence.py:1-23``). Layouts follow the reference: ``q, k, v [b, n, h, dk]``,
``beta [b, n, h]``, ``state [b, h, dk, dk]``.

The blocked form uses the WY/UT representation of the erase factors of a block of ``C`` tokens
(rows of ``K, V``): ``A = tril(diag(beta) K K^T, -1)``, ``T = (I + A)^-1 diag(beta)``,
``W = T K``, ``U = T V``, ``D = U - W H``, ``O = Q H + tril(Q K^T) D``, ``H <- H + K^T D``
(``recurrence.py:17-23``, ``:202-216``). Here ``T`` comes from a unit-lower-triangular solve
rather than an explicit inverse; the two are the same matrix.
"""

from __future__ import annotations

import torch
from torch import Tensor

KEY_NORM_FLOOR = 1e-6  # recurrence.py:31


def normalize_keys(k: Tensor) -> Tensor:
    """``k / max(||k||, 1e-6)`` computed without squaring out of range (``recurrence.py:91-115``).

    The row is first divided by its largest magnitude (floored at 1e-6, and a constant for the
    gradient), so one component of the scaled row has magnitude one unless the whole row sits under
    the floor; the squared norm is accumulated in float32 (float64 for float64 rows) and floored at
    one before the root.
    """
    if k.numel() == 0:
        return k
    # the peak is held constant under autograd (recurrence.py:103-105): it cancels algebraically
    peak = k.detach().abs().amax(dim=-1, keepdim=True).clamp_min(KEY_NORM_FLOOR)
    unit = k / peak
    wide = torch.float64 if unit.dtype == torch.float64 else torch.float32
    norm2 = (unit.to(wide) ** 2).sum(dim=-1, keepdim=True)
    return unit / norm2.clamp_min(1.0).sqrt().to(unit.dtype)


def write_strength(logits: Tensor, m: Tensor | None = None, alpha: float | None = None) -> Tensor:
    """``beta = sigmoid(logits)``; with a modulator, the write odds scaled by ``1 + alpha m``.

    ``recurrence.py:34-88``: ``sigmoid(logits + ln(1 + alpha m))`` with an exact zero where the
    factor is zero; a negative factor, a missing or negative ``alpha`` is refused.
    """
    if m is None:
        return torch.sigmoid(logits)
    if alpha is None or not 0.0 <= alpha < float("inf"):
        raise ValueError(f"alpha must be finite and non-negative with a modulator, got {alpha}")
    factor = 1.0 + alpha * m
    if bool((factor < 0).any()):
        raise ValueError("1 + alpha m must not be negative")
    tiny = torch.finfo(factor.dtype).tiny
    beta = torch.sigmoid(logits + torch.log(factor.clamp_min(tiny))[..., None])
    return torch.where((factor > 0)[..., None], beta, torch.zeros_like(beta))


def _check(q: Tensor, k: Tensor, v: Tensor, beta: Tensor, state: Tensor, tokens: bool) -> None:
    lead = 4 if tokens else 3
    if q.dim() != lead or k.shape != q.shape or v.shape != q.shape:
        raise ValueError(f"q, k, v must share one rank-{lead} shape: {q.shape} {k.shape} {v.shape}")
    if beta.shape != q.shape[:-1]:
        raise ValueError(f"beta must be {tuple(q.shape[:-1])}, got {tuple(beta.shape)}")
    b, h, dk = q.shape[0], q.shape[-2], q.shape[-1]
    if state.shape != (b, h, dk, dk):
        raise ValueError(f"state must be {(b, h, dk, dk)}, got {tuple(state.shape)}")


def delta_update(k: Tensor, v: Tensor, beta: Tensor, state: Tensor) -> Tensor:
    """The write alone, ``(I - beta k k^T) H + beta k v^T`` (``recurrence.py:118-140``).

    ``k, v [b, h, dk]``, ``beta [b, h]``, ``state [b, h, dk, dk]``; returns a new state.
    """
    _check(k, k, v, beta, state, tokens=False)
    stored = torch.einsum("bhij,bhi->bhj", state, k)  # H^T k: what the key reads now
    return state + beta[..., None, None] * k[..., :, None] * (v - stored)[..., None, :]


def delta_scan_step(q: Tensor, k: Tensor, v: Tensor, beta: Tensor, state: Tensor) -> tuple[Tensor, Tensor]:
    """One token written then read: ``(H'^T q, H')`` (``recurrence.py:143-163``)."""
    _check(q, k, v, beta, state, tokens=False)
    new = delta_update(k, v, beta, state)
    return torch.einsum("bhij,bhi->bhj", new, q), new


def delta_scan_serial(
    q: Tensor, k: Tensor, v: Tensor, beta: Tensor, state: Tensor, active: Tensor | None = None
) -> tuple[Tensor, Tensor]:
    """``n`` single steps in order: the textbook recurrence, the brute-force truth.

    With ``active`` (bool ``[b, n]``) the outputs of inactive tokens are zero while every token
    still writes the state (``loop.py:24-26``, ``:441-442``).
    """
    _check(q, k, v, beta, state, tokens=True)
    outs = []
    h_state = state
    for t in range(q.shape[1]):
        o, h_state = delta_scan_step(q[:, t], k[:, t], v[:, t], beta[:, t], h_state)
        outs.append(o)
    if not outs:
        return q, state
    o = torch.stack(outs, dim=1)
    if active is not None:
        o = torch.where(active[:, :, None, None], o, torch.zeros_like(o))
    return o, h_state


def delta_scan_chunked(
    q: Tensor,
    k: Tensor,
    v: Tensor,
    beta: Tensor,
    state: Tensor,
    block: int = 64,
    active: Tensor | None = None,
) -> tuple[Tensor, Tensor]:
    """The blocked WY/UT scan (``recurrence.py:166-217``); equals ``delta_scan_serial``.

    ``n = 0`` returns ``(q, state)`` themselves after validation (``recurrence.py:198-199``).
    ``active`` zeroes inactive outputs only, as in ``delta_scan_serial``.

    Raises:
        ValueError: on mismatched shapes or ``block < 1``.
    """
    _check(q, k, v, beta, state, tokens=True)
    if block < 1:
        raise ValueError(f"block must be at least 1, got {block}")
    n = q.shape[1]
    if n == 0:
        return q, state
    h_state = state
    pieces = []
    for s in range(0, n, block):
        e = min(s + block, n)
        qb, kb, vb = (x[:, s:e].transpose(1, 2) for x in (q, k, v))  # [b, h, C, dk]
        bb = beta[:, s:e].transpose(1, 2)  # [b, h, C]
        c = e - s
        eye = torch.eye(c, dtype=q.dtype)
        gram = kb @ kb.transpose(-1, -2)
        lower = torch.tril(bb[..., :, None] * gram, diagonal=-1)
        # T = (I + A)^-1 diag(beta): one unit-lower-triangular solve against diag(beta)
        t_mat = torch.linalg.solve_triangular(
            eye + lower, torch.diag_embed(bb), upper=False, unitriangular=True
        )
        w_rows = t_mat @ kb
        u_rows = t_mat @ vb
        delta = u_rows - w_rows @ h_state
        reads = qb @ h_state + torch.tril(qb @ kb.transpose(-1, -2)) @ delta
        pieces.append(reads.transpose(1, 2))
        h_state = h_state + kb.transpose(-1, -2) @ delta
    o = torch.cat(pieces, dim=1)
    if active is not None:
        o = torch.where(active[:, :, None, None], o, torch.zeros_like(o))
    return o, h_state


def relative_error(got: Tensor, want: Tensor) -> float:
    """Relative Frobenius error in float64 (``tests/test_delta_scan_fused.py:41-44``)."""
    a, b = got.detach().double().cpu(), want.detach().double().cpu()
    den = float(b.square().sum().sqrt())
    num = float((a - b).square().sum().sqrt())
    return num / den if den > 0 else num


def delta_scan_chunked_backward(
    q: Tensor,
    k: Tensor,
    v: Tensor,
    beta: Tensor,
    state: Tensor,
    d_o: Tensor,
    d_state: Tensor | None = None,
    block: int = 64,
    active: Tensor | None = None,
) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
    """``(dq, dk, dv, dbeta, dstate)`` of ``sum(o * d_o) + sum(state_n * d_state)`` for
    ``delta_scan_chunked``, written out per block in the WY form (the algebra the scan's backward
    kernels follow; checked against autograd through ``delta_scan_chunked``).

    Per block, with ``H`` the state at its start, ``G`` the gradient of the state at its end,
    ``L = (I + A)^-1``, ``T = L diag(beta)``, ``R = V - K H``, ``Delta = T R``, ``P = tril(Q K^T)``:
    ``dDelta = K G + P^T dO``, ``dR = T^T dDelta`` (= ``dV``), ``dQ = dO H^T + tril(dO Delta^T) K``,
    ``dT = dDelta R^T``, ``dA = tril(-L^T (dT diag(beta)) L^T, -1)``,
    ``dK = Delta G^T + tril(dO Delta^T)^T Q - dR H^T + (diag(beta) dA + dA^T diag(beta)) K``,
    ``dbeta_j = sum_i dT_ij L_ij + sum_m dA_jm (k_j . k_m)``, and the state's gradient at the block's
    start ``G + Q^T dO - K^T dR``. An inactive token's output gradient is zero (its output is).
    """
    _check(q, k, v, beta, state, tokens=True)
    b, n, h, d = q.shape
    if active is not None:
        d_o = torch.where(active[:, :, None, None], d_o, torch.zeros_like(d_o))
    # the states at the block starts
    starts, h_state = [], state
    for s in range(0, n, block):
        e = min(s + block, n)
        kb, vb = (x[:, s:e].transpose(1, 2) for x in (k, v))
        bb = beta[:, s:e].transpose(1, 2)
        c = e - s
        lower = torch.tril(bb[..., :, None] * (kb @ kb.transpose(-1, -2)), diagonal=-1)
        inv = torch.linalg.solve_triangular(torch.eye(c, dtype=q.dtype) + lower,
                                            torch.eye(c, dtype=q.dtype).expand_as(lower), upper=False,
                                            unitriangular=True)
        starts.append(h_state)
        h_state = h_state + kb.transpose(-1, -2) @ (inv @ (bb[..., None] * (vb - kb @ h_state)))
    dq, dk, dv = torch.zeros_like(q), torch.zeros_like(k), torch.zeros_like(v)
    dbeta = torch.zeros_like(beta)
    grad = torch.zeros_like(state) if d_state is None else d_state.clone()
    for idx, s in reversed(list(enumerate(range(0, n, block)))):
        e = min(s + block, n)
        qb, kb, vb, gob = (x[:, s:e].transpose(1, 2) for x in (q, k, v, d_o))
        bb = beta[:, s:e].transpose(1, 2)
        c = e - s
        hs = starts[idx]
        gram = kb @ kb.transpose(-1, -2)
        lower = torch.tril(bb[..., :, None] * gram, diagonal=-1)
        inv = torch.linalg.solve_triangular(torch.eye(c, dtype=q.dtype) + lower,
                                            torch.eye(c, dtype=q.dtype).expand_as(lower), upper=False,
                                            unitriangular=True)
        t_mat = inv * bb[..., None, :]
        r = vb - kb @ hs
        delta = t_mat @ r
        p = torch.tril(qb @ kb.transpose(-1, -2))
        d_delta = kb @ grad + p.transpose(-1, -2) @ gob
        d_r = t_mat.transpose(-1, -2) @ d_delta
        s2 = torch.tril(gob @ delta.transpose(-1, -2))
        d_q = gob @ hs.transpose(-1, -2) + s2 @ kb
        d_t = d_delta @ r.transpose(-1, -2)
        d_l = torch.tril(d_t * bb[..., None, :])
        d_a = -torch.tril(inv.transpose(-1, -2) @ d_l @ inv.transpose(-1, -2), diagonal=-1)
        m = bb[..., :, None] * d_a
        d_k = (delta @ grad.transpose(-1, -2) + s2.transpose(-1, -2) @ qb - d_r @ hs.transpose(-1, -2)
               + m @ kb + m.transpose(-1, -2) @ kb)
        d_b = (d_t * inv).sum(dim=-2) + (d_a * gram).sum(dim=-1)
        dq[:, s:e], dk[:, s:e], dv[:, s:e] = (x.transpose(1, 2) for x in (d_q, d_k, d_r))
        dbeta[:, s:e] = d_b.transpose(1, 2)
        grad = grad + qb.transpose(-1, -2) @ gob - kb.transpose(-1, -2) @ d_r
    return dq, dk, dv, dbeta, grad
