"""CPU oracle of sliding-window causal attention (test infrastructure only; see ``oracle/__init__.py``).

Semantics restated from the reference:

- ``window_attention`` (``vesper/kernels/window_attn.py:27-39``): ``q [b, n, h, dk]`` against
  ``keys, values [b, m + n, hkv, dk]`` whose first ``m`` rows are the cache; query ``i`` sits at
  key index ``m + i`` and attends key indices ``[m + i - w + 1, m + i]``; scale ``1/sqrt(dk)``;
  query head ``j`` reads KV head ``j // (h / hkv)`` (``enable_gqa``, pinned by
  ``tests/test_attention_independent.py:82-99``).
- ``attend_positions`` (``vesper/attention.py:384-407``): the same window over absolute positions,
  computed in query blocks of ``w`` against at most ``3w`` keys, mask ``p_i - w < p_j <= p_i``.
- ``attention_full_mask``: one unblocked masked softmax (``tests/test_attention.py:44-55``).
- ``ring_attend`` / ``kv_ring_write`` (``vesper/attention.py:62-139``, ``:298-338``): one decoding
  token per row over a ring whose visibility is ``valid`` and the position mask, never slot
  order; the new key is attended once from its argument and then written to slot ``p % w``.
- ``kv_cache_push`` (``vesper/attention.py:142-175``): keep the newest ``min(m + n, w)`` entries.
- ``rotary`` (``vesper/attention.py:178-217``): pairs ``(x[2j], x[2j+1])`` rotated by
  ``pos * base^(-2j/dk)``, the phases in float64, ``cos`` and ``sin`` cast to ``x``'s dtype and the
  rotation computed in that dtype.

An optional ``active`` (bool ``[b, n]``) zeroes the outputs of inactive queries; their keys and
values stay visible to every other query (``vesper/loop.py:24-26``, ``:441-442``).
"""

from __future__ import annotations

import math

import torch
from torch import Tensor


def _expand_kv(x: Tensor, heads: int) -> Tensor:
    """``[b, s, hkv, dk] -> [b, s, h, dk]``: query head j reads KV head ``j // (h / hkv)``."""
    hkv = x.shape[2]
    if heads % hkv != 0:
        raise ValueError(f"heads {heads} must be a multiple of KV heads {hkv}")
    return x.repeat_interleave(heads // hkv, dim=2)


def attention_full_mask(
    q: Tensor, keys: Tensor, values: Tensor, qpos: Tensor, kpos: Tensor, window: int
) -> Tensor:
    """Masked softmax over every key at once: ``kpos <= qpos`` and ``kpos > qpos - window``.

    ``q [b, n, h, dk]``, ``keys, values [b, s, hkv, dk]``, ``qpos [b, n]``, ``kpos [b, s]``.
    A query with no visible key gets zeros (it cannot arise in the index-space contract).
    """
    h, dk = q.shape[2], q.shape[3]
    kk = _expand_kv(keys, h).permute(0, 2, 3, 1)  # [b, h, dk, s]
    vv = _expand_kv(values, h).permute(0, 2, 1, 3)  # [b, h, s, dk]
    scores = (q.permute(0, 2, 1, 3) @ kk) / math.sqrt(dk)  # [b, h, n, s]
    allowed = (kpos[:, None, :] <= qpos[:, :, None]) & (kpos[:, None, :] > qpos[:, :, None] - window)
    scores = scores.masked_fill(~allowed[:, None], float("-inf"))
    peak = scores.amax(dim=-1, keepdim=True).clamp_min(torch.finfo(scores.dtype).min)
    weights = torch.exp(scores - peak)
    weights = weights / weights.sum(dim=-1, keepdim=True).clamp_min(torch.finfo(scores.dtype).tiny)
    return (weights @ vv).permute(0, 2, 1, 3)


def window_attention(
    q: Tensor, keys: Tensor, values: Tensor, window: int, active: Tensor | None = None, block: int | None = None
) -> Tensor:
    """Outputs ``[b, n, h, dk]`` of ``q`` over ``keys, values [b, m + n, hkv, dk]`` in index space.

    Computed in query blocks (``block`` rows, default ``window``) against the keys the block can
    see, so memory stays O(block * (block + window)) however long the sequence is.
    """
    if window < 1:
        raise ValueError(f"window must be at least 1, got {window}")
    b, n, _, _ = q.shape
    m = keys.shape[1] - n
    if m < 0:
        raise ValueError(f"keys hold {keys.shape[1]} rows, fewer than the {n} queries")
    step = block or max(window, 1)
    out = torch.zeros_like(q)
    for s in range(0, n, step):
        e = min(s + step, n)
        first = max(0, m + s - window + 1)
        last = m + e  # exclusive
        qpos = torch.arange(m + s, m + e).expand(b, e - s)
        kpos = torch.arange(first, last).expand(b, last - first)
        out[:, s:e] = attention_full_mask(q[:, s:e], keys[:, first:last], values[:, first:last], qpos, kpos, window)
    if active is not None:
        out = torch.where(active[:, :, None, None], out, torch.zeros_like(out))
    return out


def attend_positions(
    q: Tensor,
    k: Tensor,
    v: Tensor,
    pos: Tensor,
    cache_k: Tensor,
    cache_v: Tensor,
    cache_pos: Tensor,
    window: int,
) -> Tensor:
    """The reference's blocked path over absolute positions (``vesper/attention.py:384-407``).

    Query block ``[s, e)`` of ``w`` rows attends the cache only while ``s < w`` and the chunk keys
    ``[s - w + 1, e)``, under the position mask.
    """
    n, w = q.shape[1], window
    outs = []
    for s in range(0, n, w):
        e = min(s + w, n)
        first = max(0, s - w + 1)
        if s < w:
            keys = torch.cat([cache_k, k[:, first:e]], dim=1)
            vals = torch.cat([cache_v, v[:, first:e]], dim=1)
            kpos = torch.cat([cache_pos, pos[:, first:e]], dim=1)
        else:
            keys, vals, kpos = k[:, first:e], v[:, first:e], pos[:, first:e]
        outs.append(attention_full_mask(q[:, s:e], keys, vals, pos[:, s:e], kpos, w))
    if not outs:
        return q.new_zeros(q.shape)
    return torch.cat(outs, dim=1)


def kv_cache_push(
    cache_k: Tensor, cache_v: Tensor, cache_pos: Tensor, k: Tensor, v: Tensor, pos: Tensor, window: int
) -> tuple[Tensor, Tensor, Tensor]:
    """The newest ``min(m + n, window)`` entries, oldest first (``vesper/attention.py:142-175``)."""
    m, n = cache_k.shape[1], k.shape[1]
    if n == 0:
        return cache_k, cache_v, cache_pos
    keep_new = min(n, window)
    keep_old = min(m, window - keep_new)
    return (
        torch.cat([cache_k[:, m - keep_old :], k[:, n - keep_new :]], dim=1),
        torch.cat([cache_v[:, m - keep_old :], v[:, n - keep_new :]], dim=1),
        torch.cat([cache_pos[:, m - keep_old :], pos[:, n - keep_new :]], dim=1),
    )


def ring_attend(
    q: Tensor,
    k: Tensor,
    v: Tensor,
    pos: Tensor,
    ring_k: Tensor,
    ring_v: Tensor,
    ring_pos: Tensor,
    ring_valid: Tensor,
    window: int,
) -> Tensor:
    """One token per row over the ring and itself (``vesper/attention.py:298-338``).

    ``q [b, 1, h, dk]``, ``k, v [b, 1, hkv, dk]``, ``pos [b, 1]``, ring ``[b, w, hkv, dk]`` with
    ``ring_pos [b, w]`` and ``ring_valid [b, w]``. Keys are the ring's slots then the new token;
    visibility is ``valid & kpos <= p & kpos > p - w`` (the new token is always visible).
    """
    keys = torch.cat([ring_k.to(q.dtype), k.to(q.dtype)], dim=1)
    vals = torch.cat([ring_v.to(q.dtype), v.to(q.dtype)], dim=1)
    kpos = torch.cat([ring_pos, pos], dim=1)
    valid = torch.cat([ring_valid, torch.ones_like(ring_valid[:, :1])], dim=1)
    # an invalid slot is given a position no query can see, so the shared mask applies as is
    hidden = pos.max() + window + 1
    kpos = torch.where(valid, kpos, torch.full_like(kpos, int(hidden)))
    return attention_full_mask(q, keys, vals, pos, kpos, window)


def kv_ring_write(
    ring_k: Tensor, ring_v: Tensor, ring_pos: Tensor, ring_valid: Tensor, k: Tensor, v: Tensor, pos: Tensor
) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    """Each row writes its token into slot ``pos % w`` (``vesper/attention.py:104-139``); new tensors."""
    if bool((pos < 0).any()):
        raise ValueError("positions must be nonnegative")
    w = ring_k.shape[1]
    rows = torch.arange(ring_k.shape[0])
    slot = (pos[:, 0] % w).long()
    nk, nv, npos, nvalid = ring_k.clone(), ring_v.clone(), ring_pos.clone(), ring_valid.clone()
    nk[rows, slot] = k[:, 0].to(nk.dtype)
    nv[rows, slot] = v[:, 0].to(nv.dtype)
    npos[rows, slot] = pos[:, 0]
    nvalid[rows, slot] = True
    return nk, nv, npos, nvalid


def rotary(x: Tensor, pos: Tensor, base: float) -> Tensor:
    """Rotary position embedding of ``x [b, n, heads, dk]`` at int64 positions ``pos [b, n]``
    (``vesper/attention.py:178-217``): the inverse frequencies ``base^(-2j/dk)`` and the angles
    ``pos * inv_freq`` in float64, their ``cos`` and ``sin`` cast to ``x.dtype``, then
    ``(x1 cos - x2 sin, x1 sin + x2 cos)`` per pair in ``x.dtype``. ``pos = 0`` returns ``x``."""
    b, n, _, dk = x.shape
    if pos.shape != (b, n) or pos.dtype != torch.long:
        raise ValueError(f"pos must be int64 {(b, n)}, got {pos.dtype} {tuple(pos.shape)}")
    if dk % 2 != 0:
        raise ValueError(f"dk must be even for rotary pairs, got {dk}")
    if not 1.0 < base < float("inf"):
        raise ValueError(f"rotary base must be finite and above 1, got {base}")
    exponent = torch.arange(0, dk // 2, dtype=torch.float64) * (2.0 / dk)
    angle = pos.to(torch.float64)[:, :, None] * base ** (-exponent)
    cos = angle.cos().to(x.dtype)[:, :, None, :]
    sin = angle.sin().to(x.dtype)[:, :, None, :]
    x1, x2 = x[..., 0::2], x[..., 1::2]
    return torch.stack([x1 * cos - x2 * sin, x1 * sin + x2 * cos], dim=-1).flatten(-2)
