"""CPU oracle of the causal key filter and key normalization (test infrastructure only; see
``oracle/__init__.py``).

Restated from ``RecurrentSublayer.keys`` (``vesper/column.py:255-289``), which the reference's
fused kernel ``fused_keys`` (``vesper/kernels/keys.py:28-32``) computes on CUDA:

- ``u[t, j] = sum_{r=0}^{K-1} taps[r, j] * z[t - r, j]``: depthwise, no bias, ``r = 0`` the current
  token; positions before the chunk come from ``history [b, K-1, d]`` (oldest first);
- the key is ``normalize_keys`` of ``u`` per head (``[b, n, heads, d / heads]``), after the filter;
- the filter runs in float32 or wider, and the key returns in ``z``'s dtype;
- the next history is the newest ``K - 1`` inputs of ``(history, z)`` in the filter's dtype: the
  history itself for an empty chunk, partly old for a chunk shorter than ``K - 1``;
- with no filter (``taps`` None) the key is ``normalize_keys(z)`` and the history passes through.

``filter_keys_literal`` is the operator by its definition, one position and tap at a time (the form
of the reference's own test, ``tests/test_key_conv.py:58-69``); ``filter_keys`` is the same
arithmetic vectorized, in the reference module's order of operations (``column.py:284-288``).
``filter_keys_grads`` is its backward by autograd, ``filter_keys_grads_literal`` the same gradients
written out per position; both are pinned by finite differences.
"""

from __future__ import annotations

import torch
from torch import Tensor

from oracle.delta import normalize_keys


def _compute_dtype(z: Tensor) -> torch.dtype:
    return torch.promote_types(z.dtype, torch.float32)


def filter_keys(z: Tensor, history: Tensor, taps: Tensor | None, heads: int) -> tuple[Tensor, Tensor]:
    """``(keys [b, n, heads, d / heads] in z's dtype, next history [b, K-1, d])``."""
    b, n, d = z.shape
    head_dim = d // heads
    if taps is None or n == 0:
        return normalize_keys(z.view(b, n, heads, head_dim)), history
    width = int(taps.shape[0])
    compute = _compute_dtype(z)
    full = torch.cat([history.to(compute), z.to(compute)], dim=1)  # [b, K - 1 + n, d]
    w = taps.to(compute)
    u = w[0] * full[:, width - 1 : width - 1 + n]
    for r in range(1, width):
        u = u + w[r] * full[:, width - 1 - r : width - 1 - r + n]
    keys = normalize_keys(u.view(b, n, heads, head_dim)).to(z.dtype)
    return keys, full[:, n:].clone()


def filter_keys_literal(z: Tensor, history: Tensor, taps: Tensor, heads: int) -> tuple[Tensor, Tensor]:
    """The operator by its definition, one position and tap at a time (float64 in, float64 out)."""
    b, n, d = z.shape
    width = int(taps.shape[0])
    full = torch.cat([history, z], dim=1)  # chunk position t is row K - 1 + t
    u = torch.zeros(b, n, d, dtype=z.dtype)
    for t in range(n):
        for r in range(width):
            u[:, t] += taps[r] * full[:, width - 1 + t - r]
    keys = normalize_keys(u.view(b, n, heads, d // heads))
    return keys, full[:, full.shape[1] - (width - 1) :]


def filter_keys_grads(z: Tensor, history: Tensor, taps: Tensor, heads: int,
                      grad_keys: Tensor) -> tuple[Tensor, Tensor, Tensor]:
    """``(d z, d history, d taps)`` of ``sum(keys * grad_keys)`` by autograd through ``filter_keys``.

    The backward the reference's ``_FusedKeys`` computes on CUDA (``vesper/kernels/keys.py:46-78``):
    the normalization's peak held constant (``recurrence.py:103-105``), the clamp of the squared
    norm at one passing gradient at and above one.
    """
    zs = z.detach().clone().requires_grad_()
    hs = history.detach().clone().requires_grad_()
    ts = taps.detach().clone().requires_grad_()
    keys, _ = filter_keys(zs, hs, ts, heads)
    (keys * grad_keys.to(keys.dtype)).sum().backward()
    assert zs.grad is not None and hs.grad is not None and ts.grad is not None
    return zs.grad, hs.grad, ts.grad


def filter_keys_grads_literal(z: Tensor, history: Tensor, taps: Tensor, heads: int,
                              grad_keys: Tensor) -> tuple[Tensor, Tensor, Tensor]:
    """The same gradients written out per position (float64 in, float64 out).

    Per token and head, with ``s = u / peak``, ``q = |s|^2``, ``den = sqrt(max(q, 1))`` and the key's
    gradient ``g``: ``d u = (g / den - [q >= 1] s (g . s) / den^3) / peak`` (``keys_triton.py:87-94``);
    then ``d z[t] = sum_r taps[r] d u[t + r]``, ``d taps[r] = sum_t d u[t] full[t - r]`` and history
    row ``p`` collects ``taps[r] d u[t]`` for ``t = p - (K - 1) + r`` (``keys.py:66-78``).
    """
    b, n, d = z.shape
    width = int(taps.shape[0])
    hd = d // heads
    full = torch.cat([history, z], dim=1)  # chunk position t is row K - 1 + t
    u = torch.zeros(b, n, d, dtype=z.dtype)
    for t in range(n):
        for r in range(width):
            u[:, t] += taps[r] * full[:, width - 1 + t - r]
    uh = u.view(b, n, heads, hd)
    peak = uh.abs().amax(dim=-1, keepdim=True).clamp_min(1e-6)
    s = uh / peak
    q = (s * s).sum(dim=-1, keepdim=True)
    den = q.clamp_min(1.0).sqrt()
    g = grad_keys.view(b, n, heads, hd).to(z.dtype)
    through = torch.where(q >= 1.0, s * ((g * s).sum(dim=-1, keepdim=True) / den**3), torch.zeros_like(s))
    du = ((g / den - through) / peak).view(b, n, d)
    dz = torch.zeros_like(z)
    dtaps = torch.zeros_like(taps)
    dhist = torch.zeros_like(history)
    for t in range(n):
        for r in range(width):
            if t + r < n:
                dz[:, t] += taps[r] * du[:, t + r]
            dtaps[r] += (du[:, t] * full[:, width - 1 + t - r]).sum(dim=0)
    for p in range(width - 1):
        for r in range(width - 1 - p, width):
            t = p - (width - 1) + r
            if t < n:
                dhist[:, p] += taps[r] * du[:, t]
    return dz, dhist, dtaps
