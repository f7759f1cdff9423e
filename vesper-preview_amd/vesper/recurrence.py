"""The delta rule's reference backend: the chunked scan in plain PyTorch, for the scan switch.

The reference names three scan implementations (``vesper/column.py:47-53``): "fused" and
"fused-fp32" (here the HIP kernels, ``vesper.kernels.delta_scan``) and "reference", its own
pure-PyTorch chunked scan (``vesper/recurrence.py:166-217``), which stays valid on any device as
the eager truth of equivalence tests and as the CPU path. ``delta_scan_chunked`` here is that
backend, written for this package: per block of ``C`` tokens, with ``A = tril(diag(beta) K K^T,
-1)``, the UT factors ``W = (I + A)^-1 diag(beta) K`` and ``U = (I + A)^-1 diag(beta) V`` by one
unit-triangular solve each, then ``Delta = U - W H``, ``O = Q H + tril(Q K^T) Delta`` and
``H <- H + K^T Delta`` (the WY/UT form, Yang et al. 2024).

It runs only when a caller selects "reference" (``vesper.column.set_scan``): the HIP entry points
never fall back to it, and it never imports anything of the test oracle.
"""

from __future__ import annotations

import torch
from torch import Tensor

from vesper.contracts import ContractError, Dims, check_shape


def delta_scan_chunked(q: Tensor, k: Tensor, v: Tensor, beta: Tensor, state: Tensor, block: int = 64, *,
                       active: Tensor | None = None) -> tuple[Tensor, Tensor]:
    """``(o [b, n, h, dk], state')`` of the delta rule over ``n`` tokens, in ``q``'s dtype.

    ``q, k, v [b, n, h, dk]``, ``beta [b, n, h]``, ``state [b, h, dk, dk]`` read as ``H^T q``. With
    ``active`` (bool ``[b, n]``) inactive tokens' outputs are zero; every token writes the state.
    ``n == 0`` returns ``(q, state)``, the same objects (``recurrence.py:198-199``).

    Raises:
        ContractError: on shapes that disagree; ValueError: ``block`` below 1.
    """
    dims: Dims = {}
    check_shape("q", q, ("b", "n", "h", "dk"), dims)
    check_shape("k", k, ("b", "n", "h", "dk"), dims)
    check_shape("v", v, ("b", "n", "h", "dk"), dims)
    check_shape("beta", beta, ("b", "n", "h"), dims)
    check_shape("state", state, ("b", "h", "dk", "dk"), dims)
    if block < 1:
        raise ValueError(f"block must be at least 1, got {block}")
    n = dims["n"]
    if n == 0:
        return q, state
    h_state = state
    outs = []
    for s in range(0, n, block):
        e = min(s + block, n)
        qc, kc, vc = (t[:, s:e].transpose(1, 2) for t in (q, k, v))  # [b, h, c, dk]
        bc = beta[:, s:e].transpose(1, 2).unsqueeze(-1)  # [b, h, c, 1]
        c = e - s
        unit = torch.eye(c, dtype=q.dtype, device=q.device)
        lower = unit + torch.tril(bc * (kc @ kc.transpose(-1, -2)), -1)
        w_rows = torch.linalg.solve_triangular(lower, bc * kc, upper=False, unitriangular=True)
        u_rows = torch.linalg.solve_triangular(lower, bc * vc, upper=False, unitriangular=True)
        delta = u_rows - w_rows @ h_state
        outs.append((qc @ h_state + torch.tril(qc @ kc.transpose(-1, -2)) @ delta).transpose(1, 2))
        h_state = h_state + kc.transpose(-1, -2) @ delta
    o = torch.cat(outs, dim=1)
    if active is not None:
        if active.shape != (dims["b"], n) or active.dtype != torch.bool:
            raise ContractError(f"active: expected bool {(dims['b'], n)}, got {active.dtype} {tuple(active.shape)}")
        o = torch.where(active[:, :, None, None], o, torch.zeros_like(o))
    return o, h_state
