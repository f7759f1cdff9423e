"""The column's scan switch, for the HIP scans: which delta-rule kernel a recurrent sublayer runs.

Mirrors the reference's backend selection (``vesper/column.py:47-53``, ``:291-326``,
``:382-426``) with the same names and the same refusals, so a driver written against the
reference keeps its checks:

- ``ScanImpl`` / ``SCAN_IMPLS`` / ``FUSED_INPUT_DTYPES``: "fused" runs ``delta_scan_fused``
  (bfloat16 inputs, float32 state), "fused-fp32" runs ``delta_scan_fused_fp32`` (float32
  throughout). "reference" names the reference's pure-PyTorch scan (``vesper/recurrence.py``),
  which this build does not ship: asking for it is refused with a message saying so.
- ``check_scan`` / ``check_capturable_scan``: the device checks of a choice, before any step.
- ``recurrent_scan``: the kernel part of ``RecurrentSublayer.scan`` (``column.py:308-315``):
  cast ``q, k, v, beta`` to the choice's input dtype and the state to float32 with autocast off,
  run the kernel, return the reads in the projections' dtype and the new float32 state. The
  output projection ``W_o`` stays with the caller.
- ``recurrent_keys``: ``RecurrentSublayer.keys`` (``column.py:255-289``) on the key filter kernel:
  the normalized keys and the next key history, for a filter or none.
"""

from __future__ import annotations

from typing import Literal

import torch
from torch import Tensor

from vesper.kernels.keys import fused_keys, key_step
from vesper.kernels.delta_scan import (
    FP32_INPUT_DTYPE,
    INPUT_DTYPE,
    STATE_DTYPE,
    delta_scan_fused,
    delta_scan_fused_fp32,
    fused_scan_available,
)

ScanImpl = Literal["reference", "fused", "fused-fp32"]
SCAN_IMPLS: tuple[ScanImpl, ...] = ("reference", "fused", "fused-fp32")
# what each HIP scan takes its q, k, v, beta in
FUSED_INPUT_DTYPES: dict[ScanImpl, torch.dtype] = {
    "fused": INPUT_DTYPE,
    "fused-fp32": FP32_INPUT_DTYPE,
}


def check_scan(impl: str, device: torch.device) -> ScanImpl:
    """The one check of a scan choice against the device it would run on; returns it typed.

    Raises:
        ValueError: if ``impl`` is not one of ``SCAN_IMPLS``; for "reference" (not shipped by this
            build); for a HIP scan off the GPU or without the built kernel library.
    """
    if impl == "reference":
        raise ValueError(
            "the reference scan is the pure-PyTorch path of vesper/recurrence.py, which this build does "
            "not ship; use fused or fused-fp32"
        )
    if impl not in FUSED_INPUT_DTYPES:
        raise ValueError(f"scan must be one of {SCAN_IMPLS}, got {impl!r}")
    if device.type != "cuda":
        raise ValueError(f"the fused scan needs the model on CUDA, got {device}")
    if not fused_scan_available():
        raise ValueError("the fused scan needs a HIP device and the built kernel library (libvesper_kernels.so)")
    return "fused" if impl == "fused" else "fused-fp32"


def check_capturable_scan(impl: str, device: torch.device) -> ScanImpl:
    """``check_scan``: both HIP scans run inside a captured HIP graph (no allocation in the library,
    no host synchronisation), so every choice that passes it can be captured."""
    return check_scan(impl, device)


def recurrent_scan(impl: str, q: Tensor, k: Tensor, v: Tensor, beta: Tensor, state: Tensor, *,
                   active: Tensor | None = None) -> tuple[Tensor, Tensor]:
    """The scan of ``RecurrentSublayer.scan`` without its output projection: ``(o, state')``.

    ``q, k, v [b, n, h, dk]`` and ``beta [b, n, h]`` in the projections' dtype; ``state
    [b, h, dk, dk]`` in any float dtype. Returns ``o`` in ``q``'s dtype and the state in float32.

    Raises:
        ValueError: as ``check_scan``.
        ContractError: from the kernel's contract check.
    """
    chosen = check_scan(impl, q.device)
    kernel = delta_scan_fused if chosen == "fused" else delta_scan_fused_fp32
    dtype = FUSED_INPUT_DTYPES[chosen]
    with torch.autocast(device_type=q.device.type, enabled=False):
        o, new_state = kernel(q.to(dtype), k.to(dtype), v.to(dtype), beta.to(dtype), state.to(STATE_DTYPE),
                              active=active)
    return o.to(q.dtype), new_state


def recurrent_keys(z: Tensor, history: Tensor, taps: Tensor | None, heads: int, *, active: Tensor | None = None,
                   carried_z: Tensor | None = None) -> tuple[Tensor, Tensor]:
    """Normalized keys ``[b, n, heads, d / heads]`` of key inputs ``z [b, n, d]`` and the next history.

    With a filter (``taps [K, d]``) the key of token ``t`` is ``normalize_keys`` per head of
    ``sum_r taps[r] * z[t - r]``, the positions before the chunk from ``history [b, K-1, d]``
    (oldest first); the next history is the newest ``K - 1`` inputs of ``(history, z)`` as an owned
    float32 copy. With no filter (``taps`` None) the key is ``normalize_keys(z)`` and the history
    object passes through; so it does for an empty chunk. ``carried_z`` with ``active`` replaces the
    key inputs of inactive tokens, in the keys (inside the kernel's loads) and in the next history.

    Raises:
        ContractError: as ``fused_keys``.
    """
    b, n, d = z.shape
    if taps is None or n == 0:
        if n == 0:
            return z.new_empty(b, 0, heads, d // heads), history
        ones = torch.ones(1, d, dtype=torch.float32, device=z.device)
        return fused_keys(z, z.new_empty(b, 0, d, dtype=torch.float32), ones, heads, active=active,
                          carried_z=carried_z), history
    inputs = (z, history, taps) if carried_z is None else (z, history, taps, carried_z)
    if not (torch.is_grad_enabled() and any(t.requires_grad for t in inputs)):
        return key_step(z, history, taps, heads, active=active, carried_z=carried_z)  # keys and history, one launch
    width = int(taps.shape[0])
    keys = fused_keys(z, history, taps, heads, active=active, carried_z=carried_z)
    first = max(0, n - (width - 1))
    tail = z[:, first:]
    if carried_z is not None and active is not None:
        tail = torch.where(active[:, first:, None], tail, carried_z[:, first:])
    return keys, torch.cat([history.to(torch.float32)[:, n:], tail.to(torch.float32)], dim=1)
