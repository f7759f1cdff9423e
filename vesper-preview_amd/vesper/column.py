"""The column's recurrent sublayer and scan switch on MI355X: which delta-rule scan runs, and where.

Mirrors the reference's backend selection (``vesper/column.py:47-53``, ``:192-352``,
``:353-441``) with the same names, the same refusals and the same messages' key phrases, so a
driver written against the reference keeps its checks:

- ``ScanImpl`` / ``SCAN_IMPLS`` / ``FUSED_INPUT_DTYPES``: "fused" runs ``delta_scan_fused``
  (bfloat16 inputs, float32 state), "fused-fp32" runs ``delta_scan_fused_fp32`` (float32
  throughout), both HIP kernels; "reference" runs ``vesper.recurrence.delta_scan_chunked``, the
  plain PyTorch chunked scan, on whatever device the tensors are on (the reference's eager truth
  and CPU path; never chosen implicitly, never a fallback of the HIP scans).
- ``check_scan`` / ``check_capturable_scan``: the device checks of a choice, before any step;
  "reference" passes ``check_scan`` anywhere and is refused by ``check_capturable_scan`` on the
  GPU (a triangular solve per block is not a capturable scan).
- ``set_scan`` / ``scan_of``: one choice for every ``RecurrentSublayer`` of a model.
- ``RecurrentSublayer``: the projections around the scan: ``project`` (``q``, the key input
  ``z``, ``v``, ``beta = sigmoid(W_beta x)``), ``keys`` (the causal key filter and
  ``normalize_keys``, ``recurrent_keys``), ``scan`` (the chosen scan and ``W_o``).
- ``recurrent_scan``: the scan part of ``RecurrentSublayer.scan`` (``column.py:291-326``).
- ``recurrent_keys``: ``RecurrentSublayer.keys`` (``column.py:255-289``) on the key filter kernel.
"""

from __future__ import annotations

import math
from typing import Literal

import torch
from torch import Tensor, nn

from vesper.kernels.keys import fused_keys, key_step
from vesper.kernels.delta_scan import (
    FP32_INPUT_DTYPE,
    INPUT_DTYPE,
    STATE_DTYPE,
    delta_scan_fused,
    delta_scan_fused_fp32,
    fused_scan_available,
)
from vesper.recurrence import delta_scan_chunked

ScanImpl = Literal["reference", "fused", "fused-fp32"]
SCAN_IMPLS: tuple[ScanImpl, ...] = ("reference", "fused", "fused-fp32")
# what each HIP scan takes its q, k, v, beta in; the reference takes promote_types(dtype, float32)
FUSED_INPUT_DTYPES: dict[ScanImpl, torch.dtype] = {
    "fused": INPUT_DTYPE,
    "fused-fp32": FP32_INPUT_DTYPE,
}


def check_scan(impl: str, device: torch.device) -> ScanImpl:
    """Validate ``impl`` for a model whose parameters live on ``device`` and return it as a
    ``ScanImpl`` (the contract of ``column.py:382-405``).

    The PyTorch "reference" scan is accepted on any device; "fused" and "fused-fp32" are this
    package's HIP kernels, so they need a GPU device and ``libvesper_kernels.so`` loaded.

    Raises:
        ValueError: for a name outside ``SCAN_IMPLS``; for a HIP scan on a non-GPU device or when
            the kernel library is not available.
    """
    if impl == "reference":
        return "reference"
    if impl not in FUSED_INPUT_DTYPES:
        raise ValueError(f"scan must be one of {SCAN_IMPLS}, got {impl!r}")
    if device.type != "cuda":
        raise ValueError(f"the fused scan needs the model on CUDA, got {device}")
    if not fused_scan_available():
        raise ValueError("the fused scan needs a HIP device and the built kernel library (libvesper_kernels.so)")
    return "fused" if impl == "fused" else "fused-fp32"


def check_capturable_scan(impl: str, device: torch.device) -> ScanImpl:
    """Like ``check_scan``, for a caller that will replay the scan from a captured HIP graph
    (``column.py:408-426``). The HIP scans allocate nothing and never synchronise with the host,
    so either captures; the PyTorch scan on a GPU does not (it solves a triangular system per
    block) and is turned down there.

    Raises:
        ValueError: whatever ``check_scan`` raises, and for "reference" on a GPU device.
    """
    chosen = check_scan(impl, device)
    if chosen == "reference" and device.type == "cuda":
        raise ValueError("the reference scan cannot run as a captured graph (a triangular solve per block); "
                         "on the GPU use fused or fused-fp32")
    return chosen


def set_scan(model: nn.Module, impl: str) -> int:
    """Switch every ``RecurrentSublayer`` of ``model`` to the scan ``impl`` (``column.py:353-380``).

    The choice is validated with ``check_scan`` for the device of each parameter first, so a
    refused choice leaves the model as it was.

    Returns:
        How many sublayers now use ``impl``.

    Raises:
        ValueError: for a name outside ``SCAN_IMPLS``, a model without recurrent sublayers, or a
            HIP scan on a device where ``check_scan`` turns it down.
    """
    if impl not in SCAN_IMPLS:
        raise ValueError(f"scan must be one of {SCAN_IMPLS}, got {impl!r}")
    sublayers = [m for m in model.modules() if isinstance(m, RecurrentSublayer)]
    if not sublayers:
        raise ValueError("the model has no recurrent sublayer to set")
    chosen: ScanImpl = "reference"
    for device in sorted({p.device for p in model.parameters()}, key=str):
        chosen = check_scan(impl, device)
    for sublayer in sublayers:
        sublayer.scan_impl = chosen
    return len(sublayers)


def scan_of(model: nn.Module) -> ScanImpl:
    """The one scan implementation shared by all of ``model``'s ``RecurrentSublayer`` modules
    (``column.py:428-441``).

    Raises:
        ValueError: when there is no recurrent sublayer, or when they do not all use the same scan.
    """
    impls = {m.scan_impl for m in model.modules() if isinstance(m, RecurrentSublayer)}
    if len(impls) != 1:
        raise ValueError(f"recurrent sublayers use {sorted(impls)} scan implementations, expected exactly one")
    return impls.pop()


def recurrent_scan(impl: str, q: Tensor, k: Tensor, v: Tensor, beta: Tensor, state: Tensor, *,
                   active: Tensor | None = None, block: int = 64) -> tuple[Tensor, Tensor]:
    """The scan of ``RecurrentSublayer.scan`` without its output projection: ``(o, state')``.

    ``q, k, v [b, n, h, dk]`` and ``beta [b, n, h]`` in the projections' dtype; ``state
    [b, h, dk, dk]``. The HIP scans take their input dtype with autocast off and return ``o`` in
    ``q``'s dtype and the state in float32; the reference scan runs in ``promote_types(dtype,
    float32)`` (``column.py:316-325``) and returns its state in that dtype.

    Raises:
        ValueError: as ``check_scan``.
        ContractError: from the kernel's contract check.
    """
    chosen = check_scan(impl, q.device)
    if chosen == "reference":
        compute = torch.promote_types(q.dtype, torch.float32)
        with torch.autocast(device_type=q.device.type, enabled=False):
            o, new_state = delta_scan_chunked(q.to(compute), k.to(compute), v.to(compute), beta.to(compute),
                                              state.to(compute), block, active=active)
        return o.to(q.dtype), new_state
    kernel = delta_scan_fused if chosen == "fused" else delta_scan_fused_fp32
    dtype = FUSED_INPUT_DTYPES[chosen]
    with torch.autocast(device_type=q.device.type, enabled=False):
        o, new_state = kernel(q.to(dtype), k.to(dtype), v.to(dtype), beta.to(dtype), state.to(STATE_DTYPE),
                              active=active)
    return o.to(q.dtype), new_state


class RecurrentSublayer(nn.Module):
    """The projections around the delta-rule scan (``column.py:192-352``).

    ``w_q, w_k, w_v, w_o`` of ``[d, d]`` and ``w_beta`` of ``[h, d]``, drawn ``N(0, 1/d)`` in that
    order, then the optional causal key filter ``conv_k [K, d]`` ~ ``U(-1/sqrt(K), 1/sqrt(K))``
    (``column.py:216-233``). ``scan_impl`` is module state (``set_scan``), never a parameter.
    """

    def __init__(self, d: int, heads: int, key_conv: int = 0, block: int = 64,
                 generator: torch.Generator | None = None) -> None:
        super().__init__()
        if d % heads != 0:
            raise ValueError(f"heads ({heads}) must divide d ({d})")
        if block < 1:
            raise ValueError(f"block must be at least 1, got {block}")
        self.heads, self.head_dim, self.block, self.key_conv = heads, d // heads, block, key_conv
        self.scan_impl: ScanImpl = "reference"
        std = 1.0 / math.sqrt(d)
        self.w_q = nn.Parameter(torch.randn(d, d, generator=generator) * std)
        self.w_k = nn.Parameter(torch.randn(d, d, generator=generator) * std)
        self.w_v = nn.Parameter(torch.randn(d, d, generator=generator) * std)
        self.w_o = nn.Parameter(torch.randn(d, d, generator=generator) * std)
        self.w_beta = nn.Parameter(torch.randn(heads, d, generator=generator) * std)
        self.conv_k: nn.Parameter | None = None
        if key_conv:
            bound = 1.0 / math.sqrt(key_conv)
            self.conv_k = nn.Parameter(torch.rand(key_conv, d, generator=generator) * (2 * bound) - bound)

    def project(self, x: Tensor) -> tuple[Tensor, Tensor, Tensor, Tensor]:
        """``[b, n, d]`` to ``q [b, n, h, dk]`` (not normalized), the key input ``z [b, n, d]``,
        ``v [b, n, h, dk]`` and ``beta = sigmoid(W_beta x) [b, n, h]`` (``column.py:236-253``)."""
        b, n, _ = x.shape
        q = nn.functional.linear(x, self.w_q).view(b, n, self.heads, self.head_dim)
        z = nn.functional.linear(x, self.w_k)
        v = nn.functional.linear(x, self.w_v).view(b, n, self.heads, self.head_dim)
        return q, z, v, torch.sigmoid(nn.functional.linear(x, self.w_beta))

    def keys(self, z: Tensor, history: Tensor) -> tuple[Tensor, Tensor]:
        """Normalized keys and the next key history (``column.py:255-289``) on the key kernel."""
        return recurrent_keys(z, history, self.conv_k, self.heads)

    def scan(self, q: Tensor, k: Tensor, v: Tensor, beta: Tensor, state: Tensor) -> tuple[Tensor, Tensor]:
        """The chosen scan and the output projection: ``(y [b, n, d], state')`` (``column.py:291-326``)."""
        o, new_state = recurrent_scan(self.scan_impl, q, k, v, beta, state, block=self.block)
        return nn.functional.linear(o.flatten(2), self.w_o), new_state

    def forward(self, x: Tensor, state: Tensor, history: Tensor) -> tuple[Tensor, Tensor, Tensor]:
        """Project, make the keys, scan: ``(y, state', history')`` (``column.py:328-350``)."""
        q, z, v, beta = self.project(x)
        k, history_next = self.keys(z, history)
        y, state_next = self.scan(q, k, v, beta, state)
        return y, state_next, history_next


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
