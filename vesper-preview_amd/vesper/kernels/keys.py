"""The causal key filter and key normalization on MI355X: HIP kernels behind the reference's contract.

``fused_keys(z, history, taps, heads)`` keeps the signature, result and gradients of the
reference's ``vesper/kernels/keys.py:28-78`` (what ``RecurrentSublayer.keys``,
``vesper/column.py:255-289``, computes for its key): ``u[t] = sum_r taps[r] * z[t - r]`` with the
chunk's predecessors from ``history``, then ``normalize_keys`` per head, float32 arithmetic, the key
in ``z``'s dtype. Where the reference runs Triton kernels, this calls ``vsp_key_filter_*`` (forward)
and ``vsp_key_filter_backward_*`` (the gradients of ``z``, ``taps`` and, when it needs one,
``history``; the normalization's peak held constant as the reference detaches it) through the C ABI.

For: float32, bfloat16 or float16 key inputs on the GPU, a filter of 1 to 8 taps, head widths that
are powers of two from 8 to 512.

With ``active`` and ``carried_z`` (the copy-forward of halted tokens' key inputs, selected before the
filter, ``vesper/column.py:779-782``) the kernel reads token ``t``'s input row from ``carried_z``
where ``active[:, t]`` is false, inside its loads, in place of a ``where`` merge before the call.
``key_step`` returns the next key history too, written by the same kernel launch
(``vsp_key_step_*``): the whole of ``RecurrentSublayer.keys`` (``vesper/column.py:255-289``).

``normalize_keys(k)`` is the reference's ``vesper/recurrence.py:91-115`` alone on rows of any width
(``vsp_normalize_keys_*``, one wave a row, with its gradient), for rows the filter's head widths
do not cover: wider than 512, or not a power of two.
"""

from __future__ import annotations

from typing import Any

import torch
from torch import Tensor

from vesper.contracts import ContractError, Dims, check_shape
from vesper.kernels import _lib

FUSED_KEY_DTYPES = (torch.float32, torch.bfloat16, torch.float16)
MAX_TAPS = 8
_SUFFIX = {torch.bfloat16: "bf16", torch.float16: "f16", torch.float32: "f32"}


def _aligned(t: Tensor) -> Tensor:
    t = t.contiguous()
    return t if t.data_ptr() % 16 == 0 else t.clone()


def _check(z: Tensor, history: Tensor, taps: Tensor, heads: int) -> tuple[int, int, int, int]:
    dims: Dims = {}
    check_shape("z", z, ("b", "n", "d"), dims)
    check_shape("taps", taps, ("K", "d"), dims)
    width = dims["K"]
    dims["Kh"] = width - 1
    check_shape("history", history, ("b", "Kh", "d"), dims)
    if z.dtype not in FUSED_KEY_DTYPES:
        raise ContractError(f"z: dtype must be float32, bfloat16 or float16, got {z.dtype}")
    if z.device.type != "cuda":
        raise ContractError(f"the key filter kernel runs on CUDA only, got z on {z.device}")
    for name, t in (("history", history), ("taps", taps)):
        if t.device != z.device:
            raise ContractError(f"{name} is on {t.device}, z on {z.device}")
    if not 1 <= width <= MAX_TAPS:
        raise ContractError(f"taps: the kernel takes 1..{MAX_TAPS} taps, got {width}")
    d = dims["d"]
    if heads < 1 or d % heads != 0:
        raise ContractError(f"{d} features are not a multiple of {heads} heads")
    head_dim = d // heads
    if head_dim < 8 or head_dim > 512 or head_dim & (head_dim - 1):
        raise ContractError(f"head width {head_dim}: the kernel takes powers of two 8..512")
    return dims["b"], dims["n"], d, width


class _FusedKeys(torch.autograd.Function):
    @staticmethod
    def forward(ctx: Any, z: Tensor, history: Tensor, taps: Tensor, heads: int) -> Tensor:  # noqa: D102
        b, n, d, width = _check(z, history, taps, heads)
        zc = _aligned(z)
        hist = _aligned(history.detach().to(torch.float32))
        wide = _aligned(taps.detach().to(torch.float32))
        out = torch.empty(b, n, heads, d // heads, dtype=z.dtype, device=z.device)
        if b and n:
            _lib.call(f"vsp_key_filter_{_SUFFIX[z.dtype]}", _lib.ptr(zc), _lib.ptr(hist) if width > 1 else None,
                      _lib.ptr(wide), _lib.ptr(out), b, n, d, heads, width, _lib.stream_of(z.device))
        ctx.save_for_backward(zc, hist, wide)
        ctx.heads = heads
        ctx.dtypes = (history.dtype, taps.dtype)
        return out

    @staticmethod
    def backward(ctx: Any, grad_keys: Tensor) -> tuple[Tensor | None, Tensor | None, Tensor | None, None]:  # noqa: D102
        zc, hist, wide = ctx.saved_tensors
        heads: int = ctx.heads
        b, n, d = zc.shape
        width = int(wide.shape[0])
        g = _aligned(grad_keys.to(zc.dtype).reshape(b, n, d))
        grad_z = torch.empty_like(zc)
        grad_taps = torch.empty(width, d, dtype=torch.float32, device=zc.device)
        want_history = ctx.needs_input_grad[1] and width > 1
        grad_history = torch.empty(b, width - 1, d, dtype=torch.float32, device=zc.device) if want_history else None
        nbytes = int(_lib.library().vsp_key_filter_backward_workspace_bytes(b, n, d, width))
        workspace = torch.empty(max(nbytes, 16), dtype=torch.uint8, device=zc.device)
        _lib.call(f"vsp_key_filter_backward_{_SUFFIX[zc.dtype]}", _lib.ptr(zc),
                  _lib.ptr(hist) if width > 1 else None, _lib.ptr(wide), _lib.ptr(g), _lib.ptr(grad_z),
                  _lib.ptr(grad_taps), None if grad_history is None else _lib.ptr(grad_history),
                  _lib.ptr(workspace), nbytes, b, n, d, heads, width, _lib.stream_of(zc.device))
        history_dtype, taps_dtype = ctx.dtypes
        d_history = None
        if ctx.needs_input_grad[1]:
            d_history = grad_history.to(history_dtype) if grad_history is not None else torch.zeros(
                b, 0, d, dtype=history_dtype, device=zc.device)
        return (grad_z if ctx.needs_input_grad[0] else None, d_history,
                grad_taps.to(taps_dtype) if ctx.needs_input_grad[2] else None, None)


def _key_step(z: Tensor, history: Tensor, taps: Tensor, heads: int, active: Tensor | None,
              carried_z: Tensor | None, want_history: bool, in_place: bool = False) -> tuple[Tensor, Tensor | None]:
    b, n, d, width = _check(z, history, taps, heads)
    zc = _aligned(z)
    held = None if carried_z is None else _aligned(carried_z)
    flags = None if carried_z is None or active is None else active.contiguous().view(torch.uint8)
    hist = history if in_place else _aligned(history.to(torch.float32))
    wide = _aligned(taps.to(torch.float32))
    out = torch.empty(b, n, heads, d // heads, dtype=z.dtype, device=z.device)
    if in_place:
        nxt = history
    else:
        nxt = torch.empty(b, width - 1, d, dtype=torch.float32, device=z.device) if want_history else None
    if b and n:
        _lib.call(f"vsp_key_step_{_SUFFIX[z.dtype]}", _lib.ptr(zc), _lib.ptr(held), _lib.ptr(flags),
                  _lib.ptr(hist) if width > 1 else None, _lib.ptr(wide), _lib.ptr(out),
                  _lib.ptr(nxt) if width > 1 else None, b, n, d, heads, width, _lib.stream_of(z.device))
    return out, nxt


def _check_carried(z: Tensor, active: Tensor | None, carried_z: Tensor) -> None:
    if active is None:
        raise ContractError("carried key inputs need the active mask that says which tokens read them")
    if carried_z.shape != z.shape or carried_z.dtype != z.dtype or carried_z.device != z.device:
        raise ContractError(f"carried_z: {tuple(carried_z.shape)} {carried_z.dtype} on {carried_z.device}, "
                            f"z is {tuple(z.shape)} {z.dtype} on {z.device}")
    check_shape("active", active, ("b", "n"), {"b": z.shape[0], "n": z.shape[1]}, torch.bool)
    if active.device != z.device:
        raise ContractError(f"active is on {active.device}, z on {z.device}")


def key_step(z: Tensor, history: Tensor, taps: Tensor, heads: int, *, active: Tensor | None = None,
             carried_z: Tensor | None = None, in_place: bool = False) -> tuple[Tensor, Tensor]:
    """The keys and the next key history of key inputs ``z [b, n, d]``, no gradient.

    As ``fused_keys`` for the keys; the next history is the newest ``K - 1`` inputs of ``(history,
    z)`` (with ``carried_z``, the carried rows of inactive tokens) as a new float32 ``[b, K-1, d]``
    tensor, written by the same launch; with ``in_place`` it is written into ``history`` itself
    (a contiguous float32 tensor) and that tensor returned: a decode step's update, for chunks of
    at most 16 tokens (8 with float32 ``z``). An empty chunk (``n == 0``) returns empty keys and
    the history unchanged, as ``RecurrentSublayer.keys`` does (``column.py:275-277``).

    Raises:
        ContractError: as ``fused_keys``; ``in_place`` with a history that is not contiguous
            float32 or a chunk longer than that.
    """
    _check(z, history, taps, heads)
    if in_place:
        limit = 8 if z.dtype == torch.float32 else 16
        if history.dtype != torch.float32 or not history.is_contiguous() or history.data_ptr() % 16:
            raise ContractError("an in-place history must be a contiguous, 16-byte aligned float32 tensor")
        if z.shape[1] > limit:
            raise ContractError(f"an in-place history takes chunks of at most {limit} tokens, got {z.shape[1]}")
    if carried_z is not None:
        _check_carried(z, active, carried_z)
    if z.shape[1] == 0:
        b, _, d = z.shape
        return z.new_empty(b, 0, heads, d // heads), history
    keys, nxt = _key_step(z, history, taps, heads, active, carried_z, want_history=True, in_place=in_place)
    assert nxt is not None
    return keys, nxt


def fused_keys(z: Tensor, history: Tensor, taps: Tensor, heads: int, *, active: Tensor | None = None,
               carried_z: Tensor | None = None) -> Tensor:
    """Normalized keys ``[b, n, heads, d / heads]`` in ``z``'s dtype (``z [b, n, d]`` on the GPU).

    ``history [b, K-1, d]`` holds the ``K - 1`` key inputs before the chunk (oldest first) and
    ``taps [K, d]`` the filter, tap 0 on the current token; both are used in float32. Under autograd
    the gradients of ``z`` (in its dtype), ``taps`` and ``history`` (in theirs) come from the
    backward kernel. ``carried_z`` (shaped and typed as ``z``, with ``active`` bool ``[b, n]``)
    replaces the key inputs of inactive tokens.

    Raises:
        ContractError: on shapes that disagree, a dtype outside float32/bfloat16/float16, tensors
            off the GPU or on different devices, a filter wider than 8 taps, or a head width that
            is not a power of two in 8..512; carried key inputs without ``active`` or unlike ``z``.
    """
    _check(z, history, taps, heads)  # the contract first, before autograd records anything
    if carried_z is not None:
        _check_carried(z, active, carried_z)
        if not (torch.is_grad_enabled() and any(t.requires_grad for t in (z, history, taps, carried_z))):
            return _key_step(z, history, taps, heads, active, carried_z, want_history=False)[0]
        assert active is not None
        z = torch.where(active[..., None], z, carried_z)  # under autograd: the merge, explicit
    out: Tensor = _FusedKeys.apply(z, history, taps, heads)
    return out


class _NormalizeKeys(torch.autograd.Function):
    @staticmethod
    def forward(ctx: Any, k: Tensor) -> Tensor:  # noqa: D102
        x = _aligned(k.detach())
        y = torch.empty_like(x)
        width = x.shape[-1]
        with torch.cuda.device(x.device):
            _lib.call(f"vsp_normalize_keys_{_SUFFIX[x.dtype]}", x.data_ptr(), y.data_ptr(), x.numel() // width,
                      width, _lib.stream_of(x.device))
        ctx.save_for_backward(x)
        return y

    @staticmethod
    def backward(ctx: Any, grad: Tensor) -> Tensor:  # noqa: D102
        (x,) = ctx.saved_tensors
        g = _aligned(grad.to(x.dtype))
        gx = torch.empty_like(x)
        width = x.shape[-1]
        with torch.cuda.device(x.device):
            _lib.call(f"vsp_normalize_keys_backward_{_SUFFIX[x.dtype]}", x.data_ptr(), g.data_ptr(), gx.data_ptr(),
                      x.numel() // width, width, _lib.stream_of(x.device))
        return gx


def normalize_keys(k: Tensor) -> Tensor:
    """``k / max(||k||_2, 1e-6)`` per row of ``k [..., dk]`` on the GPU, at any width
    (``vesper/recurrence.py:91-115``): the row divided by its peak magnitude (floored at 1e-6, held
    constant under autograd), then by the scaled row's norm floored at one, in float32, returned in
    ``k``'s dtype (float32, bfloat16 or float16). An empty ``k`` comes back as it is.

    Raises:
        ContractError: on a tensor off the GPU, a dtype outside float32/bfloat16/float16, or a
            zero-dimensional tensor.
    """
    if k.dim() == 0:
        raise ContractError("normalize_keys needs at least one dimension (the key features)")
    if k.dtype not in FUSED_KEY_DTYPES:
        raise ContractError(f"k: dtype must be float32, bfloat16 or float16, got {k.dtype}")
    if k.device.type != "cuda":
        raise ContractError(f"the key normalization kernel runs on CUDA only, got k on {k.device}")
    if k.shape[-1] >= 2**31:
        raise ContractError(f"rows of {k.shape[-1]} features exceed the kernel's int32 width")
    if k.numel() == 0:
        return k
    out: Tensor = _NormalizeKeys.apply(k)
    return out
