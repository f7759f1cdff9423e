"""The looped column's copy-forward bookkeeping on MI355X: flagged token rows copied in place.

``copy_rows_where(items)`` performs, for each ``(src, dst, flags)``, ``dst[flags] = src[flags]``
over the leading ``[b, n]`` token dimensions, every item in one kernel launch
(``vsp_copy_rows_where``). It stands in for the row-wise ``where`` selects of the reference's
pass loop: the freezing of the projections of the tokens that halt now into the carried ones
(``vesper/loop.py:523-537``, ``_merge``) and the carried hidden state of halted tokens
(``vesper/loop.py:441-452``). Only flagged rows are read and written.
"""

from __future__ import annotations

import ctypes
from collections.abc import Sequence

import torch
from torch import Tensor

from vesper.contracts import ContractError
from vesper.kernels import _lib

MAX_ITEMS = 8  # tensors per launch


def copy_rows_where(items: Sequence[tuple[Tensor, Tensor, Tensor]]) -> None:
    """``dst[flags] = src[flags]`` in place for each ``(src, dst, flags)``, one launch for all.

    Args:
        items: up to eight triples on one GPU: ``src`` and ``dst`` of one shape and dtype with
            leading dimensions ``[b, n]`` (``dst`` contiguous: it is written in place), ``flags``
            bool ``[b, n]``; every item has the same ``b * n``.

    Raises:
        ContractError: on more than eight items, shapes, dtypes or devices that disagree, or a
            ``dst`` that is not contiguous.
    """
    if len(items) > MAX_ITEMS:
        raise ContractError(f"{len(items)} tensors: at most {MAX_ITEMS} per launch")
    if not items:
        return
    device = items[0][1].device
    rows = None
    srcs, dsts, flags, sizes = [], [], [], []
    for i, (src, dst, flag) in enumerate(items):
        if src.shape != dst.shape or src.dtype != dst.dtype:
            raise ContractError(f"item {i}: src {tuple(src.shape)} {src.dtype}, dst {tuple(dst.shape)} {dst.dtype}")
        if flag.dtype != torch.bool or flag.dim() != 2 or tuple(dst.shape[:2]) != tuple(flag.shape):
            raise ContractError(f"item {i}: flags must be bool {tuple(dst.shape[:2])}, got {tuple(flag.shape)} {flag.dtype}")
        if any(t.device != device for t in (src, dst, flag)) or device.type != "cuda":
            raise ContractError(f"item {i}: every tensor must be on one GPU ({device})")
        if not dst.is_contiguous():
            raise ContractError(f"item {i}: dst must be contiguous (it is written in place)")
        n_rows = flag.numel()
        if rows is None:
            rows = n_rows
        elif rows != n_rows:
            raise ContractError(f"item {i}: {n_rows} token rows, the first item has {rows}")
        src_c, flag_c = src.contiguous(), flag.contiguous()
        srcs.append(src_c)
        dsts.append(dst)
        flags.append(flag_c)
        sizes.append(dst.numel() * dst.element_size() // max(n_rows, 1))
    count = len(items)
    src_arr = (ctypes.c_void_p * count)(*[t.data_ptr() for t in srcs])
    dst_arr = (ctypes.c_void_p * count)(*[t.data_ptr() for t in dsts])
    flag_arr = (ctypes.c_void_p * count)(*[t.data_ptr() for t in flags])
    size_arr = (ctypes.c_size_t * count)(*sizes)
    with torch.cuda.device(device):
        _lib.call("vsp_copy_rows_where", count, ctypes.cast(src_arr, ctypes.c_void_p),
                  ctypes.cast(dst_arr, ctypes.c_void_p), ctypes.cast(size_arr, ctypes.c_void_p),
                  ctypes.cast(flag_arr, ctypes.c_void_p), int(rows or 0), _lib.stream_of(device))


def halt_step(active: Tensor, exits: Tensor | None, n_iters: Tensor) -> tuple[Tensor, Tensor]:
    """One pass's halting bookkeeping in one launch (``vsp_halt_step``): ``halts = active & exits``
    (every active token when ``exits`` is None, the last pass), ``n_iters += active`` in place, and
    the next pass's ``active & ~halts``; returns ``(halts, next_active)``.

    Args:
        active: bool ``[b, n]``; exits: bool ``[b, n]`` or None; n_iters: contiguous int32 ``[b, n]``.

    Raises:
        ContractError: on shapes, dtypes or devices that disagree.
    """
    shape = tuple(active.shape)
    if active.dtype != torch.bool or active.device.type != "cuda":
        raise ContractError(f"active: bool on CUDA, got {active.dtype} on {active.device}")
    if exits is not None and (tuple(exits.shape) != shape or exits.dtype != torch.bool or exits.device != active.device):
        raise ContractError(f"exits: bool {shape} on {active.device}")
    if (tuple(n_iters.shape) != shape or n_iters.dtype != torch.int32 or n_iters.device != active.device
            or not n_iters.is_contiguous()):
        raise ContractError(f"n_iters: contiguous int32 {shape} on {active.device}")
    a = active.contiguous()
    e = None if exits is None else exits.contiguous()
    halts = torch.empty_like(a)
    nxt = torch.empty_like(a)
    with torch.cuda.device(active.device):
        _lib.call("vsp_halt_step", a.data_ptr(), _lib.ptr(e), n_iters.data_ptr(), halts.data_ptr(), nxt.data_ptr(),
                  a.numel(), _lib.stream_of(active.device))
    return halts, nxt


def residual_rows_where(x1: Tensor, a: Tensor, x: Tensor, flags: Tensor | None) -> None:
    """``x[r] = x1[r] + a[r]`` in place for the token rows with ``flags[r]`` set (every row when
    ``flags`` is None), one launch (``vsp_residual_rows_where``): the residual add after a pass's
    attention written straight into the loop's hidden state, only for the tokens still in the
    loop (``vesper/loop.py:452``).

    Args:
        x1: float32 ``[b, n, d]``; a: bfloat16 ``[b, n, d]`` (added in float32); x: contiguous
            float32 ``[b, n, d]``, written in place (not ``x1``); flags: bool ``[b, n]`` or None.

    Raises:
        ContractError: on shapes, dtypes or devices that disagree.
    """
    if x1.dim() != 3 or x1.dtype != torch.float32 or x1.device.type != "cuda":
        raise ContractError(f"x1: float32 [b, n, d] on CUDA, got {tuple(x1.shape)} {x1.dtype} on {x1.device}")
    if a.shape != x1.shape or a.dtype != torch.bfloat16 or a.device != x1.device:
        raise ContractError(f"a: bf16 {tuple(x1.shape)}, got {tuple(a.shape)} {a.dtype}")
    if x.shape != x1.shape or x.dtype != torch.float32 or x.device != x1.device or not x.is_contiguous():
        raise ContractError(f"x: contiguous float32 {tuple(x1.shape)} on {x1.device}")
    if x.data_ptr() == x1.data_ptr():
        raise ContractError("x must not be x1")
    if flags is not None and (tuple(flags.shape) != tuple(x1.shape[:2]) or flags.dtype != torch.bool
                              or flags.device != x1.device):
        raise ContractError(f"flags: bool {tuple(x1.shape[:2])} on {x1.device}")
    x1c, ac = x1.contiguous(), a.contiguous()
    for name, t in (("x1", x1c), ("a", ac), ("x", x)):
        if t.data_ptr() % 16:
            raise ContractError(f"{name} must be 16-byte aligned")
    fl = None if flags is None else flags.contiguous().view(torch.uint8)
    b, n, d = x1.shape
    with torch.cuda.device(x1.device):
        _lib.call("vsp_residual_rows_where", x1c.data_ptr(), ac.data_ptr(), x.data_ptr(), _lib.ptr(fl), b * n, d,
                  _lib.stream_of(x1.device))
