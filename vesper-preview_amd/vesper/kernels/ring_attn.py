"""Decoding attention over a fixed-capacity KV ring on MI355X (HIP kernels through the C ABI).

``RingKVCache`` and ``kv_ring_empty`` mirror the reference's ``vesper/attention.py:62-101``: keys and
values ``[b, window, hkv, dk]``, positions ``[b, window]`` int64 and ``valid [b, window]`` bool; a
token at position ``p`` lives in slot ``p % window``, unwritten slots hold zeros and ``valid``
False. ``ring_attention`` is the attention core of ``WindowedAttention.attend_ring``
(``vesper/attention.py:298-338``) followed by ``kv_ring_write`` (``:104-139``): the query at
position ``p`` attends the valid slots with positions in ``(p - window, p]`` and the new token,
which is attended once from its argument and then written into its slot. Visibility is decided by
positions and ``valid``, never by slot order.

The kernel updates the ring in place (``inplace=True``, what a captured decoder wants); by default
the ring is copied first and the copy returned, which is the reference's functional contract.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch
from torch import Tensor

from vesper.contracts import ContractError, Dims, check_shape, require
from vesper.kernels import _lib

MAX_HEAD_DIM = 256  # head widths: multiples of 8 (16-byte rows) up to this
MAX_GROUP = 8


def _aligned(t: Tensor) -> Tensor:
    t = t.contiguous()
    return t if t.data_ptr() % 16 == 0 else t.clone()


@dataclass(frozen=True)
class RingKVCache:
    """A decoding window of ``window`` slots; slot order is not age order."""

    k: Tensor
    v: Tensor
    pos: Tensor
    valid: Tensor
    window: int


def kv_ring_empty(b: int, hkv: int, dk: int, window: int, dtype: torch.dtype, device: torch.device) -> RingKVCache:
    """Every slot unwritten: zero keys and values, positions 0, ``valid`` False."""
    if window < 1:
        raise ValueError(f"window must be at least 1, got {window}")
    return RingKVCache(
        k=torch.zeros(b, window, hkv, dk, dtype=dtype, device=device),
        v=torch.zeros(b, window, hkv, dk, dtype=dtype, device=device),
        pos=torch.zeros(b, window, dtype=torch.long, device=device),
        valid=torch.zeros(b, window, dtype=torch.bool, device=device),
        window=window,
    )


def ring_attention(q: Tensor, k: Tensor, v: Tensor, pos: Tensor, cache: RingKVCache, *, active: Tensor | None = None,
                   inplace: bool = False, check_positions: bool = True,
                   workspace: Tensor | None = None) -> tuple[Tensor, RingKVCache]:
    """One new token per row over the ring and itself; then the token is written into its slot.

    Args:
        q: ``[b, 1, h, dk]`` rotated queries, bfloat16 or float16.
        k, v: ``[b, 1, hkv, dk]`` the new token's rotated key and value, q's dtype.
        pos: ``[b, 1]`` int64 nonnegative positions.
        cache: the ring, its keys and values in q's dtype or in float32 (the reference decoder's
            allocation; each element is then rounded to q's dtype as it is read, and the new token
            is written widened to float32).
        active: optional bool ``[b]``; an inactive row's output is zero, its token is still written.
        inplace: write into ``cache``'s tensors instead of a copy.
        check_positions: hold ``pos >= 0`` with ``require`` (a device assert under graph capture).
        workspace: optional int32 tensor of at least ``b`` zeros on q's device, the per-row arrival
            counters of the in-kernel write; every call leaves it zero, so a decoder can keep one
            (calls that overlap in time must not share it). By default a fresh one is made.

    Returns:
        ``(o [b, 1, h, dk], ring)`` with the ring that holds the new tokens.
    """
    dims: Dims = {"one": 1, "w": cache.window}
    check_shape("q", q, ("b", "one", "h", "dk"), dims)
    check_shape("k", k, ("b", "one", "hkv", "dk"), dims)
    check_shape("v", v, ("b", "one", "hkv", "dk"), dims)
    check_shape("pos", pos, ("b", "one"), dims, torch.long)
    check_shape("cache.k", cache.k, ("b", "w", "hkv", "dk"), dims)
    check_shape("cache.v", cache.v, ("b", "w", "hkv", "dk"), dims)
    check_shape("cache.pos", cache.pos, ("b", "w"), dims, torch.long)
    check_shape("cache.valid", cache.valid, ("b", "w"), dims, torch.bool)
    if q.dtype not in (torch.bfloat16, torch.float16):
        raise ContractError(f"q: dtype must be bfloat16 or float16, got {q.dtype}")
    for name, t in (("k", k), ("v", v)):
        if t.dtype != q.dtype:
            raise ContractError(f"{name}: dtype must be {q.dtype}, got {t.dtype}")
    # the ring in q's dtype, or in float32 as the reference's decoder allocates it (decode.py:81,85;
    # column.py:492): then each element is rounded to q's dtype as it is read (attention.py:325)
    ring_dtype = cache.k.dtype
    if ring_dtype not in (q.dtype, torch.float32) or cache.v.dtype != ring_dtype:
        raise ContractError(f"cache.k, cache.v: dtype must be {q.dtype} or torch.float32 (both alike), got "
                            f"{cache.k.dtype} and {cache.v.dtype}")
    if q.device.type != "cuda":
        raise ContractError(f"the ring attention kernel runs on CUDA only, got q on {q.device}")
    for name, t in (("k", k), ("v", v), ("pos", pos), ("cache.k", cache.k), ("cache.v", cache.v),
                    ("cache.pos", cache.pos), ("cache.valid", cache.valid)):
        if t.device != q.device:
            raise ContractError(f"{name} is on {t.device}, q on {q.device}")
    b, _, h, dk = q.shape
    hkv = dims["hkv"]
    if h % hkv != 0 or h // hkv > MAX_GROUP:
        raise ContractError(f"{h} query heads over {hkv} KV heads: need a multiple, at most {MAX_GROUP} per KV head")
    if dk % 8 != 0 or not 8 <= dk <= MAX_HEAD_DIM:
        raise ContractError(f"head dimension {dk}: the kernel takes multiples of 8 up to {MAX_HEAD_DIM}")
    if torch.is_grad_enabled() and any(t.requires_grad for t in (q, k, v)):
        raise ContractError("the HIP ring attention is forward only: call it under torch.no_grad()")
    if check_positions and b > 0:
        require((pos >= 0).all().reshape(1), "ring_attention: positions must be nonnegative")
    mask = None
    if active is not None:
        check_shape("active", active, ("b",), dims, torch.bool)
        mask = active.contiguous().view(torch.uint8)
    ring = cache
    if not inplace:
        ring = RingKVCache(cache.k.clone(), cache.v.clone(), cache.pos.clone(), cache.valid.clone(), cache.window)
    for name, t in (("k", ring.k), ("v", ring.v), ("pos", ring.pos), ("valid", ring.valid)):
        if not t.is_contiguous():
            raise ContractError(f"cache.{name} must be contiguous for an in-place ring")
    q, k, v, pos = (_aligned(t) for t in (q, k, v, pos))
    for name, t in (("k", ring.k), ("v", ring.v)):
        if t.data_ptr() % 16 != 0:
            raise ContractError(f"cache.{name} must be 16-byte aligned for an in-place ring")
    o = torch.empty_like(q)
    # per-row arrival counters of the in-kernel write: zero before, and the kernel leaves them zero
    if workspace is None:
        counters = torch.zeros(max(b, 1), dtype=torch.int32, device=q.device)
    else:
        counters = workspace
        if counters.dtype != torch.int32 or counters.device != q.device or not counters.is_contiguous():
            raise ContractError("workspace must be a contiguous int32 tensor on q's device")
        if counters.numel() < b:
            raise ContractError(f"workspace holds {counters.numel()} counters, {b} rows need {b}")
    entry = "vsp_ring_attn_bf16" if q.dtype == torch.bfloat16 else "vsp_ring_attn_f16"
    if ring_dtype == torch.float32:
        entry += "_ring_f32"
    with torch.cuda.device(q.device):
        _lib.call(entry, q.data_ptr(), k.data_ptr(), v.data_ptr(), pos.data_ptr(), ring.k.data_ptr(),
                  ring.v.data_ptr(), ring.pos.data_ptr(), ring.valid.data_ptr(), o.data_ptr(), _lib.ptr(mask),
                  counters.data_ptr(), counters.numel() * 4, b, h, hkv, dk, cache.window, 1.0 / math.sqrt(dk), 1,
                  _lib.stream_of(q.device))
    return o, ring
