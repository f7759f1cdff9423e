"""The attention sublayer's window across chunks and its rotary embedding, on MI355X.

Mirrors the pieces of the reference's ``vesper/attention.py`` around the window attention kernel:

- ``KVCache`` / ``kv_cache_empty`` / ``kv_cache_push`` (``attention.py:30-59``, ``:142-175``): the
  chronological window a pass carries from one chunk to the next, the newest ``min(m + n, w)``
  entries oldest first; the push is one launch (``vsp_kv_cache_push``).
- ``rotary`` / ``rotary_qk`` (``attention.py:178-217``, applied to q and k in ``project``,
  ``:292``): one launch rotates the queries and keys of a chunk (``vsp_rotary_qk_*``); phases in
  float64, the rotation in the activations' dtype, as the reference computes it. Differentiable:
  the backward is the rotation by the opposite angle (the same kernel at negated positions).
- ``attend`` (``WindowedAttention.attend``, ``attention.py:340-407``, without the output
  projection): the chunk's queries over the cache and the chunk through ``window_attention`` (the
  cache's rows first, ``window_attn.py:36``) in bfloat16 / float16, the reference's blocked eager
  branch for float32; then the pushed cache.
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Any

import torch
from torch import Tensor

from vesper.contracts import ContractError, Dims, check_shape, require
from vesper.kernels import _lib
from vesper.kernels.window_attn import WINDOW_KERNEL_DTYPES, window_attention_cached

_SUFFIX = {torch.bfloat16: "bf16", torch.float16: "f16", torch.float32: "f32"}


@dataclass(frozen=True)
class KVCache:
    """The last ``m <= window`` entries of one attention window, oldest first: keys and values
    ``[b, m, hkv, dk]`` (keys already rotated), positions ``[b, m]`` int64."""

    k: Tensor
    v: Tensor
    pos: Tensor
    window: int


def kv_cache_empty(b: int, hkv: int, dk: int, window: int, dtype: torch.dtype, device: torch.device) -> KVCache:
    """An empty cache (``m = 0``) for ``window`` entries (``attention.py:42-59``).

    Raises:
        ValueError: if ``window`` is below 1.
    """
    if window < 1:
        raise ValueError(f"window must be at least 1, got {window}")
    return KVCache(torch.zeros(b, 0, hkv, dk, dtype=dtype, device=device),
                   torch.zeros(b, 0, hkv, dk, dtype=dtype, device=device),
                   torch.zeros(b, 0, dtype=torch.long, device=device), window)


def kv_cache_push(cache: KVCache, k: Tensor, v: Tensor, pos: Tensor) -> KVCache:
    """Append a chunk's rotated keys, values and positions and keep the last ``window`` entries
    (``attention.py:142-175``): a new cache at exactly ``min(m + n, window)`` entries; the inputs
    are not modified; with no new entries the cache itself is returned. On the GPU one launch
    writes all three (``vsp_kv_cache_push``); under autograd the same selection by concatenation,
    so gradients reach the pushed keys and values.

    Raises:
        ContractError: on shapes or dtypes that disagree.
    """
    dims: Dims = {}
    check_shape("cache.k", cache.k, ("b", "m", "hkv", "dk"), dims)
    check_shape("cache.v", cache.v, ("b", "m", "hkv", "dk"), dims)
    check_shape("cache.pos", cache.pos, ("b", "m"), dims, torch.long)
    check_shape("k", k, ("b", "n", "hkv", "dk"), dims)
    check_shape("v", v, ("b", "n", "hkv", "dk"), dims)
    check_shape("pos", pos, ("b", "n"), dims, torch.long)
    w, m, n = cache.window, dims["m"], dims["n"]
    if n == 0:
        return cache
    keep_new = min(n, w)
    keep_old = min(m, w - keep_new)
    if k.dtype != cache.k.dtype or v.dtype != cache.v.dtype or k.dtype != v.dtype:
        raise ContractError(f"cache and chunk dtypes differ: {cache.k.dtype}, {k.dtype}, {v.dtype}")
    if torch.is_grad_enabled() and any(t.requires_grad for t in (cache.k, cache.v, k, v)):
        return KVCache(torch.cat([cache.k[:, m - keep_old:], k[:, n - keep_new:]], dim=1),
                       torch.cat([cache.v[:, m - keep_old:], v[:, n - keep_new:]], dim=1),
                       torch.cat([cache.pos[:, m - keep_old:], pos[:, n - keep_new:]], dim=1), w)
    if k.device.type != "cuda" or any(t.device != k.device for t in (v, pos, cache.k, cache.v, cache.pos)):
        raise ContractError(f"the cache push runs on CUDA with every tensor on one device, k is on {k.device}")
    if k.element_size() not in (2, 4):
        raise ContractError(f"k: dtype {k.dtype} is not a 16- or 32-bit float")
    b, hkv, dk = dims["b"], dims["hkv"], dims["dk"]
    keep = keep_old + keep_new
    out = KVCache(torch.empty(b, keep, hkv, dk, dtype=k.dtype, device=k.device),
                  torch.empty(b, keep, hkv, dk, dtype=v.dtype, device=k.device),
                  torch.empty(b, keep, dtype=torch.long, device=k.device), w)
    ck, cv, cp, kk, vv, pp = (t.contiguous() for t in (cache.k, cache.v, cache.pos, k, v, pos))
    with torch.cuda.device(k.device):
        _lib.call("vsp_kv_cache_push", ck.data_ptr(), cv.data_ptr(), cp.data_ptr(), kk.data_ptr(), vv.data_ptr(),
                  pp.data_ptr(), out.k.data_ptr(), out.v.data_ptr(), out.pos.data_ptr(), b, m, n, hkv, dk,
                  k.element_size(), w, _lib.stream_of(k.device))
    return out


_INV_FREQ: dict[tuple[float, int, torch.device], Tensor] = {}


def _inv_freq(base: float, dk: int, device: torch.device) -> Tensor:
    """``base^(-2j/dk)`` for ``j < dk/2`` in float64, computed on the host as the reference does
    (``attention.py:211-212``) and kept on the device."""
    key = (float(base), dk, device)
    table = _INV_FREQ.get(key)
    if table is None:
        exponent = torch.arange(0, dk // 2, dtype=torch.float64) * (2.0 / dk)
        table = (base ** (-exponent)).to(device)
        _INV_FREQ[key] = table
    return table


def rotary_inv_freq(base: float, dk: int, device: torch.device) -> Tensor:
    """The float64 table ``base^(-2j/dk)`` the rotary kernels read (``attention.py:211-212``)."""
    return _inv_freq(base, dk, device)


def _check_rotary(x: Tensor, pos: Tensor, base: float, name: str = "x") -> int:
    dims: Dims = {}
    check_shape(name, x, ("b", "n", "heads", "dk"), dims)
    check_shape("pos", pos, ("b", "n"), dims, torch.long)
    dk = dims["dk"]
    if dk % 2 != 0:
        raise ValueError(f"dk must be even for rotary pairs, got {dk}")
    if not 1.0 < base < float("inf"):  # NaN fails too
        raise ValueError(f"rotary base must be finite and above 1, got {base}")
    if x.dtype not in _SUFFIX:
        raise ContractError(f"{name}: dtype must be bfloat16, float16 or float32, got {x.dtype}")
    if x.device.type != "cuda" or pos.device != x.device:
        raise ContractError(f"the rotary kernel runs on CUDA with pos on x's device, {name} is on {x.device}")
    if dk > 1024:
        raise ContractError(f"head dimension {dk} exceeds the rotary kernel's 1024")
    return dk


def _launch_rotary(q: Tensor, k: Tensor | None, pos: Tensor, base: float) -> tuple[Tensor, Tensor | None]:
    b, n, h, dk = q.shape
    hkv = 0 if k is None else k.shape[2]
    qc = q.contiguous()
    kc = None if k is None else k.contiguous()
    qo = torch.empty_like(qc)
    ko = None if kc is None else torch.empty_like(kc)
    pc = pos.contiguous()
    with torch.cuda.device(q.device):
        _lib.call(f"vsp_rotary_qk_{_SUFFIX[q.dtype]}", qc.data_ptr(), _lib.ptr(kc), pc.data_ptr(),
                  _inv_freq(base, dk, q.device).data_ptr(), qo.data_ptr(), _lib.ptr(ko), b, n, h, hkv, dk,
                  _lib.stream_of(q.device))
    return qo, ko


class _Rotary(torch.autograd.Function):
    @staticmethod
    def forward(ctx: Any, q: Tensor, k: Tensor | None, pos: Tensor, base: float) -> tuple[Tensor, Tensor | None]:  # noqa: D102
        ctx.save_for_backward(pos)
        ctx.base = base
        return _launch_rotary(q.detach(), None if k is None else k.detach(), pos, base)

    @staticmethod
    def backward(ctx: Any, gq: Tensor, gk: Tensor | None) -> tuple[Tensor | None, ...]:  # noqa: D102
        (pos,) = ctx.saved_tensors
        dq, dk_ = _launch_rotary(gq, gk, -pos, ctx.base)  # the transpose of a rotation turns back
        return dq, dk_, None, None


def _rotate(q: Tensor, k: Tensor | None, pos: Tensor, base: float) -> tuple[Tensor, Tensor | None]:
    if torch.is_grad_enabled() and (q.requires_grad or (k is not None and k.requires_grad)):
        return _Rotary.apply(q, k, pos, base)
    return _launch_rotary(q, k, pos, base)


def rotary(x: Tensor, pos: Tensor, base: float) -> Tensor:
    """Rotary position embedding of ``x [b, n, heads, dk]`` at int64 positions ``pos [b, n]``
    (``attention.py:178-217``); ``pos = 0`` returns ``x``'s values exactly.

    Raises:
        ContractError: if ``pos`` is not int64 ``[b, n]`` for ``x``, or a dtype or device the kernel
            does not take; ValueError: if ``dk`` is odd or ``base`` is not finite and above 1.
    """
    _check_rotary(x, pos, base)
    if x.numel() == 0:
        return x.clone()
    return _rotate(x, None, pos, base)[0]


def rotary_qk(q: Tensor, k: Tensor, pos: Tensor, base: float) -> tuple[Tensor, Tensor]:
    """``(rotary(q, pos, base), rotary(k, pos, base))`` in one launch: each token's phases are
    computed once for its query and key heads (``WindowedAttention.project``, ``attention.py:292``).

    Raises:
        ContractError / ValueError: as ``rotary``, for either tensor, or dtypes that differ.
    """
    dk = _check_rotary(q, pos, base, "q")
    _check_rotary(k, pos, base, "k")
    if k.dtype != q.dtype or k.shape[-1] != dk:
        raise ContractError(f"k: {k.dtype} [..., {k.shape[-1]}] against q's {q.dtype} [..., {dk}]")
    if q.numel() == 0 or k.numel() == 0:
        return rotary(q, pos, base), rotary(k, pos, base)
    qo, ko = _rotate(q, k, pos, base)
    assert ko is not None
    return qo, ko


def attend(q: Tensor, k: Tensor, v: Tensor, pos: Tensor, cache: KVCache) -> tuple[Tensor, KVCache]:
    """Windowed softmax of a chunk's rotated ``q [b, n, h, dk]`` over the cache and the chunk's
    rotated ``k``, ``v [b, n, hkv, dk]`` at positions ``pos [b, n]``; returns the attention output
    ``[b, n, h, dk]`` (before the output projection) and the pushed cache. The two branches of
    ``WindowedAttention.attend`` (``attention.py:340-407``):

    - bfloat16 / float16 on the GPU (``:373-383``): the cache's ``m`` rows then the chunk's as the
      keys of ``window_attention`` (read from the two tensors in place,
      ``window_attention_cached``, not concatenated first), which places query ``i`` at key index
      ``m + i``; positions must be consecutive across the cache and the chunk.
    - float32 (any other dtype) on the GPU (``:384-407``, the reference's eager branch): blocks of
      ``window`` queries, each over the keys its first query can still see, masked by position
      (``kpos <= qpos < kpos + window``), through torch's ``scaled_dot_product_attention`` with
      the key heads shared by ``h / hkv`` query heads; differentiable.

    Tensors off the GPU are refused (the cache push, like the kernel, runs on CUDA).

    A chunk of zero tokens returns an empty output and the cache unchanged.

    Raises:
        ContractError: on shapes or dtypes that disagree; on the kernel branch, positions that are
            not consecutive across the cache and the chunk (eagerly; a device assert under graph
            capture).
    """
    dims: Dims = {}
    check_shape("q", q, ("b", "n", "h", "dk"), dims)
    check_shape("k", k, ("b", "n", "hkv", "dk"), dims)
    check_shape("v", v, ("b", "n", "hkv", "dk"), dims)
    check_shape("pos", pos, ("b", "n"), dims, torch.long)
    check_shape("cache.k", cache.k, ("b", "m", "hkv", "dk"), dims)
    check_shape("cache.v", cache.v, ("b", "m", "hkv", "dk"), dims)
    check_shape("cache.pos", cache.pos, ("b", "m"), dims, torch.long)
    if dims["n"] == 0:
        return q.new_zeros(q.shape), cache
    if q.is_cuda and q.dtype not in WINDOW_KERNEL_DTYPES:
        return _attend_blocked(q, k, v, pos, cache), kv_cache_push(cache, k, v, pos)
    kpos = torch.cat([cache.pos, pos], dim=1)
    if kpos.shape[1] > 1:
        require((kpos[:, 1:] - kpos[:, :-1] == 1).all().reshape(1), "attend: cache and chunk positions must be consecutive")
    # the cache's rows and the chunk's as two sources of one kernel call (no concatenated copy)
    o = window_attention_cached(q, cache.k.to(q.dtype), cache.v.to(q.dtype), k.to(q.dtype), v.to(q.dtype),
                                cache.window)
    return o, kv_cache_push(cache, k, v, pos)


def _attend_blocked(q: Tensor, k: Tensor, v: Tensor, pos: Tensor, cache: KVCache) -> Tensor:
    """``attend``'s eager branch (``attention.py:384-407``): query block ``[s, s + w)`` attends the
    chunk's keys from ``s - w + 1`` on, plus the cache while ``s < w`` (older entries are out of every
    query's window by then), under the position mask. The keys and values are taken in q's dtype
    (the cache may be wider: an empty float32 cache promotes what is pushed onto it)."""
    n, w = q.shape[1], cache.window
    ck, cv = cache.k.to(q.dtype), cache.v.to(q.dtype)
    kc, vc = k.to(q.dtype), v.to(q.dtype)
    outs: list[Tensor] = []
    for s in range(0, n, w):
        e = min(s + w, n)
        first = max(0, s - w + 1)
        keys, vals, kpos = kc[:, first:e], vc[:, first:e], pos[:, first:e]
        if s < w:
            keys, vals = torch.cat([ck, keys], dim=1), torch.cat([cv, vals], dim=1)
            kpos = torch.cat([cache.pos, kpos], dim=1)
        qpos = pos[:, s:e]
        visible = (kpos[:, None, :] <= qpos[:, :, None]) & (kpos[:, None, :] > qpos[:, :, None] - w)
        block = torch.nn.functional.scaled_dot_product_attention(
            q[:, s:e].transpose(1, 2), keys.transpose(1, 2), vals.transpose(1, 2), attn_mask=visible[:, None],
            enable_gqa=True)
        outs.append(block.transpose(1, 2))
    return torch.cat(outs, dim=1)


def scale_of(dk: int) -> float:
    """The attention scale ``1/sqrt(dk)`` (``window_attn.py:38``)."""
    return 1.0 / math.sqrt(dk)
