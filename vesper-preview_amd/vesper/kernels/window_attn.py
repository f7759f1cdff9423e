"""Sliding-window causal attention on MI355X: a hand-written HIP kernel behind the reference's contract.

``window_attention(q, keys, values, window)`` keeps the signature and semantics of the reference's
``vesper/kernels/window_attn.py:27-39`` (registry row ``docs/registry.md:108``): the outputs of the
``n`` newest positions of ``m + n`` consecutive key positions (the cache's ``m`` first), each query
at index ``i`` attending key indices ``[i - window + 1, i]``, scale ``1 / sqrt(dk)``, query head
``j`` reading KV head ``j // (h / hkv)``. Where the reference calls fla-core's ``parallel_attn`` on
a query tensor padded with ``m`` zero rows, this calls ``vsp_window_attn_bf16`` / ``_f16`` through
the C ABI with the cache offset as an argument, so nothing is padded.

For: bfloat16 or float16 on the GPU with consecutive positions (the window counts indices, as the
reference's kernel does; ``WindowedAttention.attend`` checks the positions before calling).
An optional keyword ``active`` (bool ``[b, n]``) skips inactive queries, whose outputs are zero;
their keys and values stay visible to every other query. With ``active``, ``carried = (keys,
values)`` (``[b, n, hkv, dk]``) is the copy-forward of halted tokens (``vesper/column.py:795-796``):
key rows ``m + t`` of an inactive token ``t`` are read from row ``t`` of the carried tensors inside
the kernel's tile loads (``vsp_window_attn_carried_*``), in place of ``where`` merges before the
call. Under autograd the forward also keeps
each query's log-sum-exp and the backward (``vsp_window_attn_backward_*``) gives the gradients of
``q``, ``keys`` and ``values`` (an inactive query passes none), as the reference's kernel does.
"""

from __future__ import annotations

import math
from typing import Any

import torch
from torch import Tensor

from vesper.contracts import ContractError, Dims, check_shape
from vesper.kernels import _lib

WINDOW_KERNEL_DTYPES = (torch.bfloat16, torch.float16)
HEAD_DIMS = (16, 32, 64, 128, 256)


def _aligned(t: Tensor) -> Tensor:
    t = t.contiguous()
    return t if t.data_ptr() % 16 == 0 else t.clone()


class _WindowAttention(torch.autograd.Function):
    @staticmethod
    def forward(ctx: Any, q: Tensor, keys: Tensor, values: Tensor, window: int, mask: Tensor | None,
                scale: float) -> Tensor:  # noqa: D102
        b, n, h, dk = q.shape
        s, hkv = keys.shape[1], keys.shape[2]
        m = s - n
        suffix = "bf16" if q.dtype == torch.bfloat16 else "f16"
        if n == 0:
            ctx.save_for_backward(q, keys, values, q, q.new_empty(0))
            ctx.meta = (window, m, scale)
            return q.new_zeros(q.shape)
        qc, kc, vc = _aligned(q.detach()), _aligned(keys.detach()), _aligned(values.detach())
        o = torch.empty_like(qc)
        args = (b, n, m, h, hkv, dk, int(window), scale, _lib.stream_of(q.device))
        with torch.cuda.device(q.device):
            if any(ctx.needs_input_grad[:3]):
                lse = torch.empty(b, h, n, dtype=torch.float32, device=q.device)
                _lib.call(f"vsp_window_attn_lse_{suffix}", qc.data_ptr(), kc.data_ptr(), vc.data_ptr(), o.data_ptr(),
                          lse.data_ptr(), _lib.ptr(mask), *args)
                ctx.save_for_backward(qc, kc, vc, o, lse)
                ctx.meta = (window, m, scale)
            else:
                _lib.call(f"vsp_window_attn_{suffix}", qc.data_ptr(), kc.data_ptr(), vc.data_ptr(), o.data_ptr(),
                          _lib.ptr(mask), *args)
        return o

    @staticmethod
    def backward(ctx: Any, grad_o: Tensor) -> tuple[Tensor | None, ...]:  # noqa: D102
        qc, kc, vc, o, lse = ctx.saved_tensors
        window, m, scale = ctx.meta
        b, n, h, dk = qc.shape
        hkv = kc.shape[2]
        if n == 0:
            return torch.zeros_like(qc), torch.zeros_like(kc), torch.zeros_like(vc), None, None, None
        go = _aligned(grad_o.to(qc.dtype))
        dq, dk_, dv = torch.empty_like(qc), torch.empty_like(kc), torch.empty_like(vc)
        workspace = torch.empty(b * h * n, dtype=torch.float32, device=qc.device)
        suffix = "bf16" if qc.dtype == torch.bfloat16 else "f16"
        with torch.cuda.device(qc.device):
            _lib.call(f"vsp_window_attn_backward_{suffix}", qc.data_ptr(), kc.data_ptr(), vc.data_ptr(), o.data_ptr(),
                      go.data_ptr(), lse.data_ptr(), workspace.data_ptr(), dq.data_ptr(), dk_.data_ptr(), dv.data_ptr(),
                      b, n, m, h, hkv, dk, int(window), scale, _lib.stream_of(qc.device))
        return (dq if ctx.needs_input_grad[0] else None, dk_ if ctx.needs_input_grad[1] else None,
                dv if ctx.needs_input_grad[2] else None, None, None, None)


def _carried_call(q: Tensor, keys: Tensor, values: Tensor, carried: tuple[Tensor, Tensor], window: int,
                  mask: Tensor, scale: float) -> Tensor:
    b, n, h, dk = q.shape
    s, hkv = keys.shape[1], keys.shape[2]
    qc, kc, vc = _aligned(q), _aligned(keys), _aligned(values)
    kh, vh = _aligned(carried[0]), _aligned(carried[1])
    o = torch.empty_like(qc)
    suffix = "bf16" if q.dtype == torch.bfloat16 else "f16"
    with torch.cuda.device(q.device):
        _lib.call(f"vsp_window_attn_carried_{suffix}", qc.data_ptr(), kc.data_ptr(), vc.data_ptr(), kh.data_ptr(),
                  vh.data_ptr(), o.data_ptr(), mask.data_ptr(), b, n, s - n, h, hkv, dk, int(window), scale,
                  _lib.stream_of(q.device))
    return o


def window_attention(q: Tensor, keys: Tensor, values: Tensor, window: int, *, active: Tensor | None = None,
                     carried: tuple[Tensor, Tensor] | None = None) -> Tensor:
    """Outputs ``[b, n, h, dk]`` of ``q`` over ``keys, values [b, m + n, hkv, dk]``.

    Raises:
        ContractError: on shapes that disagree, a dtype other than bfloat16/float16 (or mixed), a
            tensor off the GPU, ``h`` not a multiple of ``hkv``, a head width the kernel does not
            tile (above 256; narrower widths between the kernels' 16, 32, 64, 128 and 256 run with zero
            features added up to the next one, which change no score and no output), fewer key rows
            than queries, or carried keys and values without ``active`` or not shaped
            ``[b, n, hkv, dk]`` in the dtype of ``keys``.
        ValueError: if ``window`` is below 1.
    """
    if window < 1:
        raise ValueError(f"window must be at least 1, got {window}")
    dims: Dims = {}
    check_shape("q", q, ("b", "n", "h", "dk"), dims)
    check_shape("keys", keys, ("b", "s", "hkv", "dk"), dims)
    check_shape("values", values, ("b", "s", "hkv", "dk"), dims)
    if q.dtype not in WINDOW_KERNEL_DTYPES:
        raise ContractError(f"q: dtype must be bfloat16 or float16, got {q.dtype}")
    for name, t in (("keys", keys), ("values", values)):
        if t.dtype != q.dtype:
            raise ContractError(f"{name}: dtype must be {q.dtype}, got {t.dtype}")
    if q.device.type != "cuda":
        raise ContractError(f"the window attention kernel runs on CUDA only, got q on {q.device}")
    for name, t in (("keys", keys), ("values", values)):
        if t.device != q.device:
            raise ContractError(f"{name} is on {t.device}, q on {q.device}")
    b, n, h, dk = q.shape
    s, hkv = dims["s"], dims["hkv"]
    m = s - n
    if m < 0:
        raise ContractError(f"keys hold {s} positions, fewer than the {n} queries")
    if h % hkv != 0:
        raise ContractError(f"{h} query heads are not a multiple of {hkv} KV heads")
    width = next((w for w in HEAD_DIMS if w >= dk), None)
    if width is None:
        raise ContractError(f"head dimension {dk} exceeds the kernel's {HEAD_DIMS[-1]}")
    mask = None
    if active is not None:
        check_shape("active", active, ("b", "n"), {"b": b, "n": n}, torch.bool)
        if active.device != q.device:
            raise ContractError(f"active is on {active.device}, q on {q.device}")
        mask = active.contiguous().view(torch.uint8)
    if carried is not None:
        if active is None or mask is None:
            raise ContractError("carried keys and values need the active mask that says which tokens read them")
        if len(carried) != 2:
            raise ContractError(f"carried holds keys and values, got {len(carried)} tensors")
        for name, held in zip(("keys", "values"), carried):
            if held.shape != (b, n, hkv, dk) or held.dtype != q.dtype or held.device != q.device:
                raise ContractError(f"carried {name}: {tuple(held.shape)} {held.dtype} on {held.device}, "
                                    f"want {(b, n, hkv, dk)} {q.dtype} on {q.device}")
        if n > 0 and not (torch.is_grad_enabled() and any(t.requires_grad for t in (q, keys, values, *carried))):
            if width != dk:
                pad = (0, width - dk)
                q, keys, values = (torch.nn.functional.pad(t, pad) for t in (q, keys, values))
                carried = (torch.nn.functional.pad(carried[0], pad), torch.nn.functional.pad(carried[1], pad))
                return _carried_call(q, keys, values, carried, window, mask, 1.0 / math.sqrt(dk))[..., :dk].contiguous()
            return _carried_call(q, keys, values, carried, window, mask, 1.0 / math.sqrt(dk))
        # under autograd the merge is explicit, so the gradient reaches the carried tensors
        keep = active.reshape(b, n, 1, 1)
        m = s - n
        keys = torch.cat([keys[:, :m], torch.where(keep, keys[:, m:], carried[0])], dim=1)
        values = torch.cat([values[:, :m], torch.where(keep, values[:, m:], carried[1])], dim=1)
    if width != dk:
        # zero features of q, keys and values add zero to every score and give zero outputs there
        # (the scale stays 1 / sqrt(dk)); the padding's outputs are dropped, its gradients never
        # reach the inputs
        pad = (0, width - dk)
        qp, kp, vp = (torch.nn.functional.pad(t, pad) for t in (q, keys, values))
        padded: Tensor = _WindowAttention.apply(qp, kp, vp, int(window), mask, 1.0 / math.sqrt(dk))
        return padded[..., :dk].contiguous()
    out: Tensor = _WindowAttention.apply(q, keys, values, int(window), mask, 1.0 / math.sqrt(dk))
    return out


def window_attention_cached(q: Tensor, cache_keys: Tensor, cache_values: Tensor, keys: Tensor, values: Tensor,
                            window: int) -> Tensor:
    """``window_attention(q, cat([cache_keys, keys], 1), cat([cache_values, values], 1), window)``
    with the cache's rows ``[b, m, hkv, dk]`` and the chunk's ``[b, n, hkv, dk]`` held apart: the
    kernel (``vsp_window_attn_cached_*``) reads each key row from its own tensor, so neither is
    copied, and the outputs are the concatenated call's bit for bit. Under autograd, and at head
    widths between the kernels', the concatenated call runs (its backward takes one key tensor).

    Raises:
        ContractError / ValueError: as ``window_attention``, for shapes or dtypes that disagree.
    """
    if window < 1:
        raise ValueError(f"window must be at least 1, got {window}")
    dims: Dims = {}
    check_shape("q", q, ("b", "n", "h", "dk"), dims)
    check_shape("cache_keys", cache_keys, ("b", "m", "hkv", "dk"), dims)
    check_shape("cache_values", cache_values, ("b", "m", "hkv", "dk"), dims)
    check_shape("keys", keys, ("b", "n", "hkv", "dk"), dims)
    check_shape("values", values, ("b", "n", "hkv", "dk"), dims)
    b, n, h, dk = q.shape
    m, hkv = dims["m"], dims["hkv"]
    tensors = (q, cache_keys, cache_values, keys, values)
    needs_grad = torch.is_grad_enabled() and any(t.requires_grad for t in tensors)
    plain = (m == 0 or n == 0 or needs_grad or dk not in HEAD_DIMS or h % hkv != 0 or q.dtype not in WINDOW_KERNEL_DTYPES
             or any(t.dtype != q.dtype or t.device != q.device for t in tensors) or q.device.type != "cuda")
    if plain:  # the one-tensor call, which also raises whatever the arguments break
        if m == 0:
            return window_attention(q, keys, values, window)
        return window_attention(q, torch.cat([cache_keys, keys], 1), torch.cat([cache_values, values], 1), window)
    qc, ck, cv, kc, vc = (_aligned(t) for t in tensors)
    o = torch.empty_like(qc)
    suffix = "bf16" if q.dtype == torch.bfloat16 else "f16"
    with torch.cuda.device(q.device):
        _lib.call(f"vsp_window_attn_cached_{suffix}", qc.data_ptr(), ck.data_ptr(), cv.data_ptr(), kc.data_ptr(),
                  vc.data_ptr(), o.data_ptr(), None, b, n, m, h, hkv, dk, int(window), 1.0 / math.sqrt(dk),
                  _lib.stream_of(q.device))
    return o
