"""The looped column's sublayer pre-normalization on MI355X: ``RMSNorm`` of float32 rows to bf16.

``rms_norm_bf16(x, gain)`` is ``RMSNorm.forward`` (``vesper/column.py:146-188``) on the float32
residual stream, ``x / sqrt(mean(x^2) + 1e-6) * gain`` computed scale-safely as the reference does,
returned in bfloat16 for the bf16 projection GEMMs (``vsp_rms_norm_bf16``, one launch).
"""

from __future__ import annotations

import torch
from torch import Tensor

from vesper.contracts import ContractError
from vesper.kernels import _lib


def rms_norm_bf16(x: Tensor, gain: Tensor | None = None, *, residual: Tensor | None = None,
                  sum_out: Tensor | None = None) -> Tensor:
    """``RMSNorm`` over the last axis of float32 ``x [..., d]`` on the GPU, as bfloat16.

    Args:
        x: float32, its last axis ``d`` a multiple of 8 in 8..2048.
        gain: optional float32 ``[d]`` (the norm's weight; ones when omitted).
        residual: optional bfloat16 tensor shaped like ``x``: the norm is then of ``x + residual``
            (added in float32, the column's residual add), in the same launch
            (``vsp_add_rms_norm_bf16``), bitwise the add followed by the norm.
        sum_out: with ``residual``, an optional contiguous float32 tensor shaped like ``x`` (not
            ``x`` itself) that receives ``x + residual``.

    Raises:
        ContractError: on a dtype, width or device outside that contract.
    """
    if x.dtype != torch.float32:
        raise ContractError(f"x: dtype must be torch.float32, got {x.dtype}")
    if x.device.type != "cuda":
        raise ContractError(f"the norm kernel runs on CUDA only, x is on {x.device}")
    d = x.shape[-1]
    if d < 8 or d > 2048 or d % 8:
        raise ContractError(f"x: last axis {d} is not a multiple of 8 in 8..2048")
    xc = x.contiguous()
    if xc.data_ptr() % 16:
        xc = xc.clone()
    g = None
    if gain is not None:
        if gain.shape != (d,) or gain.dtype != torch.float32 or gain.device != x.device:
            raise ContractError(f"gain: must be float32 [{d}] on {x.device}, got {tuple(gain.shape)} {gain.dtype}")
        g = gain.contiguous()
        if g.data_ptr() % 16:
            g = g.clone()
    out = torch.empty(x.shape, dtype=torch.bfloat16, device=x.device)
    rows = xc.numel() // d
    if residual is None:
        if sum_out is not None:
            raise ContractError("sum_out needs a residual")
        with torch.cuda.device(x.device):
            _lib.call("vsp_rms_norm_bf16", xc.data_ptr(), _lib.ptr(g), out.data_ptr(), rows, d,
                      _lib.stream_of(x.device))
        return out
    if residual.shape != x.shape or residual.dtype != torch.bfloat16 or residual.device != x.device:
        raise ContractError(f"residual: bf16 {tuple(x.shape)} on {x.device}, got {tuple(residual.shape)} "
                            f"{residual.dtype} on {residual.device}")
    rc = residual.contiguous()
    if rc.data_ptr() % 16:
        rc = rc.clone()
    if sum_out is not None:
        if (sum_out.shape != x.shape or sum_out.dtype != torch.float32 or sum_out.device != x.device
                or not sum_out.is_contiguous() or sum_out.data_ptr() % 16):
            raise ContractError(f"sum_out: contiguous, aligned float32 {tuple(x.shape)} on {x.device}")
        if sum_out.data_ptr() == xc.data_ptr():
            raise ContractError("sum_out must not be x")
    with torch.cuda.device(x.device):
        _lib.call("vsp_add_rms_norm_bf16", xc.data_ptr(), rc.data_ptr(), _lib.ptr(sum_out), _lib.ptr(g),
                  out.data_ptr(), rows, d, _lib.stream_of(x.device))
    return out


def decode_projection(x: Tensor, weights_t: Tensor, used: tuple[int, ...], *, residual: Tensor | None = None,
                      sum_out: Tensor | None = None, gain: Tensor | None = None,
                      sigmoid_block: int | None = None,
                      rotary: tuple[Tensor, Tensor, int, tuple[int, ...]] | None = None) -> list[Tensor]:
    """A decode step's sublayer projections in one launch (``vsp_decode_proj_bf16``): the residual
    sum ``s = x + residual`` (written into ``sum_out`` when given), ``z = RMSNorm(s, gain)`` in
    bfloat16 exactly as ``rms_norm_bf16`` computes it, and ``z W_j[:, :used_j]`` for each block of
    the stacked projection weight (``vesper/column.py:192-260``, ``vesper/attention.py:269-292``).

    Args:
        x: float32 ``[M, d]`` (one row a token), ``d`` a multiple of 32 in 32..2048.
        weights_t: bf16 ``[p, cols, d]``: the stacked ``[p, d, cols]`` weight, each block transposed.
        used: the columns kept of each of the ``p`` (1..4) blocks.
        residual: optional bf16 ``[M, d]`` added to ``x`` (the previous mixer's output).
        sum_out: optional float32 ``[M, d]`` that receives ``s`` (not ``x`` itself).
        gain: optional float32 ``[d]`` (the norm's weight; ones when omitted).
        sigmoid_block: the block whose outputs pass through the logistic function (the write strength).
        rotary: ``(positions, inv_freq, dk, blocks)``: the blocks rotated as they are stored, as
            ``rotary_qk`` rotates queries and keys (heads of ``dk`` columns, token ``m`` at
            ``positions[m]`` int64 ``[M]``, ``inv_freq`` the float64 ``[dk / 2]`` table), bitwise
            the separate launch's result.

    Returns:
        one bf16 ``[M, used_j]`` tensor per block.

    Raises:
        ContractError: on shapes, dtypes or devices outside that contract.
    """
    if x.dim() != 2 or x.dtype != torch.float32 or x.device.type != "cuda":
        raise ContractError(f"x: float32 [M, d] on CUDA, got {tuple(x.shape)} {x.dtype} on {x.device}")
    m, d = x.shape
    if weights_t.dim() != 3 or weights_t.dtype != torch.bfloat16 or weights_t.shape[2] != d:
        raise ContractError(f"weights_t: bf16 [p, cols, {d}], got {tuple(weights_t.shape)} {weights_t.dtype}")
    p, cols = weights_t.shape[0], weights_t.shape[1]
    if len(used) != p or not 1 <= p <= 4 or any(not 1 <= u <= cols for u in used):
        raise ContractError(f"used: {p} widths in 1..{cols}, got {tuple(used)}")
    if d % 32 or not 32 <= d <= 2048:
        raise ContractError(f"x: width {d} is not a multiple of 32 in 32..2048")
    tensors = [("weights_t", weights_t)]
    if residual is not None:
        if residual.shape != (m, d) or residual.dtype != torch.bfloat16:
            raise ContractError(f"residual: bf16 [{m}, {d}], got {tuple(residual.shape)} {residual.dtype}")
        tensors.append(("residual", residual))
    if sum_out is not None:
        if sum_out.shape != (m, d) or sum_out.dtype != torch.float32 or not sum_out.is_contiguous():
            raise ContractError(f"sum_out: contiguous float32 [{m}, {d}], got {tuple(sum_out.shape)} {sum_out.dtype}")
        if sum_out.data_ptr() == x.data_ptr():
            raise ContractError("sum_out must not be x")
        tensors.append(("sum_out", sum_out))
    if gain is not None:
        if gain.shape != (d,) or gain.dtype != torch.float32:
            raise ContractError(f"gain: float32 [{d}], got {tuple(gain.shape)} {gain.dtype}")
        tensors.append(("gain", gain))
    for name, t in tensors:
        if t.device != x.device:
            raise ContractError(f"{name} is on {t.device}, x on {x.device}")
    if sigmoid_block is not None and not 0 <= sigmoid_block < p:
        raise ContractError(f"sigmoid_block {sigmoid_block} is not one of the {p} blocks")
    rot_pos, rot_freq, rot_dk, rot_mask = None, None, 0, 0
    if rotary is not None:
        rot_pos, rot_freq, rot_dk, blocks = rotary
        if rot_pos.shape != (m,) or rot_pos.dtype != torch.long or rot_pos.device != x.device:
            raise ContractError(f"rotary positions: int64 [{m}] on {x.device}, got {tuple(rot_pos.shape)} {rot_pos.dtype}")
        if rot_freq.shape != (rot_dk // 2,) or rot_freq.dtype != torch.float64 or rot_freq.device != x.device:
            raise ContractError(f"rotary frequencies: float64 [{rot_dk // 2}] on {x.device}")
        for j in blocks:
            if not 0 <= j < p or used[j] % rot_dk or j == sigmoid_block:
                raise ContractError(f"block {j} cannot be rotated in heads of {rot_dk}")
            rot_mask |= 1 << j
        rot_pos, rot_freq = rot_pos.contiguous(), rot_freq.contiguous()
    xc, wc = x.contiguous(), weights_t.contiguous()
    rc = None if residual is None else residual.contiguous()
    gc = None if gain is None else gain.contiguous()
    for name, t in (("x", xc), ("weights_t", wc), ("residual", rc), ("sum_out", sum_out), ("gain", gc)):
        if t is not None and t.data_ptr() % 16:
            raise ContractError(f"{name} must be 16-byte aligned")
    outs = [torch.empty(m, u, dtype=torch.bfloat16, device=x.device) for u in used]
    ptrs = [o.data_ptr() for o in outs] + [0] * (4 - p)
    widths = list(used) + [1] * (4 - p)
    with torch.cuda.device(x.device):
        _lib.call("vsp_decode_proj_bf16", xc.data_ptr(), _lib.ptr(rc), _lib.ptr(sum_out), _lib.ptr(gc), wc.data_ptr(),
                  p, cols, d, m, *widths, *ptrs, -1 if sigmoid_block is None else sigmoid_block,
                  _lib.ptr(rot_pos), _lib.ptr(rot_freq), rot_mask, rot_dk, _lib.stream_of(x.device))
    return outs


def projection(z: Tensor, weights_t: Tensor, used: tuple[int, ...], *,
               sigmoid_block: int | None = None) -> list[Tensor]:
    """A prefill's sublayer projections in one launch (``vsp_project_bf16``): ``z W_j[:, :used_j]``
    for each block of the stacked projection weight (``vesper/column.py:192-260``,
    ``vesper/attention.py:269-292``), each block computed over the columns it uses only.

    Args:
        z: bf16 ``[M, d]``, the normalized input (one row a token), ``d`` a multiple of 64 in
            64..16384.
        weights_t: bf16 ``[p, cols, d]``: the stacked ``[p, d, cols]`` weight, each block transposed.
        used: the columns kept of each of the ``p`` (1..4) blocks.
        sigmoid_block: the block whose outputs pass through the logistic function (the write
            strength), as ``decode_projection`` stores it.

    Returns:
        one bf16 ``[M, used_j]`` tensor per block.

    Raises:
        ContractError: on shapes, dtypes or devices outside that contract.
    """
    if z.dim() != 2 or z.dtype != torch.bfloat16 or z.device.type != "cuda":
        raise ContractError(f"z: bf16 [M, d] on CUDA, got {tuple(z.shape)} {z.dtype} on {z.device}")
    m, d = z.shape
    if weights_t.dim() != 3 or weights_t.dtype != torch.bfloat16 or weights_t.shape[2] != d:
        raise ContractError(f"weights_t: bf16 [p, cols, {d}], got {tuple(weights_t.shape)} {weights_t.dtype}")
    if weights_t.device != z.device:
        raise ContractError(f"weights_t is on {weights_t.device}, z on {z.device}")
    p, cols = weights_t.shape[0], weights_t.shape[1]
    if len(used) != p or not 1 <= p <= 4 or any(not 1 <= u <= cols for u in used):
        raise ContractError(f"used: {p} widths in 1..{cols}, got {tuple(used)}")
    if d % 64 or not 64 <= d <= 16384:
        raise ContractError(f"z: width {d} is not a multiple of 64 in 64..16384")
    if (m + 256) * d * 2 >= 1 << 32 or (cols + 256) * d * 2 >= 1 << 32:
        raise ContractError(f"z [{m}, {d}] or a weight block of {cols} columns over 4 GiB")
    if sigmoid_block is not None and not 0 <= sigmoid_block < p:
        raise ContractError(f"sigmoid_block {sigmoid_block} is not one of the {p} blocks")
    zc, wc = z.contiguous(), weights_t.contiguous()
    for name, t in (("z", zc), ("weights_t", wc)):
        if t.data_ptr() % 16:
            raise ContractError(f"{name} must be 16-byte aligned")
    outs = [torch.empty(m, u, dtype=torch.bfloat16, device=z.device) for u in used]
    ptrs = [o.data_ptr() for o in outs] + [0] * (4 - p)
    widths = list(used) + [1] * (4 - p)
    with torch.cuda.device(z.device):
        _lib.call("vsp_project_bf16", zc.data_ptr(), wc.data_ptr(), p, cols, d, m, *widths, *ptrs,
                  -1 if sigmoid_block is None else sigmoid_block, _lib.stream_of(z.device))
    return outs
