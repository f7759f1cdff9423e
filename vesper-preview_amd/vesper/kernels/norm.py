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


def rms_norm_bf16(x: Tensor, gain: Tensor | None = None) -> Tensor:
    """``RMSNorm`` over the last axis of float32 ``x [..., d]`` on the GPU, as bfloat16.

    Args:
        x: float32, its last axis ``d`` a multiple of 8 in 8..2048.
        gain: optional float32 ``[d]`` (the norm's weight; ones when omitted).

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
    with torch.cuda.device(x.device):
        _lib.call("vsp_rms_norm_bf16", xc.data_ptr(), _lib.ptr(g), out.data_ptr(), rows, d, _lib.stream_of(x.device))
    return out
