"""The causal key filter and key normalization on MI355X: a HIP kernel behind the reference's contract.

``fused_keys(z, history, taps, heads)`` keeps the signature and result of the reference's
``vesper/kernels/keys.py:28-32`` (what ``RecurrentSublayer.keys``, ``vesper/column.py:255-289``,
computes for its key): ``u[t] = sum_r taps[r] * z[t - r]`` with the chunk's predecessors from
``history``, then ``normalize_keys`` per head, float32 arithmetic, the key in ``z``'s dtype. Where
the reference runs a Triton kernel, this calls ``vsp_key_filter_{bf16,f16,f32}`` through the C ABI.

For: float32, bfloat16 or float16 key inputs on the GPU, a filter of 1 to 8 taps, head widths that
are powers of two from 8 to 512. Forward only: inputs that need a gradient are refused.
"""

from __future__ import annotations

import torch
from torch import Tensor

from vesper.contracts import ContractError, Dims, check_shape
from vesper.kernels import _lib

FUSED_KEY_DTYPES = (torch.float32, torch.bfloat16, torch.float16)
MAX_TAPS = 8
_ENTRY = {torch.bfloat16: "vsp_key_filter_bf16", torch.float16: "vsp_key_filter_f16", torch.float32: "vsp_key_filter_f32"}


def _aligned(t: Tensor) -> Tensor:
    t = t.contiguous()
    return t if t.data_ptr() % 16 == 0 else t.clone()


def fused_keys(z: Tensor, history: Tensor, taps: Tensor, heads: int) -> Tensor:
    """Normalized keys ``[b, n, heads, d / heads]`` in ``z``'s dtype (``z [b, n, d]`` on the GPU).

    ``history [b, K-1, d]`` holds the ``K - 1`` key inputs before the chunk (oldest first) and
    ``taps [K, d]`` the filter, tap 0 on the current token; both are used in float32.

    Raises:
        ContractError: on shapes that disagree, a dtype outside float32/bfloat16/float16, tensors
            off the GPU or on different devices, a filter wider than 8 taps, a head width that is
            not a power of two in 8..512, or inputs needing a gradient.
    """
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
    if any(t.requires_grad for t in (z, history, taps)):
        raise ContractError("fused_keys is forward only here: an input requires a gradient")
    if not 1 <= width <= MAX_TAPS:
        raise ContractError(f"taps: the kernel takes 1..{MAX_TAPS} taps, got {width}")
    b, n, d = dims["b"], dims["n"], dims["d"]
    if heads < 1 or d % heads != 0:
        raise ContractError(f"{d} features are not a multiple of {heads} heads")
    head_dim = d // heads
    if head_dim < 8 or head_dim > 512 or head_dim & (head_dim - 1):
        raise ContractError(f"head width {head_dim}: the kernel takes powers of two 8..512")
    out = torch.empty(b, n, heads, head_dim, dtype=z.dtype, device=z.device)
    if b == 0 or n == 0:
        return out
    zc = _aligned(z)
    hc = _aligned(history.to(torch.float32))
    tc = _aligned(taps.to(torch.float32))
    _lib.call(_ENTRY[z.dtype], _lib.ptr(zc), _lib.ptr(hc) if width > 1 else None, _lib.ptr(tc), _lib.ptr(out),
              b, n, d, heads, width, _lib.stream_of(z.device))
    return out
