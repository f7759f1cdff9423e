"""Boundary checks for the mixer entry points: shapes, dtypes and device-side value contracts.

The interface and the error texts match the reference's ``vesper/contracts.py:31-131``
(``ContractError`` is a ``ValueError``; messages name the tensor, the axis and both values; a
dtype mismatch says "dtype"), so callers and tests written against the reference keep working.
"""

from __future__ import annotations

import torch

Dims = dict[str, int]
DimSpec = tuple


class ContractError(ValueError):
    """A tensor did not meet its contract (rank, dimension binding, dtype or device)."""


def check_shape(name: str, tensor: torch.Tensor, spec: DimSpec, dims: Dims, dtype: torch.dtype | None = None) -> None:
    """Check rank, named dimensions (bound on first sight) and, if given, the exact dtype.

    Raises:
        ContractError: on a rank, dimension or dtype mismatch.
    """
    shape = tuple(tensor.shape)
    if len(shape) != len(spec):
        raise ContractError(f"{name}: expected rank {len(spec)} {spec}, got shape {shape}")
    for axis, (want, got) in enumerate(zip(spec, shape)):
        if isinstance(want, int):
            if got != want:
                raise ContractError(f"{name}: axis {axis} must be {want}, got {got} (shape {shape})")
            continue
        bound = dims.get(want)
        if bound is None:
            dims[want] = got
        elif bound != got:
            raise ContractError(f"{name}: axis {axis} '{want}' is {got}, but '{want}' = {bound} elsewhere")
    if dtype is not None and tensor.dtype != dtype:
        raise ContractError(f"{name}: dtype must be {dtype}, got {tensor.dtype}")


def require(condition: torch.Tensor, message: str) -> None:
    """A value contract on device data: ``ContractError`` eagerly, a device assert under capture.

    ``condition`` is a one-element bool tensor. While the current stream is capturing a graph a
    read-back would end the capture, so the check is recorded as an asynchronous device assert.
    """
    if condition.dtype != torch.bool or condition.numel() != 1:
        raise ContractError(f"require: the condition must be one bool, got {condition.dtype} {tuple(condition.shape)}")
    if condition.is_cuda and torch.cuda.is_current_stream_capturing():
        torch._assert_async(condition, message)  # noqa: SLF001
        return
    if not bool(condition.item()):
        raise ContractError(message)
