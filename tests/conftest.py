"""Shared test setup: import paths, the ``gpu`` marker, and seeded input builders.

``-m "not gpu"`` runs on any machine: the oracle against the reference's known answers, the host
logic and the boundary's refusals, and that the C-ABI library loads and exports its symbols.
``-m gpu`` runs the parity tests proper on a GPU through the C ABI; each one skips (never falls
back) when no GPU is present.
"""

from __future__ import annotations

import json
import os
import sys
from fractions import Fraction
from pathlib import Path

import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]
PACKAGE_ROOT = ROOT / "vesper-preview_amd"
for p in (str(ROOT), str(PACKAGE_ROOT)):
    if p not in sys.path:
        sys.path.insert(0, p)

GOLDEN = ROOT / "tests" / "golden"

# the CPU oracle is float64 and small; keep the container's cores for it
torch.set_num_threads(max(1, min(16, os.cpu_count() or 1)))


def pytest_configure(config: pytest.Config) -> None:
    config.addinivalue_line("markers", "gpu: needs a HIP device (MI355X); runs the kernels through the C ABI")


def has_gpu() -> bool:
    return torch.cuda.is_available()


needs_gpu = pytest.mark.skipif(not has_gpu(), reason="needs a HIP device")


def reference_vectors() -> dict:
    with open(GOLDEN / "reference_vectors.json", encoding="utf-8") as f:
        return json.load(f)


def frac_tensor(values, dtype: torch.dtype = torch.float64) -> torch.Tensor:
    """Nested lists of ``'p/q'`` strings as a tensor."""

    def conv(x):
        if isinstance(x, list):
            return [conv(y) for y in x]
        return float(Fraction(x)) if "e" not in str(x) else float(x)

    return torch.tensor(conv(values), dtype=dtype)


def scan_inputs(b: int, n: int, h: int, dk: int, seed: int = 0, state_scale: float = 0.5):
    """Seeded scan inputs on the CPU in float32: q, k (L2-normalised), v, beta, h0.

    Draw order q, k, v, beta logits, h0 from one generator (``tests/test_delta_scan_fused.py:47-62``).
    """
    from oracle.delta import normalize_keys, write_strength

    g = torch.Generator().manual_seed(seed)
    q = torch.randn(b, n, h, dk, generator=g)
    k = normalize_keys(torch.randn(b, n, h, dk, generator=g))
    v = torch.randn(b, n, h, dk, generator=g)
    beta = write_strength(torch.randn(b, n, h, generator=g))
    h0 = state_scale * torch.randn(b, h, dk, dk, generator=g)
    return q, k, v, beta, h0
