"""Two fresh processes compute bitwise the same outputs and gradients.

Mirrors the reference's cross-process determinism check (tests/test_determinism.py:181): no kernel
of the scan or of the window attention uses atomics or an order that depends on scheduling, so a
second interpreter on the same seeded inputs must reproduce every byte, forward and backward.
"""

from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]

# Runs in a child interpreter: seeded inputs on the CPU, the bf16 scan and the window attention on
# cuda:0 with their gradients, then one SHA-256 over every output's bytes.
CHILD = r"""
import hashlib, sys
import torch
from vesper.kernels.delta_scan import delta_scan_fused
from vesper.kernels.window_attn import window_attention

dev = torch.device("cuda:0")
g = torch.Generator().manual_seed(11)
b, n, h, d = 2, 700, 4, 64
q = torch.randn(b, n, h, d, generator=g)
k = torch.randn(b, n, h, d, generator=g)
q = q / q.norm(dim=-1, keepdim=True)
k = k / k.norm(dim=-1, keepdim=True)
v = torch.randn(b, n, h, d, generator=g)
beta = torch.sigmoid(torch.randn(b, n, h, generator=g))
s0 = 0.02 * torch.randn(b, h, d, d, generator=g)
do = torch.randn(b, n, h, d, generator=g)
ds = torch.randn(b, h, d, d, generator=g)
leaves = [t.to(dev, torch.bfloat16).requires_grad_() for t in (q, k, v, beta)]
s0d = s0.to(dev).requires_grad_()
o, s = delta_scan_fused(*leaves, s0d)
((o.float() * do.to(dev)).sum() + (s * ds.to(dev)).sum()).backward()

qa = torch.randn(b, n, 8, d, generator=g).to(dev, torch.bfloat16).requires_grad_()
ka = torch.randn(b, n, 2, d, generator=g).to(dev, torch.bfloat16).requires_grad_()
va = torch.randn(b, n, 2, d, generator=g).to(dev, torch.bfloat16).requires_grad_()
da = torch.randn(b, n, 8, d, generator=g).to(dev)
a = window_attention(qa, ka, va, 256)
(a.float() * da).sum().backward()
torch.cuda.synchronize()

digest = hashlib.sha256()
for t in [o, s] + [x.grad for x in leaves] + [s0d.grad, a, qa.grad, ka.grad, va.grad]:
    digest.update(t.detach().cpu().contiguous().view(torch.uint8).numpy().tobytes())
print("DIGEST", digest.hexdigest())
"""


def _digest() -> str:
    env = dict(os.environ)
    paths = [str(ROOT), str(ROOT / "vesper-preview_amd")]
    env["PYTHONPATH"] = os.pathsep.join(paths + ([env["PYTHONPATH"]] if env.get("PYTHONPATH") else []))
    print(f"child process: scan + window attention forward and backward (b2 n700)", flush=True)
    proc = subprocess.run([sys.executable, "-c", CHILD], env=env, capture_output=True, text=True, timeout=300)
    assert proc.returncode == 0, proc.stderr[-3000:]
    lines = [line for line in proc.stdout.splitlines() if line.startswith("DIGEST ")]
    assert len(lines) == 1, proc.stdout[-2000:]
    return lines[0].split()[1]


@pytest.mark.gpu
def test_two_fresh_processes_agree_bitwise():
    first = _digest()
    second = _digest()
    assert first == second
