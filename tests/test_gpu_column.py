"""The scan switch (``vesper.column``) on the GPU: each choice runs its HIP kernel, bit for bit, and a
recurrent sublayer switched between the reference scan and the HIP scans agrees at their bounds."""

from __future__ import annotations

import pytest
import torch

from conftest import needs_gpu, scan_inputs
from oracle.delta import relative_error

pytestmark = [pytest.mark.gpu, needs_gpu]

GPU = torch.device("cuda")


def test_each_choice_runs_its_kernel_on_cast_inputs():
    from vesper.column import check_capturable_scan, check_scan, recurrent_scan
    from vesper.kernels.delta_scan import delta_scan_fused, delta_scan_fused_fp32

    assert check_scan("fused", GPU) == "fused" and check_capturable_scan("fused-fp32", GPU) == "fused-fp32"
    q, k, v, beta, h0 = (t.to(GPU) for t in scan_inputs(2, 150, 3, 64, seed=2))
    o, s = recurrent_scan("fused", q, k, v, beta, h0.double())
    o_ref, s_ref = delta_scan_fused(*(t.to(torch.bfloat16) for t in (q, k, v, beta)), h0)
    assert o.dtype == torch.float32 and s.dtype == torch.float32
    assert torch.equal(o, o_ref.float()) and torch.equal(s, s_ref)
    o, s = recurrent_scan("fused-fp32", q.to(torch.bfloat16), k.to(torch.bfloat16), v.to(torch.bfloat16),
                          beta.to(torch.bfloat16), h0)
    o_ref, s_ref = delta_scan_fused_fp32(*(t.to(torch.bfloat16).float() for t in (q, k, v, beta)), h0)
    assert o.dtype == torch.bfloat16 and torch.equal(o, o_ref.to(torch.bfloat16)) and torch.equal(s, s_ref)


def test_autocast_does_not_reach_the_kernel():
    from vesper.column import recurrent_scan

    q, k, v, beta, h0 = (t.to(GPU) for t in scan_inputs(1, 70, 2, 64, seed=3))
    eager = recurrent_scan("fused-fp32", q, k, v, beta, h0)
    with torch.autocast(device_type="cuda", dtype=torch.bfloat16):
        under = recurrent_scan("fused-fp32", q, k, v, beta, h0)
    assert torch.equal(eager[0], under[0]) and torch.equal(eager[1], under[1])


def test_a_recurrent_sublayer_switches_between_the_reference_and_the_hip_scans():
    # set_scan (column.py:353-380) on a module: the same sublayer, the same inputs, each backend;
    # the HIP scans against the reference scan at the reference's bounds (1e-5 fp32, 1.5e-2 bf16)
    from vesper.column import RecurrentSublayer, scan_of, set_scan

    g = torch.Generator().manual_seed(3)
    layer = RecurrentSublayer(128, 2, key_conv=4, generator=g).to(GPU)
    x = torch.randn(2, 150, 128, generator=g).to(GPU)
    s0 = (0.1 * torch.randn(2, 2, 64, 64, generator=g)).to(GPU)
    hist = torch.randn(2, 3, 128, generator=g).to(GPU)
    out = {}
    with torch.no_grad():
        for impl in ("reference", "fused-fp32", "fused"):
            assert set_scan(layer, impl) == 1 and scan_of(layer) == impl
            out[impl] = layer(x, s0, hist)
    y_ref, s_ref, h_ref = out["reference"]
    for impl, bound in (("fused-fp32", 1e-5), ("fused", 1.5e-2)):
        y, s, h = out[impl]
        assert relative_error(y, y_ref) < bound, impl
        assert relative_error(s, s_ref) < bound, impl
        assert torch.equal(h, h_ref)
