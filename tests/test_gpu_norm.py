"""The sublayers' pre-normalization kernel (``vsp_rms_norm_bf16`` via ``vesper.kernels.norm``)
against the oracle's ``RMSNorm`` (``oracle.loop.rms_norm``, ``vesper/column.py:146-188``).

The kernel computes in float32 and rounds once to bf16, so its rows equal the oracle's float64
rows to within one bf16 rounding (relative 2^-8) element-wise; rows at the scale floor, a zero row
and rows near float32's range take the reference's scale-safe path.
"""

from __future__ import annotations

import pytest
import torch

from conftest import needs_gpu
from oracle.loop import rms_norm

pytestmark = [pytest.mark.gpu, needs_gpu]

GPU = torch.device("cuda")


@pytest.mark.parametrize("d", [8, 64, 512, 520, 1024, 2048])
def test_rows_match_the_oracle(d):
    from vesper.kernels.norm import rms_norm_bf16

    g = torch.Generator().manual_seed(d)
    x = torch.randn(5, 7, d, generator=g) * 3
    x[0, 0] = 0.0  # the floor: a zero row stays zero
    x[0, 1] = 1e-7 * torch.randn(d, generator=g)  # under the 1e-3 scale floor
    x[0, 2] = 1e30 * torch.randn(d, generator=g)  # squares would overflow float32 unscaled
    gain = 1 + 0.1 * torch.randn(d, generator=g)
    for gn in (None, gain):
        got = rms_norm_bf16(x.to(GPU), None if gn is None else gn.to(GPU))
        want = rms_norm(x.double())
        if gn is not None:
            want = want * gn.double()
        assert got.dtype == torch.bfloat16 and got.shape == x.shape
        torch.testing.assert_close(got.cpu().double(), want, rtol=2 ** -8, atol=1e-30)
    assert not bool(rms_norm_bf16(x.to(GPU))[0, 0].any())


def test_refusals():
    from vesper.contracts import ContractError
    from vesper.kernels.norm import rms_norm_bf16

    with pytest.raises(ContractError, match="dtype"):
        rms_norm_bf16(torch.zeros(2, 64, device=GPU, dtype=torch.bfloat16))
    with pytest.raises(ContractError, match="multiple of 8"):
        rms_norm_bf16(torch.zeros(2, 60, device=GPU))
    with pytest.raises(ContractError, match="gain"):
        rms_norm_bf16(torch.zeros(2, 64, device=GPU), torch.ones(32, device=GPU))


@pytest.mark.parametrize("d", [8, 64, 512, 1000, 2048])
@pytest.mark.parametrize("with_gain", [False, True])
def test_the_residual_add_inside_the_norm_equals_the_two_launches_bitwise(d, with_gain):
    """vsp_add_rms_norm_bf16: x + r (bf16 r added in float32) normalized in one launch equals the
    add followed by the norm, and the sum it writes equals the add, bit for bit."""
    from vesper.kernels.norm import rms_norm_bf16

    g = torch.Generator().manual_seed(d)
    x = (torch.randn(37, d, generator=g) * torch.logspace(-3, 3, 37)[:, None]).to(GPU)
    r = torch.randn(37, d, generator=g).to(torch.bfloat16).to(GPU)
    gain = (0.5 + torch.rand(d, generator=g)).to(GPU) if with_gain else None
    s = torch.empty_like(x)
    got = rms_norm_bf16(x, gain, residual=r, sum_out=s)
    want_s = x + r.float()
    assert torch.equal(s, want_s)
    assert torch.equal(got, rms_norm_bf16(want_s, gain))
    assert torch.equal(rms_norm_bf16(x, gain, residual=r), got)  # without the sum written
