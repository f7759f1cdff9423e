"""The decode step's fused projection (``vsp_decode_proj_bf16``): residual add, RMSNorm and the
stacked projections of a few single-token rows in one launch, through the C ABI.

Parity: the residual sum is the float32 add of the bf16 residual, bitwise; the normalized operand is
``rms_norm_bf16`` of that sum (the norm kernel's own arithmetic, itself pinned against the oracle
in ``test_gpu_norm.py``), so each output column is checked against that operand times the weight
in float64: within one bf16 rounding of the exact product (2^-8 relative, plus the float32
accumulation's share of the row's magnitude). The write strength's block is the logistic of its
bf16-rounded product, within one bf16 rounding of float64's.
"""

from __future__ import annotations

import pytest
import torch

from conftest import needs_gpu

pytestmark = [pytest.mark.gpu, needs_gpu]

GPU = torch.device("cuda")
BF16 = torch.bfloat16


def _check_block(got, z, w, sigmoid=False):
    exact = z.double() @ w.double()  # [M, used]
    if sigmoid:
        exact = torch.sigmoid(exact.to(BF16).double())
    got = got.double()
    scale = (z.double().abs() @ w.double().abs()).clamp_min(1e-30)
    bound = 2.0 ** -8 * exact.abs() + 3e-5 * scale + (2.0 ** -8 if sigmoid else 0.0)
    bad = (got - exact).abs() > bound
    assert not bool(bad.any()), f"{int(bad.sum())} of {bad.numel()} outside, worst {float((got - exact).abs().max())}"


@pytest.mark.parametrize(("m", "d"), [(1, 64), (5, 96), (16, 128), (64, 512), (70, 512), (33, 1024), (17, 2048)])
@pytest.mark.parametrize("residual", [False, True])
def test_fused_projection_matches_norm_then_product(m, d, residual):
    from vesper.kernels.norm import decode_projection, rms_norm_bf16

    g = torch.Generator().manual_seed(m * 7 + d)
    cols = 256 if d <= 128 else 512
    used = (cols, cols // 2, 40, 8)
    x = (3.0 * torch.randn(m, d, generator=g)).to(GPU)
    r = torch.randn(m, d, generator=g).to(BF16).to(GPU) if residual else None
    w = (torch.randn(4, d, cols, generator=g) / d ** 0.5).to(BF16).to(GPU)
    wt = w.transpose(1, 2).contiguous()
    s = torch.empty(m, d, device=GPU)
    outs = decode_projection(x, wt, used, residual=r, sum_out=s if residual else None, sigmoid_block=3)
    torch.cuda.synchronize()
    want_s = x + r.float() if residual else x
    if residual:
        assert torch.equal(s, want_s)
    z = rms_norm_bf16(want_s)
    for j, (o, u) in enumerate(zip(outs, used)):
        assert o.shape == (m, u) and o.dtype == BF16 and o.is_contiguous()
        _check_block(o, z, w[j, :, :u], sigmoid=j == 3)


def test_a_gain_scales_the_normalized_operand():
    from vesper.kernels.norm import decode_projection, rms_norm_bf16

    g = torch.Generator().manual_seed(11)
    m, d, cols = 24, 256, 128
    x = torch.randn(m, d, generator=g).to(GPU)
    gain = (0.5 + torch.rand(d, generator=g)).to(GPU)
    w = (torch.randn(2, d, cols, generator=g) / d ** 0.5).to(BF16).to(GPU)
    outs = decode_projection(x, w.transpose(1, 2).contiguous(), (cols, 96), gain=gain)
    z = rms_norm_bf16(x, gain)
    _check_block(outs[0], z, w[0])
    _check_block(outs[1], z, w[1, :, :96])


def test_a_mistaken_operand_is_caught():
    # the same bound fails for the product with the weight's blocks swapped: the check is tight
    from vesper.kernels.norm import decode_projection, rms_norm_bf16

    g = torch.Generator().manual_seed(12)
    m, d, cols = 16, 128, 64
    x = torch.randn(m, d, generator=g).to(GPU)
    w = (torch.randn(2, d, cols, generator=g) / d ** 0.5).to(BF16).to(GPU)
    outs = decode_projection(x, w.transpose(1, 2).contiguous(), (cols, cols))
    z = rms_norm_bf16(x)
    with pytest.raises(AssertionError):
        _check_block(outs[0], z, w[1])


def test_refusals():
    from vesper.contracts import ContractError
    from vesper.kernels.norm import decode_projection

    x = torch.zeros(4, 64, device=GPU)
    wt = torch.zeros(2, 32, 64, dtype=BF16, device=GPU)
    with pytest.raises(ContractError, match="multiple of 32"):
        decode_projection(torch.zeros(4, 48, device=GPU), torch.zeros(2, 32, 48, dtype=BF16, device=GPU), (32, 32))
    with pytest.raises(ContractError, match="widths"):
        decode_projection(x, wt, (32, 33))
    with pytest.raises(ContractError, match="must not be x"):
        decode_projection(x, wt, (32, 32), residual=torch.zeros(4, 64, dtype=BF16, device=GPU), sum_out=x)


@pytest.mark.parametrize(("m", "h", "hkv", "dk"), [(64, 8, 8, 64), (5, 4, 2, 32), (17, 2, 1, 128)])
def test_rotation_as_stored_equals_the_rotary_launch_bitwise(m, h, hkv, dk):
    """q and k rotated by the projection's stores equal the projection then rotary_qk, bit for bit
    (the rotary kernel is pinned against the reference's scalar-trig pairs)."""
    from vesper.attention import rotary_inv_freq, rotary_qk
    from vesper.kernels.norm import decode_projection

    g = torch.Generator().manual_seed(m + dk)
    d, cols = 256, h * dk
    x = torch.randn(m, d, generator=g).to(GPU)
    w = (torch.randn(3, d, cols, generator=g) / d ** 0.5).to(BF16).to(GPU)
    wt = w.transpose(1, 2).contiguous()
    used = (h * dk, hkv * dk, hkv * dk)
    pos = torch.randint(0, 100_000, (m,), generator=g).to(GPU)
    plain = decode_projection(x, wt, used)
    rot = decode_projection(x, wt, used, rotary=(pos, rotary_inv_freq(10000.0, dk, GPU), dk, (0, 1)))
    want_q, want_k = rotary_qk(plain[0].view(m, 1, h, dk), plain[1].view(m, 1, hkv, dk), pos.view(m, 1), 10000.0)
    assert torch.equal(rot[0].view(m, 1, h, dk), want_q)
    assert torch.equal(rot[1].view(m, 1, hkv, dk), want_k)
    assert torch.equal(rot[2], plain[2])
