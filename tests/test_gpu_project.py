"""The prefill's stacked projections (``vsp_project_bf16``): every block of a pass's weight over the
columns it uses, one launch, through the C ABI.

Parity: each output column against the float64 product of the same bf16 operands: within one bf16
rounding of the exact product (2^-8 relative) plus the float32 accumulation's share of the row's
magnitude. The write strength's block is the logistic of its bf16-rounded product, within one bf16
rounding of float64's, and bitwise what the decode step's fused projection stores for the same
operand (the two launches share that arithmetic).
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


def _operands(m, d, p, cols, seed):
    g = torch.Generator().manual_seed(seed)
    z = torch.randn(m, d, generator=g).to(BF16).to(GPU)
    w = (torch.randn(p, d, cols, generator=g) / d ** 0.5).to(BF16).to(GPU)
    return z, w, w.transpose(1, 2).contiguous()


@pytest.mark.parametrize(("m", "d"), [(1, 64), (77, 128), (256, 512), (300, 512), (1000, 192), (4097, 512), (33, 1024)])
def test_every_block_matches_the_float64_product(m, d):
    from vesper.kernels.norm import projection

    cols = 512 if d >= 512 else 256
    used = (cols, cols // 2 + 8, 40, 8)
    z, w, wt = _operands(m, d, 4, cols, m * 13 + d)
    outs = projection(z, wt, used, sigmoid_block=3)
    torch.cuda.synchronize()
    for j, (o, u) in enumerate(zip(outs, used)):
        assert o.shape == (m, u) and o.dtype == BF16 and o.is_contiguous()
        _check_block(o, z, w[j, :, :u], sigmoid=j == 3)


@pytest.mark.parametrize("used", [(512,), (130, 3), (5, 129, 512)])
def test_fewer_blocks_and_ragged_widths(used):
    from vesper.kernels.norm import projection

    m, d, cols = 515, 256, 512
    z, w, wt = _operands(m, d, len(used), cols, sum(used))
    outs = projection(z, wt, used)
    for j, (o, u) in enumerate(zip(outs, used)):
        _check_block(o, z, w[j, :, :u])


def test_the_looped_column_shape_and_repeats():
    # B4 T2048 d512, the recurrent sublayer's four blocks (q, z, v and the 8-column write strength)
    from vesper.kernels.norm import projection

    m, d, cols = 8192, 512, 512
    used = (512, 512, 512, 8)
    z, w, wt = _operands(m, d, 4, cols, 5)
    outs = projection(z, wt, used, sigmoid_block=3)
    again = projection(z, wt, used, sigmoid_block=3)
    for j, (o, u) in enumerate(zip(outs, used)):
        assert torch.equal(o, again[j])
        rows = torch.arange(0, m, 61, device=GPU)  # a sample of rows, every tile of them
        _check_block(o[rows], z[rows], w[j, :, :u], sigmoid=j == 3)


def test_the_write_strength_is_the_decode_projections():
    # the same operand through both launches: the logistic block bitwise equal when the products
    # round to the same bf16 (the two sum in different orders, so compare where they agree)
    from vesper.kernels.norm import decode_projection, projection, rms_norm_bf16

    g = torch.Generator().manual_seed(21)
    m, d, cols = 48, 512, 512
    x = torch.randn(m, d, generator=g).to(GPU)
    w = (torch.randn(4, d, cols, generator=g) / d ** 0.5).to(BF16).to(GPU)
    wt = w.transpose(1, 2).contiguous()
    used = (512, 512, 512, 8)
    dec = decode_projection(x, wt, used, sigmoid_block=3)
    pre = projection(rms_norm_bf16(x), wt, used)
    pre_sig = projection(rms_norm_bf16(x), wt, used, sigmoid_block=3)
    same = pre[3] == decode_projection(x, wt, used)[3]  # equal products
    assert bool(same.float().mean() > 0.9)
    assert torch.equal(pre_sig[3][same], dec[3][same])


def test_a_mistaken_operand_is_caught():
    # the same bound fails for the product with the weight's blocks swapped: the check is tight
    from vesper.kernels.norm import projection

    m, d, cols = 300, 128, 128
    z, w, wt = _operands(m, d, 2, cols, 12)
    outs = projection(z, wt, (cols, cols))
    _check_block(outs[0], z, w[0])
    with pytest.raises(AssertionError):
        _check_block(outs[0], z, w[1])
    with pytest.raises(AssertionError):  # one input feature dropped from the product
        _check_block(outs[0], z[:, 1:], w[0, 1:])


def test_refusals():
    from vesper.contracts import ContractError
    from vesper.kernels.norm import projection

    z, _, wt = _operands(16, 128, 2, 64, 3)
    with pytest.raises(ContractError):
        projection(z[:, :96].contiguous(), wt[:, :, :96].contiguous(), (64, 64))  # width not a multiple of 64
    with pytest.raises(ContractError):
        projection(z, wt, (64,))  # one width for two blocks
    with pytest.raises(ContractError):
        projection(z, wt, (64, 65))  # more columns than the block has
    with pytest.raises(ContractError):
        projection(z.float(), wt, (64, 64))
    with pytest.raises(ContractError):
        projection(z, wt, (64, 64), sigmoid_block=2)
    assert [o.shape for o in projection(z[:0], wt, (64, 8))] == [(0, 64), (0, 8)]
