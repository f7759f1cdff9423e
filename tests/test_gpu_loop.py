"""The looped column with halting (``vesper.loop``) on the GPU against the loop oracle.

Parity: relative Frobenius error of the halted hidden states and of every pass's scan state below
3e-2 (the reference's attention bound; eight bf16 mixer passes compound their roundings), the
per-token pass counts exact. At the full config size: exact size-independent properties
(determinism, pass counts from the exit trace, early-halting tokens bitwise equal to a one-pass
run) and fp32-oracle parity checks over two passes and over all eight.
"""

from __future__ import annotations

import pytest
import torch

from conftest import needs_gpu
from oracle import loop as ol
from oracle.delta import relative_error

pytestmark = [pytest.mark.gpu, needs_gpu]

GPU = torch.device("cuda")


def _setup(b, n, d, h, hkv, dk, w, passes, seed, p_halt=0.3):
    from vesper.loop import LoopedColumn

    column = LoopedColumn.random(d, h, hkv, dk, w, passes, seed, GPU)
    g = torch.Generator().manual_seed(seed + 1)
    x0 = torch.randn(b, n, d, generator=g)
    exits = [torch.rand(b, n, generator=g) < p_halt for _ in range(passes)]
    states = [0.02 * torch.randn(b, h, dk, dk, generator=g) for _ in range(passes)]
    return column, x0, exits, states


def _oracle(column, x0, exits, states, dtype=torch.float64):
    ws = {name: [t.to("cpu", dtype) for t in column.w[name]] for name in column.w}
    weights = ol.MixerWeights(**ws, heads=column.heads, kv_heads=column.kv_heads, head_dim=column.head_dim,
                              window=column.window, rotary_base=column.rotary_base)
    return ol.loop_forward(x0.to(dtype), ol.mixer_column_step(weights), [s.to(dtype) for s in states], exits)


def _expected_iters(exits, passes):
    b, n = exits[0].shape
    iters = torch.full((b, n), passes, dtype=torch.int32)
    done = torch.zeros(b, n, dtype=torch.bool)
    for t in range(passes - 1):
        now = exits[t] & ~done
        iters[now] = t + 1
        done |= now
    return iters


def test_small_loop_matches_the_oracle():
    b, n, d, h, hkv, dk, w, passes = 2, 200, 128, 2, 2, 64, 64, 4
    column, x0, exits, states = _setup(b, n, d, h, hkv, dk, w, passes, seed=5)
    got = column.forward(x0.to(GPU), [s.to(GPU) for s in states], [e.to(GPU) for e in exits])
    want = _oracle(column, x0, exits, states)
    assert torch.equal(got.n_iters.cpu(), want.n_iters)
    assert torch.equal(got.n_iters.cpu(), _expected_iters(exits, passes))
    assert relative_error(got.y, want.y) < 3e-2
    for t in range(passes):
        assert relative_error(got.states[t], want.states[t]) < 3e-2, t


def test_config_b4_t2048_d512_h8_eight_passes_properties():
    from vesper.loop import LoopedColumn

    b, n, d, h, dk, w, passes = 4, 2048, 512, 8, 64, 512, 8
    column, x0, exits, states = _setup(b, n, d, h, h, dk, w, passes, seed=7)
    dx0, dst, dex = x0.to(GPU), [s.to(GPU) for s in states], [e.to(GPU) for e in exits]
    first = column.forward(dx0, dst, dex)
    second = column.forward(dx0, dst, dex)
    assert torch.equal(first.y, second.y)
    assert all(torch.equal(a, c) for a, c in zip(first.states, second.states))
    assert bool(torch.isfinite(first.y).all())
    assert torch.equal(first.n_iters.cpu(), _expected_iters(exits, passes))
    # a token that halts after the first pass keeps its pass-1 hidden state: that of a one-pass run
    one = LoopedColumn({name: column.w[name][:1] for name in column.w}, h, h, dk, w)
    single = one.forward(dx0, dst[:1], dex[:1])
    early = (first.n_iters == 1)
    assert int(early.sum()) > 0
    assert torch.equal(first.y[early], single.y[early])
    assert torch.equal(first.states[0], single.states[0])


def test_config_size_two_passes_match_the_fp32_oracle():
    b, n, d, h, dk, w, passes = 4, 2048, 512, 8, 64, 512, 2
    column, x0, exits, states = _setup(b, n, d, h, h, dk, w, passes, seed=9)
    got = column.forward(x0.to(GPU), [s.to(GPU) for s in states], [e.to(GPU) for e in exits])
    want = _oracle(column, x0, exits, states, dtype=torch.float32)
    assert relative_error(got.y, want.y) < 3e-2
    for t in range(passes):
        assert relative_error(got.states[t], want.states[t]) < 3e-2, t


def test_config_size_eight_passes_match_the_fp32_oracle():
    # the full config: B4 T2048 d512, 8 heads of 64, window 512, all 8 passes with halting 0.3
    b, n, d, h, dk, w, passes = 4, 2048, 512, 8, 64, 512, 8
    column, x0, exits, states = _setup(b, n, d, h, h, dk, w, passes, seed=17)
    got = column.forward(x0.to(GPU), [s.to(GPU) for s in states], [e.to(GPU) for e in exits])
    want = _oracle(column, x0, exits, states, dtype=torch.float32)
    assert torch.equal(got.n_iters.cpu(), want.n_iters)
    assert torch.equal(got.n_iters.cpu(), _expected_iters(exits, passes))
    assert relative_error(got.y, want.y) < 3e-2
    for t in range(passes):
        assert relative_error(got.states[t], want.states[t]) < 3e-2, t


def test_eight_passes_at_b4_t768_d512_h8_w512_match_the_oracle():
    # the config's depth and widths (8 passes, d 512, 8 heads of 64, window 512) at a shorter
    # sequence, so the float64 oracle finishes in seconds; the window still slides
    b, n, d, h, dk, w, passes = 4, 768, 512, 8, 64, 512, 8
    column, x0, exits, states = _setup(b, n, d, h, h, dk, w, passes, seed=13)
    got = column.forward(x0.to(GPU), [s.to(GPU) for s in states], [e.to(GPU) for e in exits])
    want = _oracle(column, x0, exits, states)
    assert torch.equal(got.n_iters.cpu(), want.n_iters)
    assert relative_error(got.y, want.y) < 3e-2
    for t in range(passes):
        assert relative_error(got.states[t], want.states[t]) < 3e-2, t


def test_refusals():
    from vesper.contracts import ContractError
    from vesper.loop import LoopedColumn

    column = LoopedColumn.random(64, 1, 1, 64, 16, 2, 0, GPU)
    x0 = torch.zeros(1, 8, 64, device=GPU)
    states = [torch.zeros(1, 1, 64, 64, device=GPU)] * 2
    exits = [torch.zeros(1, 8, dtype=torch.bool, device=GPU)] * 2
    with pytest.raises(ContractError, match="dtype"):
        column.forward(x0.half(), states, exits)
    with pytest.raises(ContractError, match="passes"):
        column.forward(x0, states[:1], exits)
    with pytest.raises(ContractError, match="axis"):
        column.forward(x0, states, [torch.zeros(1, 9, dtype=torch.bool, device=GPU)] * 2)


def test_the_loop_with_a_key_filter_matches_the_oracle():
    # halted tokens carry their frozen key input into the filter of later passes and their key
    # after it (column.py:779-789); each pass keeps its own key history
    from vesper.loop import LoopedColumn

    b, n, d, h, hkv, dk, w, passes, width = 2, 150, 128, 2, 2, 64, 64, 3, 4
    column = LoopedColumn.random(d, h, hkv, dk, w, passes, 11, GPU, key_conv=width)
    g = torch.Generator().manual_seed(12)
    x0 = torch.randn(b, n, d, generator=g)
    exits = [torch.rand(b, n, generator=g) < 0.3 for _ in range(passes)]
    states = [0.02 * torch.randn(b, h, dk, dk, generator=g) for _ in range(passes)]
    histories = [torch.randn(b, width - 1, d, generator=g) for _ in range(passes)]
    got = column.forward(x0.to(GPU), [s.to(GPU) for s in states], [e.to(GPU) for e in exits],
                         [z.to(GPU) for z in histories])
    ws = {name: [t.to("cpu", torch.float64) for t in column.w[name]] for name in column.w}
    weights = ol.MixerWeights(**ws, heads=h, kv_heads=hkv, head_dim=dk, window=w,
                              taps=[t.to("cpu", torch.float64) for t in column.taps], rotary_base=column.rotary_base)
    want = ol.loop_forward(x0.double(), ol.mixer_column_step(weights),
                           [(s.double(), z.double()) for s, z in zip(states, histories)], exits)
    assert torch.equal(got.n_iters.cpu(), want.n_iters)
    assert relative_error(got.y, want.y) < 3e-2
    for t in range(passes):
        assert relative_error(got.states[t], want.states[t][0]) < 3e-2, t
        assert relative_error(got.histories[t], want.states[t][1]) < 1e-2, t


# ---- copy-forward inside the kernels' loads against the where merges ----

def _both_modes(b, n, d, h, hkv, dk, w, passes, seed, key_conv=0, p_halt=0.3):
    from vesper.loop import LoopedColumn

    fused = LoopedColumn.random(d, h, hkv, dk, w, passes, seed, GPU, key_conv=key_conv)
    where = LoopedColumn.random(d, h, hkv, dk, w, passes, seed, GPU, key_conv=key_conv, copy_forward="where")
    g = torch.Generator().manual_seed(seed + 1)
    x0 = torch.randn(b, n, d, generator=g).to(GPU)
    exits = [(torch.rand(b, n, generator=g) < p_halt).to(GPU) for _ in range(passes)]
    states = [(0.02 * torch.randn(b, h, dk, dk, generator=g)).to(GPU) for _ in range(passes)]
    histories = [torch.randn(b, key_conv - 1, d, generator=g).to(GPU) for _ in range(passes)] if key_conv else None
    return fused.forward(x0, states, exits, histories), where.forward(x0, states, exits, histories), x0


@pytest.mark.parametrize(("key_conv", "p_halt"), [(0, 0.3), (4, 0.3), (4, 0.8), (2, 0.05)])
def test_fused_copy_forward_equals_the_where_merges_bitwise(key_conv, p_halt):
    got, want, x0 = _both_modes(2, 300, 128, 2, 2, 64, 64, 4, seed=21 + key_conv, key_conv=key_conv, p_halt=p_halt)
    assert torch.equal(got.y, want.y)
    assert torch.equal(got.n_iters, want.n_iters)
    for a, b in zip(got.states, want.states):
        assert torch.equal(a, b)
    if key_conv:
        for a, b in zip(got.histories, want.histories):
            assert torch.equal(a, b)
    assert not torch.equal(got.y, x0.float())  # the input is left as it was, and the passes changed it


def test_fused_copy_forward_at_b4_t2048_d512_h8_eight_passes():
    got, want, _ = _both_modes(4, 2048, 512, 8, 8, 64, 512, 8, seed=31, key_conv=4, p_halt=0.2)
    assert torch.equal(got.y, want.y) and torch.equal(got.n_iters, want.n_iters)
    for a, b in zip(got.states, want.states):
        assert torch.equal(a, b)


def test_copy_rows_where_equals_torch_where_bitwise():
    from vesper.kernels.carry import copy_rows_where

    g = torch.Generator().manual_seed(3)
    b, n = 3, 77
    flags = [(torch.rand(b, n, generator=g) < 0.4).to(GPU) for _ in range(3)]
    shapes = [((b, n, 4, 16), torch.bfloat16), ((b, n, 3), torch.bfloat16), ((b, n, 96), torch.float32),
              ((b, n, 5), torch.uint8)]
    items, want = [], []
    for i, (shape, dtype) in enumerate(shapes):
        src = (torch.randn(shape, generator=g) * 100).to(dtype).to(GPU)
        dst = (torch.randn(shape, generator=g) * 100).to(dtype).to(GPU)
        f = flags[i % 3]
        want.append(torch.where(f.reshape(b, n, *([1] * (len(shape) - 2))), src, dst))
        items.append((src, dst, f))
    copy_rows_where(items)
    for (_, dst, _), ref in zip(items, want):
        assert torch.equal(dst, ref)


def test_copy_rows_where_refusals():
    from vesper.contracts import ContractError
    from vesper.kernels.carry import copy_rows_where

    x = torch.zeros(2, 5, 8, device=GPU)
    f = torch.ones(2, 5, dtype=torch.bool, device=GPU)
    with pytest.raises(ContractError, match="at most"):
        copy_rows_where([(x, x.clone(), f)] * 9)
    with pytest.raises(ContractError, match="flags"):
        copy_rows_where([(x, x.clone(), f.float())])
    with pytest.raises(ContractError, match="contiguous"):
        copy_rows_where([(x[:, :, :4], x.clone()[:, :, ::2], f)])
    with pytest.raises(ContractError, match="token rows"):
        copy_rows_where([(x, x.clone(), f), (x[:1], x[:1].clone(), f[:1])])


def test_the_halting_step_matches_the_elementwise_steps():
    # vsp_halt_step: halts = active & exits (all active on the last pass), n_iters += active,
    # next = active & ~halts, against the torch steps it replaces
    from vesper.kernels.carry import halt_step

    g = torch.Generator().manual_seed(9)
    for last in (False, True):
        active = (torch.rand(3, 1000, generator=g) < 0.6).to(GPU)
        exits = (torch.rand(3, 1000, generator=g) < 0.3).to(GPU)
        n_iters = torch.randint(0, 5, (3, 1000), generator=g, dtype=torch.int32).to(GPU)
        want_halts = active if last else active & exits
        want_iters = n_iters + active.to(torch.int32)
        halts, nxt = halt_step(active, None if last else exits, n_iters)
        assert torch.equal(halts, want_halts) and torch.equal(n_iters, want_iters)
        assert torch.equal(nxt, active & ~want_halts)


def test_the_residual_rows_match_the_add_and_the_row_copy():
    # vsp_residual_rows_where: x[r] = x1[r] + a[r] on flagged rows (all rows without flags), the
    # other rows untouched, bit for bit the torch add followed by the row selection
    from vesper.kernels.carry import residual_rows_where

    g = torch.Generator().manual_seed(10)
    x1 = torch.randn(3, 100, 520, generator=g).to(GPU)
    a = torch.randn(3, 100, 520, generator=g).to(torch.bfloat16).to(GPU)
    flags = (torch.rand(3, 100, generator=g) < 0.5).to(GPU)
    for fl in (flags, None):
        x = torch.randn(3, 100, 520, generator=g).to(GPU)
        want = x1 + a if fl is None else torch.where(fl[..., None], x1 + a, x)
        residual_rows_where(x1, a, x, fl)
        assert torch.equal(x, want)
