"""The column's single-token decoder (``vesper.decode``) on the GPU.

As the reference's own tests of its decoder (``tests/test_decode.py:45-116``): the tokenwise
ring step against the chunked forward over the whole sequence, the captured step against the same
step run eagerly (bitwise, every output and every carried state, across the warm-up/capture
boundary), and a second generation on one decoder against a cold eager one. The numeric truth is
the oracle's tokenwise decode (``oracle.loop.mixer_decode_step``, pinned against the oracle's
chunked forward in ``tests/test_oracle_loop.py``) in float64 with the GPU path's bf16 rounding
points: relative Frobenius error below 3e-2 (the reference's attention bound; bf16 mixers and
projections compound over the passes).
"""

from __future__ import annotations

import pytest
import torch

from conftest import needs_gpu
from oracle import loop as ol
from oracle.delta import relative_error

pytestmark = [pytest.mark.gpu, needs_gpu]

GPU = torch.device("cuda")
F64 = torch.float64
PER_PASS = 6


def _column(key_conv, passes=3, d=64, h=4, hkv=2, dk=16, w=8, seed=1):
    from vesper.loop import LoopedColumn

    return LoopedColumn.random(d, h, hkv, dk, w, passes, seed, GPU, key_conv=key_conv)


def _weights(column, dtype=F64):
    ws = {name: [t.to("cpu", dtype) for t in column.w[name]] for name in column.w}
    taps = None if column.taps is None else [t.to("cpu", dtype) for t in column.taps]
    return ol.MixerWeights(**ws, heads=column.heads, kv_heads=column.kv_heads, head_dim=column.head_dim,
                           window=column.window, taps=taps, rotary_base=column.rotary_base)


def _inputs(b, n, d, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(b, n, d, generator=g)


def _at(i, b):
    return torch.full((b, 1), i, dtype=torch.long, device=GPU)


@pytest.mark.parametrize("key_conv", [0, 4])
def test_the_decode_step_matches_the_oracle(key_conv):
    from vesper.decode import cold_states, decode_step

    column = _column(key_conv)
    b, n, depth = 2, 20, 2  # window 8: every ring wraps twice
    x = _inputs(b, n, 64, seed=2)
    flat = cold_states(column, b, GPU)
    weights = _weights(column)
    step = ol.mixer_decode_step(weights, depth)
    states = ol.cold_decode_states(weights, b, F64)
    for i in range(n):
        y, *flat = decode_step(column, depth, [x[:, i : i + 1].to(GPU), _at(i, b), *flat])
        want, states = step(x[:, i : i + 1].double(), torch.full((b, 1), i, dtype=torch.long), states)
        assert relative_error(y, want) < 3e-2, i
    for t in range(depth):
        assert relative_error(flat[PER_PASS * t], states[t][0]) < 3e-2, t
        if key_conv:
            assert relative_error(flat[PER_PASS * t + 1], states[t][1]) < 1e-2, t
        assert torch.equal(flat[PER_PASS * t + 4].cpu(), states[t][2][2])  # ring positions
        assert torch.equal(flat[PER_PASS * t + 5].cpu(), states[t][2][3])  # ring valid flags
    for t in range(depth, column.passes):  # passes past the depth stay cold
        assert not bool(flat[PER_PASS * t + 5].any()) and not bool(flat[PER_PASS * t].any())


def test_tokenwise_decoding_equals_the_chunked_forward_on_the_gpu():
    from vesper.decode import cold_states, decode_step

    column = _column(4, passes=2)
    b, n = 2, 20
    x = _inputs(b, n, 64, seed=3).to(GPU)
    chunked = column.forward(x, [torch.zeros(b, 4, 16, 16, device=GPU)] * 2,
                             [torch.zeros(b, n, dtype=torch.bool, device=GPU)] * 2,
                             [torch.zeros(b, 3, 64, device=GPU)] * 2)
    flat = cold_states(column, b, GPU)
    ys = []
    for i in range(n):
        y, *flat = decode_step(column, 2, [x[:, i : i + 1], _at(i, b), *flat])
        ys.append(y)
    assert relative_error(torch.cat(ys, dim=1), chunked.y) < 3e-2
    for t in range(2):
        assert relative_error(flat[PER_PASS * t], chunked.states[t]) < 3e-2
        assert relative_error(flat[PER_PASS * t + 1], chunked.histories[t]) < 1e-2


@pytest.mark.parametrize("key_conv", [0, 4])
def test_the_captured_step_equals_the_eager_step_bitwise_across_the_capture(key_conv):
    from vesper.decode import WARM_STEPS, CapturedDecoder, cold_states, decode_step

    column = _column(key_conv)
    b, n, depth = 3, WARM_STEPS + 6, 2
    x = _inputs(b, n, 64, seed=4).to(GPU)
    decoder = CapturedDecoder(column, depth)
    eager_flat, captured_flat = cold_states(column, b, GPU), decoder.start(b)
    for i in range(n):
        eager = decode_step(column, depth, [x[:, i : i + 1], _at(i, b), *eager_flat])
        y, flat = decoder.step(x[:, i : i + 1], _at(i, b), captured_flat)
        assert torch.equal(y, eager[0]), i
        for got, want in zip(flat, eager[1:]):
            assert torch.equal(got, want), i
        eager_flat = eager[1:]
        captured_flat = [t.clone() for t in flat] if i % 2 else flat  # copied in, or the graph's own
    assert decoder.captures == 1
    assert decoder.replays == n - WARM_STEPS


def test_a_call_of_another_batch_after_the_capture_is_refused_and_the_graph_still_matches_eager():
    from vesper.contracts import ContractError
    from vesper.decode import WARM_STEPS, CapturedDecoder, cold_states, decode_step

    column = _column(0)
    b, depth = 2, 2
    x = _inputs(b, WARM_STEPS + 4, 64, seed=7).to(GPU)
    decoder = CapturedDecoder(column, depth)
    flat, eager_flat = decoder.start(b), cold_states(column, b, GPU)
    for i in range(WARM_STEPS + 4):
        if i == WARM_STEPS + 2:  # captured by now: a wider batch is refused before the graph's buffers change
            assert decoder.captures == 1
            wide = decoder.start(b + 1)
            with pytest.raises(ContractError, match="captured"):
                decoder.step(_inputs(b + 1, 1, 64, seed=8).to(GPU), _at(i, b + 1), wide)
        y, flat = decoder.step(x[:, i : i + 1], _at(i, b), flat)
        eager = decode_step(column, depth, [x[:, i : i + 1], _at(i, b), *eager_flat])
        assert torch.equal(y, eager[0]), i
        for got, want in zip(flat, eager[1:]):
            assert torch.equal(got, want), i
        eager_flat = eager[1:]


def test_a_second_generation_on_one_decoder_starts_truly_cold():
    from vesper.decode import CapturedDecoder, cold_states, decode_step

    column = _column(4)
    b = 2
    used = CapturedDecoder(column, 3)
    first, second = _inputs(b, 7, 64, seed=5).to(GPU), _inputs(b, 9, 64, seed=6).to(GPU)
    flat = used.start(b)
    for i in range(7):  # warms and captures on a discarded prompt
        _, flat = used.step(first[:, i : i + 1], _at(i, b), flat)
    assert used.captures == 1
    flat, cold = used.start(b), cold_states(column, b, GPU)
    for i in range(9):
        y, flat = used.step(second[:, i : i + 1], _at(i, b), flat)
        reference = decode_step(column, 3, [second[:, i : i + 1], _at(i, b), *cold])
        assert torch.equal(y, reference[0]), i
        cold = reference[1:]


def test_the_decode_shape_b64_d512_h8_w512_two_passes():
    from vesper.decode import CapturedDecoder, cold_states, decode_step

    column = _column(4, passes=2, d=512, h=8, hkv=8, dk=64, w=512, seed=7)
    b, n = 64, 6
    x = _inputs(b, n, 512, seed=8)
    decoder = CapturedDecoder(column, 2)
    flat, eager_flat = decoder.start(b), cold_states(column, b, GPU)
    weights = _weights(column, torch.float32)
    step = ol.mixer_decode_step(weights, 2)
    states = ol.cold_decode_states(weights, b, torch.float32)
    for i in range(n):
        pos = torch.full((b, 1), 1000 + i, dtype=torch.long)  # positions far past the window's size
        y, flat = decoder.step(x[:, i : i + 1].to(GPU), pos.to(GPU), flat)
        eager = decode_step(column, 2, [x[:, i : i + 1].to(GPU), pos.to(GPU), *eager_flat])
        eager_flat = eager[1:]
        assert torch.equal(y, eager[0])
        want, states = step(x[:, i : i + 1], pos, states)
        assert relative_error(y, want) < 3e-2, i
        assert bool(torch.isfinite(y).all())


def test_refusals():
    from vesper.contracts import ContractError
    from vesper.decode import CapturedDecoder, cold_states, decode_step
    from vesper.loop import LoopedColumn

    with pytest.raises(ContractError, match="CUDA"):
        CapturedDecoder(LoopedColumn.random(64, 4, 2, 16, 8, 2, 0, torch.device("cpu")), 1)
    column = _column(4)
    with pytest.raises(ContractError, match="depth"):
        CapturedDecoder(column, 4)
    flat = cold_states(column, 1, GPU)
    x = torch.zeros(1, 1, 64, device=GPU)
    with pytest.raises(ContractError, match="depth"):
        decode_step(column, 0, [x, _at(0, 1), *flat])
    with pytest.raises(ContractError, match="dtype"):
        decode_step(column, 1, [x.double(), _at(0, 1), *flat])
    with pytest.raises(ContractError, match="state tensors"):
        decode_step(column, 1, [x, _at(0, 1), *flat[:-1]])
