"""The loop oracle (``oracle.loop``) against the reference's hand-computed copy-forward table.

The scalar column is the one of the reference's pass-state review, section B
(``tests/test_loop.py:38-79``): one head of width one, unit key and query, value = the input,
beta 1/2, output = the state read; no attention and no residual, so the rational answers of
``tests/test_loop.py:126-175`` apply exactly.
"""

from __future__ import annotations

import dataclasses
from fractions import Fraction

import pytest
import torch

from oracle import loop as ol
from oracle.delta import delta_scan_chunked

F64 = torch.float64


def scalar_step(x, t, state, carry):
    del t
    b, n = x.shape[0], x.shape[1]
    ones = torch.ones(b, n, 1, 1, dtype=x.dtype)
    k, v = ones, x.reshape(b, n, 1, 1)
    beta = torch.full((b, n, 1), 0.5, dtype=x.dtype)
    if carry is not None:
        active, carried = carry
        k = ol.carry_in(active, k, carried.k)
        v = ol.carry_in(active, v, carried.v)
        beta = ol.carry_in(active, beta, carried.beta)
    o, new = delta_scan_chunked(ones, k, v, beta, state, 1)
    empty = torch.zeros(b, n, 1, 1, dtype=x.dtype)
    return o.reshape(b, n, 1), new, ol.Written(k=k, v=v, beta=beta, attn_k=empty, attn_v=empty)


def scalar_states(values):
    return [torch.full((1, 1, 1, 1), v, dtype=F64) for v in values]


def section_b():
    x0 = torch.tensor([[[2.0], [4.0]]], dtype=F64)
    exits = [torch.tensor([[True, False]]), torch.tensor([[False, False]])]
    return ol.loop_forward(x0, scalar_step, scalar_states([0.0, 10.0]), exits)


def test_section_b_copy_forward_table():
    # pass 1: 0 -> 1 -> 5/2; token 1 halts with output 1. Pass 2 writes token 1's saved
    # (k, v, beta) = (1, 2, 1/2) first: 10/2 + 2/2 = 6, then token 2 with its pass-1 output 5/2:
    # 6/2 + (5/2)/2 = 17/4, also its pass-2 output (tests/test_loop.py:126-138)
    out = section_b()
    assert out.states[0].item() == Fraction(5, 2)
    assert out.states[1].item() == Fraction(17, 4)
    assert out.y[0, 0, 0].item() == 1.0
    assert out.y[0, 1, 0].item() == Fraction(17, 4)
    assert out.n_iters.tolist() == [[1, 2]]
    assert out.per_pass[1][0, 0, 0].item() == 0.0  # token 1 produced nothing at pass 2


def test_the_inactive_token_still_writes():
    # tests/test_loop.py:141-150: one token, halting after pass 1: pass 2's state is 10/2 + 2/2
    x0 = torch.tensor([[[2.0]]], dtype=F64)
    out = ol.loop_forward(x0, scalar_step, scalar_states([0.0, 10.0]), [torch.tensor([[True]])] * 2)
    assert out.states[0].item() == 1.0
    assert out.states[1].item() == 6.0


def test_all_tokens_halted_passes_still_update_every_later_state():
    # tests/test_loop.py:162-175: both tokens halt after pass 1 of three
    x0 = torch.tensor([[[2.0], [4.0]]], dtype=F64)
    out = ol.loop_forward(x0, scalar_step, scalar_states([0.0, 10.0, 20.0]), [torch.tensor([[True, True]])] * 3)
    assert out.n_iters.tolist() == [[1, 1]]
    assert out.states[1].item() == 5.0  # 10 -> 6 -> 5
    assert out.states[2].item() == 7.5  # 20 -> 11 -> 7.5
    assert all(bool((p == 0).all()) for p in out.per_pass[1:])


@pytest.mark.parametrize("kind", ["no_carry", "no_write"])
def test_the_table_catches_planted_mistakes(kind, monkeypatch):
    if kind == "no_carry":  # halted tokens write their fresh projections instead of the frozen ones
        monkeypatch.setattr(ol, "carry_in", lambda active, fresh, carried: fresh)
    else:  # halted tokens stop writing (zero projections, so beta = 0)
        real = ol.carry_in
        monkeypatch.setattr(ol, "carry_in", lambda active, fresh, carried: real(active, fresh, torch.zeros_like(carried)))
    x0 = torch.tensor([[[2.0], [4.0]]], dtype=F64)
    exits = [torch.tensor([[True, False]]), torch.tensor([[False, False]]), torch.tensor([[False, False]])]
    out = ol.loop_forward(x0, scalar_step, scalar_states([0.0, 10.0, 20.0]), exits)
    # the correct third state: 20 -> (20 + 2)/2 = 11 -> (11 + 17/4)/2 = 61/8
    assert [out.states[1].item(), out.states[2].item()] != [Fraction(17, 4), Fraction(61, 8)]


def test_three_pass_table_without_mistakes():
    x0 = torch.tensor([[[2.0], [4.0]]], dtype=F64)
    exits = [torch.tensor([[True, False]]), torch.tensor([[False, False]]), torch.tensor([[False, False]])]
    out = ol.loop_forward(x0, scalar_step, scalar_states([0.0, 10.0, 20.0]), exits)
    assert [out.states[1].item(), out.states[2].item()] == [Fraction(17, 4), Fraction(61, 8)]
    assert out.y[0, 1, 0].item() == Fraction(61, 8) and out.n_iters.tolist() == [[1, 3]]


def _mixer_weights(d, h, hkv, dk, w, passes, seed):
    g = torch.Generator().manual_seed(seed)

    def mats(out):
        return [(torch.randn(d, out, generator=g) / d**0.5).to(torch.bfloat16).double() for _ in range(passes)]

    return ol.MixerWeights(wq=mats(h * dk), wk=mats(h * dk), wv=mats(h * dk), wb=mats(h), waq=mats(h * dk),
                           wak=mats(hkv * dk), wav=mats(hkv * dk), heads=h, kv_heads=hkv, head_dim=dk, window=w)


def test_masked_mixers_equal_dense_mixers_for_every_active_token():
    # the kernels skip inactive tokens' reads and outputs (loop.py:24-26): running the mixers with
    # the active mask gives, bit for bit, what the reference's dense mixers give once the loop
    # has zeroed the inactive outputs and merged the carried projections
    d, h, dk, passes = 16, 2, 8, 3
    weights = _mixer_weights(d, h, h, dk, 6, passes, seed=3)
    g = torch.Generator().manual_seed(4)
    x0 = torch.randn(2, 19, d, generator=g, dtype=F64)
    exits = [torch.rand(2, 19, generator=g) < 0.3 for _ in range(passes)]
    states = [0.1 * torch.randn(2, h, dk, dk, generator=g, dtype=F64) for _ in range(passes)]
    masked = ol.loop_forward(x0, ol.mixer_column_step(weights), states, exits)
    dense = ol.loop_forward(x0, ol.mixer_column_step(weights, masked=False), states, exits)
    assert torch.equal(masked.y, dense.y)
    assert all(torch.equal(a, b) for a, b in zip(masked.states, dense.states))
    assert torch.equal(masked.n_iters, dense.n_iters)
    assert int((masked.n_iters < passes).sum()) > 0  # some tokens did halt early
    # halted tokens carry forward the hidden state of their halting pass
    halt_pass = masked.n_iters - 1
    for t in range(passes):
        sel = halt_pass == t
        assert torch.equal(masked.y[sel], masked.per_pass[t][sel])


def _filter_weights(d, h, hkv, dk, w, passes, seed, width):
    base = _mixer_weights(d, h, hkv, dk, w, passes, seed)
    g = torch.Generator().manual_seed(seed + 100)
    taps = [(torch.rand(width, h * dk, generator=g, dtype=F64) * 2 - 1) / width**0.5 for _ in range(passes)]
    return ol.MixerWeights(**{f: getattr(base, f) for f in ("wq", "wk", "wv", "wb", "waq", "wak", "wav")},
                           heads=h, kv_heads=hkv, head_dim=dk, window=w, taps=taps)


@pytest.mark.parametrize(("width", "rotary_base"), [(0, None), (3, None), (3, 10000.0)])
def test_tokenwise_ring_decoding_equals_the_chunked_forward(width, rotary_base):
    # the reference's own check of its decoder (tests/test_decode.py:45-76): the chunked forward
    # over the whole sequence is the truth for the tokenwise ring step; window 6 against 20
    # tokens, so every ring wraps three times; exact arithmetic here (float64, no bf16 rounding);
    # with rotary, the token at position i turns as the chunk's row i does
    d, h, hkv, dk, w, passes, depth, b, n = 16, 2, 1, 8, 6, 3, 2, 2, 20
    weights = (_mixer_weights(d, h, hkv, dk, w, passes, seed=8) if width == 0
               else _filter_weights(d, h, hkv, dk, w, passes, seed=8, width=width))
    if rotary_base is not None:
        weights = dataclasses.replace(weights, rotary_base=rotary_base)
    g = torch.Generator().manual_seed(9)
    x0 = torch.randn(b, n, d, generator=g, dtype=F64)
    cold = ol.cold_decode_states(weights, b, F64)
    chunk_states = [(c[0], c[1]) if width else c[0] for c in cold[:depth]]
    exits = [torch.zeros(b, n, dtype=torch.bool)] * depth
    chunked = ol.loop_forward(x0, ol.mixer_column_step(weights, masked=False, bf16=False), chunk_states, exits)
    step = ol.mixer_decode_step(weights, depth, bf16=False)
    states = cold
    for i in range(n):
        y, states = step(x0[:, i : i + 1], torch.full((b, 1), i, dtype=torch.long), states)
        torch.testing.assert_close(y, chunked.y[:, i : i + 1], rtol=1e-10, atol=1e-10)
    for t in range(depth):
        want = chunked.states[t] if width == 0 else chunked.states[t][0]
        torch.testing.assert_close(states[t][0], want, rtol=1e-10, atol=1e-12)
        if width:
            # the newest K - 1 key inputs (per-token and whole-chunk matmuls round alike to 1e-12)
            torch.testing.assert_close(states[t][1], chunked.states[t][1], rtol=1e-12, atol=1e-12)
        assert states[t][2][3].all() and torch.equal(states[t][2][2].sort(dim=1).values,
                                                      torch.arange(n - w, n).expand(b, w))
    for t in range(depth, passes):  # passes past the depth are left as they were
        assert states[t] is cold[t]


def test_the_decode_pin_catches_a_planted_mistake():
    d, h, hkv, dk, w, passes, depth, b, n = 16, 2, 1, 8, 6, 2, 2, 1, 10
    weights = _filter_weights(d, h, hkv, dk, w, passes, seed=10, width=3)
    g = torch.Generator().manual_seed(11)
    x0 = torch.randn(b, n, d, generator=g, dtype=F64)
    cold = ol.cold_decode_states(weights, b, F64)
    exits = [torch.zeros(b, n, dtype=torch.bool)] * depth
    chunked = ol.loop_forward(x0, ol.mixer_column_step(weights, masked=False, bf16=False),
                              [(c[0], c[1]) for c in cold], exits)
    step = ol.mixer_decode_step(weights, depth, bf16=False)
    states, worst = cold, 0.0
    for i in range(n):
        # a ring written at the wrong slot age: the token's position one too small
        y, states = step(x0[:, i : i + 1], torch.full((b, 1), max(i - 1, 0), dtype=torch.long), states)
        worst = max(worst, float((y - chunked.y[:, i : i + 1]).abs().max()))
    assert worst > 1e-3


def test_the_scan_reads_the_raw_query():
    # RecurrentSublayer.project (column.py:236-253) hands F.linear(x, w_q) to the scan unchanged:
    # "q is not normalized" (docs/model-card.md:26). Unit-scale weights give queries of norm well
    # above one, where normalizing them would change the output. Zero attention values make the
    # attention sublayer add nothing, so the step's output minus its input is the scan's read.
    from oracle.delta import delta_scan_serial, normalize_keys

    d, h, dk, n = 8, 2, 4, 5
    g = torch.Generator().manual_seed(9)

    def mats(out):
        return [torch.randn(d, out, generator=g, dtype=F64)]

    weights = ol.MixerWeights(wq=mats(h * dk), wk=mats(h * dk), wv=mats(h * dk), wb=mats(h), waq=mats(h * dk),
                              wak=mats(h * dk), wav=[torch.zeros(d, h * dk, dtype=F64)], heads=h, kv_heads=h,
                              head_dim=dk, window=4)
    x = torch.randn(1, n, d, generator=g, dtype=F64)
    s0 = torch.zeros(1, h, dk, dk, dtype=F64)
    y, _, _ = ol.mixer_column_step(weights, masked=False, bf16=False)(x, 0, s0, None)
    xn = x / x.square().mean(dim=-1, keepdim=True).add(1e-6).sqrt()  # RMSNorm, gain one (column.py:146-188)
    q = (xn @ weights.wq[0]).view(1, n, h, dk)
    k = normalize_keys((xn @ weights.wk[0]).view(1, n, h, dk))
    v = (xn @ weights.wv[0]).view(1, n, h, dk)
    beta = torch.sigmoid(xn @ weights.wb[0])
    o, _ = delta_scan_serial(q, k, v, beta, s0)
    assert float(q.norm(dim=-1).min()) > 1.0
    assert torch.allclose(y - x, o.reshape(1, n, h * dk), rtol=0, atol=1e-12)
    o_normalized, _ = delta_scan_serial(normalize_keys(q), k, v, beta, s0)
    assert float((o_normalized - o).abs().max()) > 1e-2


def test_rms_norm_against_the_plain_formula_and_its_edges():
    # column.py:146-188 with unit gain: x / sqrt(mean(x^2) + 1e-6); the oracle divides by the
    # row's peak first, which changes nothing in exact arithmetic and keeps float32 finite
    x = torch.tensor([[3.0, 4.0], [0.0, 0.0], [1e-5, -2e-5], [0.5, -0.5]], dtype=F64)
    plain = x / torch.sqrt(x.square().mean(-1, keepdim=True) + 1e-6)
    assert (ol.rms_norm(x) - plain).abs().max().item() < 1e-14
    assert not bool(ol.rms_norm(x)[1].any())
    # a row far below sqrt(eps) is scaled by about 1 / 1e-3, not blown up to unit size
    assert abs(float(ol.rms_norm(x)[2, 1]) - (-2e-5 / 1e-3)) < 1e-5
    g = torch.Generator().manual_seed(3)
    big = torch.randn(6, 512, generator=g, dtype=torch.float32) * 1e30  # squares overflow float32
    out = ol.rms_norm(big)
    assert torch.isfinite(out).all()
    assert (out.double().square().mean(-1) - 1).abs().max().item() < 1e-5
    # a planted mistake: eps dropped (the tiny row would come out at unit size)
    no_eps = x / torch.sqrt(x.square().mean(-1, keepdim=True)).clamp_min(1e-300)
    assert not torch.allclose(no_eps[2], ol.rms_norm(x)[2], atol=1e-3)
