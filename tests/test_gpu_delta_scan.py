"""The HIP delta scan (``vesper.kernels.delta_scan``) against the CPU oracle, through the C ABI.

The oracle in float64, fed the same bf16- (or fp32-) valued inputs, is the truth. Tolerances are
the reference's own (``tests/test_delta_scan_fused.py:34``, ``:255``): relative Frobenius error
below 1.5e-2 for the bf16 kernel and 1e-5 for the fp32 kernel, on outputs and final states, and on
the gradients of q, k, v, beta and the initial state (``:87-102``, ``:285-300``; the oracle's by
autograd through the chunked scan, its WY form pinned in ``tests/test_oracle_delta.py``).
"""

from __future__ import annotations

import math

import pytest
import torch

from conftest import needs_gpu, scan_inputs
from oracle.delta import delta_scan_chunked, delta_scan_step, normalize_keys, relative_error

pytestmark = [pytest.mark.gpu, needs_gpu]

BF16 = torch.bfloat16
TOL = 1.5e-2
TOL_FP32 = 1e-5
GPU = torch.device("cuda")

# n = 1, one short of a chunk, one past it, two and a partial, 4096 (tests/test_delta_scan_fused.py:71)
SIZES = [(2, 1, 2, 16), (2, 63, 3, 16), (1, 65, 2, 64), (2, 130, 3, 16), (1, 4096, 2, 64)]


def _bf16_inputs(b, n, h, dk, seed=0):
    q, k, v, beta, h0 = scan_inputs(b, n, h, dk, seed)
    return [t.to(GPU, BF16) for t in (q, k, v, beta)] + [h0.to(GPU)]


def _fp32_inputs(b, n, h, dk, seed=0):
    q, k, v, beta, h0 = scan_inputs(b, n, h, dk, seed)
    q, k, v, beta = (t.to(BF16).float() for t in (q, k, v, beta))
    g = torch.Generator().manual_seed(seed + 100)  # values the bf16 grid cannot hold
    q = q + 1e-3 * torch.randn(q.shape, generator=g)
    k = normalize_keys(k + 1e-3 * torch.randn(k.shape, generator=g))
    v = v + 1e-3 * torch.randn(v.shape, generator=g)
    return [t.to(GPU) for t in (q, k, v, beta, h0)]


def _oracle(q, k, v, beta, h0, active=None):
    cpu = [t.detach().double().cpu() for t in (q, k, v, beta, h0)]
    return delta_scan_chunked(*cpu, block=64, active=None if active is None else active.cpu())


@pytest.mark.parametrize(("b", "n", "h", "dk"), SIZES)
def test_bf16_forward_and_state_match_the_oracle(b, n, h, dk):
    from vesper.kernels.delta_scan import delta_scan_fused

    q, k, v, beta, h0 = _bf16_inputs(b, n, h, dk)
    o_ref, s_ref = _oracle(q, k, v, beta, h0)
    o, s = delta_scan_fused(q, k, v, beta, h0)
    torch.cuda.synchronize()
    assert o.dtype == BF16 and s.dtype == torch.float32
    assert relative_error(o, o_ref) < TOL
    assert relative_error(s, s_ref) < TOL


@pytest.mark.parametrize(("b", "n", "h", "dk"), SIZES)
def test_fp32_forward_and_state_match_the_oracle(b, n, h, dk):
    from vesper.kernels.delta_scan import delta_scan_fused_fp32

    q, k, v, beta, h0 = _fp32_inputs(b, n, h, dk)
    o_ref, s_ref = _oracle(q, k, v, beta, h0)
    o, s = delta_scan_fused_fp32(q, k, v, beta, h0)
    torch.cuda.synchronize()
    assert (o.dtype, s.dtype) == (torch.float32, torch.float32)
    assert relative_error(o, o_ref) < TOL_FP32
    assert relative_error(s, s_ref) < TOL_FP32


@pytest.mark.parametrize("dk", [8, 16, 24, 32, 48, 64, 100, 128, 192, 256])
@pytest.mark.parametrize("n", [5, 70])
def test_every_head_width_up_to_the_bound(dk, n):
    # chunked widths (16/32/64/128) and the token-serial kernel for the rest
    from vesper.kernels.delta_scan import delta_scan_fused, delta_scan_fused_fp32

    q, k, v, beta, h0 = _fp32_inputs(2, n, 2, dk, seed=dk)
    o_ref, s_ref = _oracle(q, k, v, beta, h0)
    o, s = delta_scan_fused_fp32(q, k, v, beta, h0)
    assert relative_error(o, o_ref) < TOL_FP32 and relative_error(s, s_ref) < TOL_FP32
    qb, kb, vb, bb, h0b = _bf16_inputs(2, n, 2, dk, seed=dk)
    o_ref, s_ref = _oracle(qb, kb, vb, bb, h0b)
    o, s = delta_scan_fused(qb, kb, vb, bb, h0b)
    assert relative_error(o, o_ref) < TOL and relative_error(s, s_ref) < TOL


def test_parity_config_fp32_b2_t512_h4_d64_zero_state():
    # B=2, T=512, H=4, d=64, chunk 64, q and k L2-normalised, zero initial state
    from vesper.kernels.delta_scan import delta_scan_fused_fp32

    g = torch.Generator().manual_seed(0)
    q = normalize_keys(torch.randn(2, 512, 4, 64, generator=g))
    k = normalize_keys(torch.randn(2, 512, 4, 64, generator=g))
    v = torch.randn(2, 512, 4, 64, generator=g)
    beta = torch.sigmoid(torch.randn(2, 512, 4, generator=g))
    h0 = torch.zeros(2, 4, 64, 64)
    o_ref, s_ref = delta_scan_chunked(*(t.double() for t in (q, k, v, beta, h0)), block=64)
    o, s = delta_scan_fused_fp32(*(t.to(GPU) for t in (q, k, v, beta, h0)))
    assert relative_error(o, o_ref) < 1e-5
    assert relative_error(s, s_ref) < 1e-5


def test_prefill_config_bf16_b8_t4096_h8_d64_full_size():
    # the headline prefill shape with a nonzero initial state S0 ~ N(0, 0.02^2)
    from vesper.kernels.delta_scan import delta_scan_fused

    g = torch.Generator().manual_seed(0)
    q = normalize_keys(torch.randn(8, 4096, 8, 64, generator=g)).to(BF16)
    k = normalize_keys(torch.randn(8, 4096, 8, 64, generator=g)).to(BF16)
    v = torch.randn(8, 4096, 8, 64, generator=g).to(BF16)
    beta = torch.sigmoid(torch.randn(8, 4096, 8, generator=g)).to(BF16)
    h0 = 0.02 * torch.randn(8, 8, 64, 64, generator=g)
    o, s = delta_scan_fused(*(t.to(GPU) for t in (q, k, v, beta, h0)))
    o_ref, s_ref = delta_scan_chunked(*(t.float() for t in (q, k, v, beta, h0)), block=64)
    assert relative_error(o, o_ref) < 2e-2
    assert relative_error(s, s_ref) < 2e-2


def test_a_carried_state_continues_the_sequence():
    # 130 tokens at once against 50 then 80: the split falls inside a 64-token chunk
    from vesper.kernels.delta_scan import delta_scan_fused, delta_scan_fused_fp32

    for fn, make, tol in ((delta_scan_fused, _bf16_inputs, TOL), (delta_scan_fused_fp32, _fp32_inputs, TOL_FP32)):
        q, k, v, beta, h0 = make(2, 130, 3, 16)
        o_ref, s_ref = _oracle(q, k, v, beta, h0)
        oa, sa = fn(q[:, :50], k[:, :50], v[:, :50], beta[:, :50], h0)
        ob, sb = fn(q[:, 50:], k[:, 50:], v[:, 50:], beta[:, 50:], sa)
        assert relative_error(torch.cat([oa, ob], 1), o_ref) < tol
        assert relative_error(sb, s_ref) < tol


def test_no_tokens_return_the_state_unchanged():
    from vesper.kernels.delta_scan import delta_scan_fused, delta_scan_fused_fp32

    q, k, v, beta, h0 = _bf16_inputs(2, 0, 3, 16)
    o, s = delta_scan_fused(q, k, v, beta, h0)
    assert o.shape == (2, 0, 3, 16) and s is h0
    q, k, v, beta, h0 = _fp32_inputs(2, 0, 3, 16)
    o, s = delta_scan_fused_fp32(q, k, v, beta, h0)
    assert o is q and s is h0


def test_beta_one_with_the_key_as_query_reads_back_the_value_at_full_size():
    # the delta rule's defining overwrite (reference tests/test_recurrence.py:48-56): with beta = 1,
    # reading k right after writing (k, v) returns v whatever the state held, so o = v at every
    # token of B8 T4096 H8 d64 (bf16 keys hold k.k = 1 only to their rounding, about 4e-3)
    from vesper.kernels.delta_scan import delta_scan_fused, delta_scan_fused_fp32

    _, k, v, beta, h0 = scan_inputs(8, 4096, 8, 64, seed=9)
    k = normalize_keys(k)
    ones = torch.ones_like(beta)
    for fn, dtype, tol in ((delta_scan_fused, BF16, TOL), (delta_scan_fused_fp32, torch.float32, 1e-5)):
        kd, vd = k.to(GPU, dtype), v.to(GPU, dtype)
        o, _ = fn(kd, kd, vd, ones.to(GPU, dtype), h0.to(GPU))
        assert relative_error(o, vd) < tol, (dtype, relative_error(o, vd))


def test_causality_holds_bitwise_at_full_size():
    # later inputs never reach earlier outputs (the reference's causality property,
    # tests/test_recurrence.py:30-104): inputs changed from token p on (inside a chunk) leave every
    # output before p unchanged bit for bit, on both scan kernels at B8 T4096 H8 d64
    from vesper.kernels.delta_scan import delta_scan_fused, delta_scan_fused_fp32

    p = 2021
    for fn, inputs in ((delta_scan_fused, _bf16_inputs(8, 4096, 8, 64, seed=21)),
                       (delta_scan_fused_fp32, _fp32_inputs(8, 4096, 8, 64, seed=21))):
        o, s = fn(*inputs)
        q, k, v, beta, h0 = (t.clone() for t in inputs)
        g = torch.Generator().manual_seed(22)
        v[:, p:] += torch.randn(v[:, p:].shape, generator=g).to(GPU, v.dtype)
        q[:, p:] = -q[:, p:]
        beta[:, p:] = 1 - beta[:, p:]
        o2, s2 = fn(q, k, v, beta, h0)
        assert torch.equal(o2[:, :p], o[:, :p]) and not torch.equal(o2[:, p:], o[:, p:])
        assert not torch.equal(s2, s)


def test_refuses_what_the_contract_excludes():
    from vesper.contracts import ContractError
    from vesper.kernels.delta_scan import delta_scan_fused, delta_scan_fused_fp32

    q, k, v, beta, h0 = _bf16_inputs(1, 8, 2, 16)
    with pytest.raises(ContractError, match="dtype"):
        delta_scan_fused(q.float(), k, v, beta, h0)
    with pytest.raises(ContractError, match="dtype"):
        delta_scan_fused(q, k, v, beta, h0.to(BF16))
    with pytest.raises(ContractError, match="axis"):
        delta_scan_fused(q, k[:, :4], v, beta, h0)
    with pytest.raises(ContractError, match="is on cpu"):
        delta_scan_fused(q, k, v, beta, h0.cpu())
    wide = torch.zeros(1, 8, 1, 512, dtype=BF16, device=GPU)
    with pytest.raises(ContractError, match="exceeds"):
        delta_scan_fused(wide, wide, wide, torch.zeros(1, 8, 1, dtype=BF16, device=GPU),
                         torch.zeros(1, 1, 512, 512, device=GPU))
    with pytest.raises(ContractError, match="dtype"):
        delta_scan_fused_fp32(q, k, v, beta, h0)
    f = torch.zeros(1, 8, 1, 264, device=GPU)
    with pytest.raises(ContractError, match="exceeds"):
        delta_scan_fused_fp32(f.clone().requires_grad_(), f, f, f[..., 0], torch.zeros(1, 1, 264, 264, device=GPU))


def test_active_mask_zeroes_outputs_and_keeps_every_write():
    from vesper.kernels.delta_scan import delta_scan_fused, delta_scan_fused_fp32

    act = torch.rand(2, 130, generator=torch.Generator().manual_seed(5)) < 0.7
    for fn, make, tol in ((delta_scan_fused, _bf16_inputs, TOL), (delta_scan_fused_fp32, _fp32_inputs, TOL_FP32)):
        q, k, v, beta, h0 = make(2, 130, 3, 64)
        o_ref, s_ref = _oracle(q, k, v, beta, h0, act)
        o, s = fn(q, k, v, beta, h0, active=act.to(GPU))
        o_all, s_all = fn(q, k, v, beta, h0)
        assert torch.equal(s, s_all)
        assert torch.equal(o[act.to(GPU)], o_all[act.to(GPU)])
        assert bool((o[~act.to(GPU)] == 0).all())
        assert relative_error(o, o_ref) < tol and relative_error(s, s_ref) < tol


# ---- the bf16 scan at head width 64 in both its forms: segmented (segments of whole-head state
# joined by their affine maps H -> X + M H) and as value-slice chains over the whole sequence ------

# (b, n, h): 16, 4, 2 and 1 segments a head (at least four chunks a segment, B H segments near 256),
# every one with a partial last chunk
SEGMENTED = [(1, 4096 - 37, 2), (3, 1000, 3), (2, 520, 1), (1, 300, 1)]


def _scan_form(segments: int, fn, *args, **kwargs):
    from vesper.kernels import _lib

    previous = _lib.set_scan_segments(segments)
    try:
        out = fn(*args, **kwargs)
        torch.cuda.synchronize()
    finally:
        _lib.set_scan_segments(previous)
    return out


@pytest.mark.parametrize("segments", [True, False])
@pytest.mark.parametrize(("b", "n", "h"), SEGMENTED)
def test_both_forms_of_the_bf16_scan_match_the_oracle(segments, b, n, h):
    from vesper.kernels.delta_scan import delta_scan_fused

    q, k, v, beta, h0 = _bf16_inputs(b, n, h, 64, seed=n)
    o_ref, s_ref = _oracle(q, k, v, beta, h0)
    o, s = _scan_form(segments, delta_scan_fused, q, k, v, beta, h0)
    assert relative_error(o, o_ref) < TOL and relative_error(s, s_ref) < TOL


@pytest.mark.parametrize(("b", "n", "h"), [(16, 700, 8), (8, 200, 8)])
def test_the_form_picked_by_shape_matches_the_oracle(b, n, h):
    # B H = 128 takes the segments (two of six chunks at n = 700), B H = 64 the value-slice chains
    from vesper.kernels.delta_scan import delta_scan_fused

    q, k, v, beta, h0 = _bf16_inputs(b, n, h, 64, seed=b)
    o_ref, s_ref = _oracle(q, k, v, beta, h0)
    o, s = _scan_form(2, delta_scan_fused, q, k, v, beta, h0)
    assert relative_error(o, o_ref) < TOL and relative_error(s, s_ref) < TOL


@pytest.mark.parametrize(("b", "n", "h"), SEGMENTED[:2])
def test_the_segmented_scan_with_an_active_mask(b, n, h):
    from vesper.kernels.delta_scan import delta_scan_fused

    q, k, v, beta, h0 = _bf16_inputs(b, n, h, 64, seed=n + 1)
    act = torch.rand(b, n, generator=torch.Generator().manual_seed(n)) < 0.6
    o_ref, s_ref = _oracle(q, k, v, beta, h0, act)
    o, s = _scan_form(True, delta_scan_fused, q, k, v, beta, h0, active=act.to(GPU))
    o_all, s_all = _scan_form(True, delta_scan_fused, q, k, v, beta, h0)
    assert torch.equal(s, s_all) and torch.equal(o[act.to(GPU)], o_all[act.to(GPU)])
    assert bool((o[~act.to(GPU)] == 0).all())
    assert relative_error(o, o_ref) < TOL and relative_error(s, s_ref) < TOL


def test_the_segmented_scan_writes_the_final_state_over_the_initial_one():
    """state_out may alias state_in (include/vesper_kernels.h): with sixteen segments the last one
    writes the final state while the first starts from a copy of S0, so the result is the one with
    separate buffers, bit for bit."""
    from vesper.kernels import _lib

    previous = _lib.set_scan_segments(1)
    try:
        _in_place_case()
    finally:
        _lib.set_scan_segments(previous)


def _in_place_case():
    from vesper.kernels import _lib

    b, n, h, dk = 1, 4096, 2, 64
    q, k, v, beta, h0 = _bf16_inputs(b, n, h, dk, seed=3)
    lib = _lib.library()
    wbytes = int(lib.vsp_delta_scan_workspace_bytes(b, n, h, dk, 0))
    ws = torch.empty(wbytes, dtype=torch.uint8, device=GPU)
    o1, s1 = torch.empty_like(q), torch.empty_like(h0)
    _lib.call("vsp_delta_scan_bf16", *(_lib.ptr(t) for t in (q, k, v, beta, h0, o1, s1, ws)), wbytes, None, b, n, h,
              dk, _lib.stream_of(GPU))
    s2 = h0.clone()
    o2 = torch.empty_like(q)
    _lib.call("vsp_delta_scan_bf16", *(_lib.ptr(t) for t in (q, k, v, beta, s2, o2, s2, ws)), wbytes, None, b, n, h,
              dk, _lib.stream_of(GPU))
    torch.cuda.synchronize()
    assert torch.equal(o1, o2) and torch.equal(s1, s2)
    o_ref, s_ref = _oracle(q, k, v, beta, h0)
    assert relative_error(o1, o_ref) < TOL and relative_error(s1, s_ref) < TOL


def test_the_segmented_records_hold_each_chunks_starting_state():
    """Records over ten chunks in two segments of five: the second segment's states come from the
    first one's map."""
    b, n, h, dk = 1, 600, 2, 64
    q, k, v, beta, h0 = _bf16_inputs(b, n, h, dk, seed=11)
    o, s, rec = _scan_form(True, _record_forward, q, k, v, beta, h0)
    nc = (n + 63) // 64
    states = _unpack_records(rec, b, h, nc, dk)
    assert torch.equal(states[:, :, 0], h0.cpu().to(BF16).float())
    for c in range(1, nc):
        _, want = _oracle(q[:, : 64 * c], k[:, : 64 * c], v[:, : 64 * c], beta[:, : 64 * c], h0)
        assert relative_error(states[:, :, c], want) < 1e-2, c
    o_ref, s_ref = _oracle(q, k, v, beta, h0)
    assert relative_error(o, o_ref) < TOL and relative_error(s, s_ref) < TOL


@pytest.mark.parametrize("dtype", [torch.float32, BF16])
@pytest.mark.parametrize("dk", [16, 32, 48, 64, 100, 128, 256])
def test_the_decode_step_matches_the_oracle_step(dtype, dk):
    from vesper.kernels.delta_scan import delta_scan_step_fused

    g = torch.Generator().manual_seed(dk)
    b, h = 5, 3
    q = torch.randn(b, h, dk, generator=g).to(dtype)
    k = normalize_keys(torch.randn(b, h, dk, generator=g)).to(dtype)
    v = torch.randn(b, h, dk, generator=g).to(dtype)
    beta = torch.sigmoid(torch.randn(b, h, generator=g)).to(dtype)
    s0 = 0.5 * torch.randn(b, h, dk, dk, generator=g)
    o_ref, s_ref = delta_scan_step(*(t.double() for t in (q, k, v, beta, s0)))
    dev = [t.to(GPU) for t in (q, k, v, beta, s0)]
    o, s = delta_scan_step_fused(*dev)
    tol = 1e-6 if dtype == torch.float32 else 1e-2
    assert relative_error(o, o_ref) < tol and relative_error(s, s_ref) < 1e-6
    # in place: the new state overwrites the old one
    state = dev[4].clone()
    o2, s2 = delta_scan_step_fused(*dev[:4], state, out_state=state)
    assert s2 is state and torch.equal(state, s) and torch.equal(o2, o)
    act = torch.tensor([True, False, True, True, False], device=GPU)
    o3, s3 = delta_scan_step_fused(*dev, active=act)
    assert torch.equal(s3, s) and bool((o3[~act] == 0).all()) and torch.equal(o3[act], o[act])


def test_decode_config_256_steps_b64_h8_d64_equal_the_chunked_scan():
    # the decode workload: 256 in-place fp32 steps on S [64, 8, 64, 64] ~ N(0, 0.02^2) give the
    # outputs and final state of one chunked scan over the same 256 tokens (tests/test_decode.py:45-71)
    from vesper.kernels.delta_scan import delta_scan_step_fused

    b, n, h, dk = 64, 256, 8, 64
    g = torch.Generator().manual_seed(4)
    q = normalize_keys(torch.randn(b, n, h, dk, generator=g))
    k = normalize_keys(torch.randn(b, n, h, dk, generator=g))
    v = torch.randn(b, n, h, dk, generator=g)
    beta = torch.sigmoid(torch.randn(b, n, h, generator=g))
    s0 = 0.02 * torch.randn(b, h, dk, dk, generator=g)
    o_ref, s_ref = delta_scan_chunked(*(t.double() for t in (q, k, v, beta, s0)), 64)
    dq, dk_, dv, db = (t.to(GPU) for t in (q, k, v, beta))
    state = s0.to(GPU)
    outs = []
    for t in range(n):
        o, _ = delta_scan_step_fused(dq[:, t], dk_[:, t], dv[:, t], db[:, t], state, out_state=state)
        outs.append(o)
    o = torch.stack(outs, dim=1)
    assert relative_error(o, o_ref) < 1e-5 and relative_error(state, s_ref) < 1e-5


def test_bitwise_repeatable_and_exactly_linear_under_power_of_two_scaling():
    # a size-independent property at the headline width: doubling v and S0 doubles o and S_n
    # exactly (every rounding is scale-invariant under a power of two), and reruns are bitwise
    from vesper.kernels.delta_scan import delta_scan_fused

    q, k, v, beta, h0 = _bf16_inputs(2, 1000, 8, 64, seed=3)
    o1, s1 = delta_scan_fused(q, k, v, beta, h0)
    o2, s2 = delta_scan_fused(q, k, v, beta, h0)
    assert torch.equal(o1, o2) and torch.equal(s1, s2)
    o3, s3 = delta_scan_fused(q, k, 2 * v, beta, 2 * h0)
    assert torch.equal(o3, 2 * o1) and torch.equal(s3, 2 * s1)


def test_graph_replays_equal_the_eager_result():
    from vesper.kernels.delta_scan import delta_scan_fused

    q, k, v, beta, h0 = _bf16_inputs(2, 300, 4, 64, seed=9)
    eager_o, eager_s = delta_scan_fused(q, k, v, beta, h0)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            delta_scan_fused(q, k, v, beta, h0)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        got_o, got_s = delta_scan_fused(q, k, v, beta, h0)
    for i in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(got_o, eager_o), i
        assert torch.equal(got_s, eager_s), i
        _ = delta_scan_fused(q, k, v, beta, h0)  # eager work between replays
        torch.cuda.synchronize()


def _grad_check(fn, inputs, tol, active=None, with_state_grad=True):
    g = torch.Generator().manual_seed(7)
    b, n, h, dk = inputs[0].shape
    d_o = torch.randn(b, n, h, dk, generator=g)
    d_s = torch.randn(b, h, dk, dk, generator=g)
    ref_in = [t.cpu().double().requires_grad_() for t in inputs]
    o_ref, s_ref = delta_scan_chunked(*ref_in, 64, active=active)
    loss = (o_ref * d_o.double()).sum() + ((s_ref * d_s.double()).sum() if with_state_grad else 0)
    torch.autograd.backward([loss])
    fused_in = [t.clone().requires_grad_() for t in inputs]
    o, s = fn(*fused_in, active=None if active is None else active.to(GPU))
    loss = (o.float() * d_o.to(GPU)).sum() + ((s * d_s.to(GPU)).sum() if with_state_grad else 0)
    torch.autograd.backward([loss])
    for name, got, want in zip(["q", "k", "v", "beta", "state"], fused_in, ref_in):
        assert got.grad is not None, name
        assert relative_error(got.grad, want.grad) < tol, (name, relative_error(got.grad, want.grad))
    return fused_in


@pytest.mark.parametrize(("b", "n", "h", "dk"), SIZES[:4])
def test_every_gradient_matches_the_oracle(b, n, h, dk):
    from vesper.kernels.delta_scan import delta_scan_fused

    _grad_check(delta_scan_fused, _bf16_inputs(b, n, h, dk), TOL)


@pytest.mark.parametrize("dk", [32, 64])
def test_bf16_gradients_over_several_chunks_with_an_active_mask(dk):
    # five chunks (the last one partial), three heads: the chains' hand-over from chunk to chunk
    # in both directions, at the widths of the bf16 tile kernels
    from vesper.kernels.delta_scan import delta_scan_fused

    act = torch.rand(2, 300, generator=torch.Generator().manual_seed(11)) < 0.7
    _grad_check(delta_scan_fused, _bf16_inputs(2, 300, 3, dk, seed=dk), TOL, active=act)


def test_bf16_gradients_at_width_128_over_several_chunks_with_an_active_mask():
    # width 128: the chunk kernel reads the states' fragments from the chains' records (both
    # orientations) instead of LDS tiles
    from vesper.kernels.delta_scan import delta_scan_fused

    act = torch.rand(1, 200, generator=torch.Generator().manual_seed(12)) < 0.7
    _grad_check(delta_scan_fused, _bf16_inputs(1, 200, 2, 128, seed=128), TOL, active=act)


@pytest.mark.parametrize(("dk", "fp32"), [(48, False), (100, False), (24, True), (48, True)])
def test_gradients_at_widths_the_kernels_take_zero_padded(dk, fp32):
    # a width between the kernels' (16, 32, 64, 128 on the bf16 entry; up to 64 on the fp32 one)
    # runs padded with zero features and value columns: the same outputs and gradients
    from vesper.kernels.delta_scan import delta_scan_fused, delta_scan_fused_fp32

    fn, make, tol = (delta_scan_fused_fp32, _fp32_inputs, TOL_FP32) if fp32 else (delta_scan_fused, _bf16_inputs, TOL)
    _grad_check(fn, make(2, 130, 2, dk, seed=dk), tol)


@pytest.mark.parametrize(("dk", "fp32"), [(192, False), (200, False), (256, False), (80, True), (128, True),
                                         (256, True)])
def test_gradients_of_heads_wider_than_the_tiled_kernels(dk, fp32):
    # the wide backward (chunk-start states checkpointed by the token-serial forward, value groups
    # of 64, 32 or 16 columns, partial sums added in a fixed order): three chunks, the last partial,
    # with an active mask; 200 runs zero-padded to 208 (value groups of 16)
    from vesper.kernels.delta_scan import backward_width, delta_scan_fused, delta_scan_fused_fp32

    assert backward_width(dk, fp32) == (208 if dk == 200 else dk)
    fn, make, tol = (delta_scan_fused_fp32, _fp32_inputs, TOL_FP32) if fp32 else (delta_scan_fused, _bf16_inputs, TOL)
    act = torch.rand(2, 150, generator=torch.Generator().manual_seed(dk)) < 0.7
    first = _grad_check(fn, make(2, 150, 2, dk, seed=dk), tol, active=act)
    # deterministic: a second backward over the same inputs gives the same bits
    again = [t.detach().clone().requires_grad_() for t in first]
    o, s = fn(*again, active=act.to(GPU))
    g = torch.Generator().manual_seed(7)
    d_o = torch.randn(o.shape, generator=g).to(GPU)
    d_s = torch.randn(s.shape, generator=g).to(GPU)
    torch.autograd.backward([(o.float() * d_o).sum() + (s * d_s).sum()])
    for name, a, b_ in zip(["q", "k", "v", "beta", "state"], first, again):
        assert torch.equal(a.grad, b_.grad), name


@pytest.mark.parametrize(("b", "n", "h", "dk"), SIZES[:4])
def test_fp32_every_gradient_matches_the_oracle_to_float32(b, n, h, dk):
    from vesper.kernels.delta_scan import delta_scan_fused_fp32

    _grad_check(delta_scan_fused_fp32, _fp32_inputs(b, n, h, dk), TOL_FP32)


# the shape the reference quotes both fused scans at (kernels/delta_scan.py:22-24, "stage-1 size":
# b 32, n 88, h 2, dk 16), forward and every gradient against the float64 oracle; the reference
# reports about 2e-7 relative for its fp32 scan there
def test_the_reference_benchmark_shape_b32_n88_h2_d16():
    from vesper.kernels.delta_scan import delta_scan_fused, delta_scan_fused_fp32

    for fn, inputs, tol in ((delta_scan_fused, _bf16_inputs(32, 88, 2, 16, seed=88), TOL),
                            (delta_scan_fused_fp32, _fp32_inputs(32, 88, 2, 16, seed=88), TOL_FP32)):
        o, s = fn(*inputs)
        o_ref, s_ref = _oracle(*inputs)
        assert relative_error(o, o_ref) < tol and relative_error(s, s_ref) < tol
        _grad_check(fn, inputs, tol)


@pytest.mark.parametrize("dk", [16, 32, 64])
def test_gradients_with_an_active_mask_and_every_width(dk):
    from vesper.kernels.delta_scan import delta_scan_fused_fp32

    act = torch.rand(2, 150, generator=torch.Generator().manual_seed(8)) < 0.6
    _grad_check(delta_scan_fused_fp32, _fp32_inputs(2, 150, 2, dk, seed=dk), TOL_FP32, active=act)


def test_fp32_gradients_flow_from_a_state_that_needs_none():
    # tests/test_delta_scan_fused.py:303-323: a cold or detached state does not require a gradient
    from vesper.kernels.delta_scan import delta_scan_fused_fp32

    q, k, v, beta, h0 = _fp32_inputs(2, 63, 3, 16)
    ref_in = [t.cpu().double().requires_grad_() for t in (q, k, v, beta)]
    o_ref, _ = delta_scan_chunked(*ref_in, h0.cpu().double(), 64)
    torch.autograd.backward([o_ref.square().sum()])
    fused_in = [t.clone().requires_grad_() for t in (q, k, v, beta)]
    state = h0.clone()
    o, _ = delta_scan_fused_fp32(*fused_in, state)
    torch.autograd.backward([o.square().sum()])
    assert not state.requires_grad and state.grad is None
    for name, got, want in zip(["q", "k", "v", "beta"], fused_in, ref_in):
        assert relative_error(got.grad, want.grad) < TOL_FP32, name


def test_the_gradients_at_b8_t4096_h8_d64_and_they_repeat():
    from vesper.kernels.delta_scan import delta_scan_fused

    inputs = _bf16_inputs(8, 4096, 8, 64, seed=3)
    g = torch.Generator().manual_seed(9)
    d_o = torch.randn(8, 4096, 8, 64, generator=g).to(GPU, BF16)

    def run():
        ins = [t.clone().requires_grad_() for t in inputs]
        o, _ = delta_scan_fused(*ins)
        o.backward(d_o)
        return [t.grad for t in ins]

    first, again = run(), run()
    for a, c in zip(first, again):
        assert torch.equal(a, c)  # deterministic: no atomics
    ref_in = [t.cpu().float().requires_grad_() for t in inputs]
    o_ref, _ = delta_scan_chunked(*ref_in, 64)
    o_ref.backward(d_o.cpu().float())
    for name, got, want in zip(["q", "k", "v", "beta", "state"], first, ref_in):
        assert relative_error(got, want.grad) < TOL, name


def test_captured_forward_and_backward_equal_eager():
    from vesper.kernels.delta_scan import delta_scan_fused

    q, k, v, beta, h0 = (t.requires_grad_() for t in _bf16_inputs(2, 200, 2, 64, seed=4))
    d_o = torch.randn(2, 200, 2, 64, generator=torch.Generator().manual_seed(10)).to(GPU, BF16)

    def step():
        o, s = delta_scan_fused(q, k, v, beta, h0)
        return (o.detach(), s.detach(), *torch.autograd.grad(o, (q, k, v, beta, h0), d_o))

    eager = [t.clone() for t in step()]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        static = step()
    for _ in range(3):
        for t in static:
            t.zero_()
        graph.replay()
        torch.cuda.synchronize()
        for a, c in zip(static, eager):
            assert torch.equal(a, c)


# ---- copy-forward read inside the kernels' loads (carried k, v, beta for inactive tokens) ----

def _carry_case(b, n, h, dk, fp32, seed, frac=0.4):
    make = _fp32_inputs if fp32 else _bf16_inputs
    q, k, v, beta, h0 = make(b, n, h, dk, seed)
    _, kc, vc, bc, _ = make(b, n, h, dk, seed + 7)
    g = torch.Generator().manual_seed(seed + 11)
    active = (torch.rand(b, n, generator=g) >= frac).to(GPU)
    return q, k, v, beta, h0, (kc, vc, bc), active


def _merged(k, v, beta, carried, active):
    keep = active[..., None, None]
    return (torch.where(keep, k, carried[0]), torch.where(keep, v, carried[1]),
            torch.where(active[..., None], beta, carried[2]))


# widths 16 and 128 take the generic chain (the fp32 entry runs 128 token by token), 32 and 64 the bf16
# chain, 48 and n = 9 the serial kernel
@pytest.mark.parametrize("fp32", [False, True])
@pytest.mark.parametrize(("b", "n", "h", "dk"), [(2, 9, 2, 16), (2, 70, 2, 48), (2, 130, 3, 16), (2, 200, 2, 32),
                                                 (1, 300, 2, 64), (2, 100, 2, 128)])
def test_carried_inputs_equal_the_merged_inputs_bitwise(fp32, b, n, h, dk):
    from vesper.kernels.delta_scan import delta_scan_fused, delta_scan_fused_fp32

    scan = delta_scan_fused_fp32 if fp32 else delta_scan_fused
    q, k, v, beta, h0, carried, active = _carry_case(b, n, h, dk, fp32, seed=dk + n)
    # the fresh rows of inactive tokens must never be read: poison them
    hold = ~active
    k, v = k.masked_fill(hold[..., None, None], float("nan")), v.masked_fill(hold[..., None, None], float("nan"))
    beta = beta.masked_fill(hold[..., None], float("nan"))
    o, s = scan(q, k, v, beta, h0, active=active, carried=carried)
    o_ref, s_ref = scan(q, *_merged(k, v, beta, carried, active), h0, active=active)
    torch.cuda.synchronize()
    assert torch.equal(o, o_ref) and torch.equal(s, s_ref)
    assert bool(torch.isfinite(s).all())


@pytest.mark.parametrize("pattern", ["all_active", "all_held", "alternating", "tail_held"])
def test_carried_inputs_on_every_flag_pattern_of_a_chunk(pattern):
    from vesper.kernels.delta_scan import delta_scan_fused

    b, n, h, dk = 2, 190, 2, 64
    q, k, v, beta, h0, carried, _ = _carry_case(b, n, h, dk, False, seed=3)
    t = torch.arange(n, device=GPU).expand(b, n)
    active = {"all_active": t >= 0, "all_held": t < 0, "alternating": t % 2 == 0, "tail_held": t < 150}[pattern]
    o, s = delta_scan_fused(q, k, v, beta, h0, active=active, carried=carried)
    o_ref, s_ref = delta_scan_fused(q, *_merged(k, v, beta, carried, active), h0, active=active)
    torch.cuda.synchronize()
    assert torch.equal(o, o_ref) and torch.equal(s, s_ref)
    want, s64 = _oracle(q, *_merged(k, v, beta, carried, active), h0, active=active)
    assert relative_error(s, s64) < TOL


def test_carried_inputs_at_b8_t4096_h8_d64():
    from vesper.kernels.delta_scan import delta_scan_fused

    q, k, v, beta, h0, carried, active = _carry_case(8, 4096, 8, 64, False, seed=5, frac=0.3)
    o, s = delta_scan_fused(q, k, v, beta, h0, active=active, carried=carried)
    o_ref, s_ref = delta_scan_fused(q, *_merged(k, v, beta, carried, active), h0, active=active)
    torch.cuda.synchronize()
    assert torch.equal(o, o_ref) and torch.equal(s, s_ref)


def test_carried_inputs_under_autograd_route_gradients_to_the_carried_tensors():
    from vesper.kernels.delta_scan import delta_scan_fused

    q, k, v, beta, h0, carried, active = _carry_case(2, 100, 2, 32, False, seed=9)
    leaves = [t.clone().requires_grad_() for t in (k, v, beta, *carried)]
    o, s = delta_scan_fused(q, *leaves[:3], h0, active=active, carried=tuple(leaves[3:]))
    (o.float().square().sum() + s.square().sum()).backward()
    ref = [t.clone().requires_grad_() for t in (k, v, beta, *carried)]
    o2, s2 = delta_scan_fused(q, *_merged(*ref[:3], tuple(ref[3:]), active), h0, active=active)
    (o2.float().square().sum() + s2.square().sum()).backward()
    for got, want in zip(leaves, ref):
        assert torch.equal(got.grad, want.grad)
    assert not bool(leaves[0].grad[~active].any()) and not bool(leaves[3].grad[active].any())


def test_carried_refusals():
    from vesper.contracts import ContractError
    from vesper.kernels.delta_scan import delta_scan_fused

    q, k, v, beta, h0, carried, active = _carry_case(1, 20, 2, 16, False, seed=1)
    with pytest.raises(ContractError, match="active"):
        delta_scan_fused(q, k, v, beta, h0, carried=carried)
    with pytest.raises(ContractError, match="carried k"):
        delta_scan_fused(q, k, v, beta, h0, active=active, carried=(carried[0].float(), *carried[1:]))
    with pytest.raises(ContractError, match="carried holds"):
        delta_scan_fused(q, k, v, beta, h0, active=active, carried=carried[:2])


def test_a_wait_that_gives_up_is_recorded_and_refused_and_its_outputs_are_nan():
    """The chain's bounded hand-over waits, made to give up from the host (a limit of 0 polls): the
    kernel still runs to its end, the fault record says so, every later call raises until the record
    is cleared, and the broken workgroups' outputs are NaN; with the default limit the next call is
    right again."""
    from vesper.kernels import _lib
    from vesper.kernels.delta_scan import delta_scan_fused

    q, k, v, beta, h0 = _bf16_inputs(1, 4096, 2, 64)
    _lib.check_faults(synchronize=True)
    previous = _lib.set_wait_limit(0)
    try:
        o, s = delta_scan_fused(q, k, v, beta, h0)
        torch.cuda.synchronize()
    finally:
        _lib.set_wait_limit(previous)
    try:
        with pytest.raises(_lib.KernelLibraryError, match="bounded wait gave up"):
            _lib.check_faults()
        with pytest.raises(_lib.KernelLibraryError, match="bounded wait gave up"):
            delta_scan_fused(q, k, v, beta, h0)
        assert bool(torch.isnan(s).any()) or bool(torch.isnan(o.float()).any())
    finally:
        _lib.clear_faults()
    o, s = delta_scan_fused(q, k, v, beta, h0)
    _lib.check_faults(synchronize=True)
    o_ref, s_ref = _oracle(q, k, v, beta, h0)
    assert relative_error(o, o_ref) < TOL and relative_error(s, s_ref) < TOL


# ---- the write strength (recurrence.py:34-88): alone, and inside the scan's beta loads ----------

def _modulator(b, n, seed, alpha=0.5):
    g = torch.Generator().manual_seed(seed)
    m = torch.rand(b, n, generator=g) * 4 - 1  # [-1, 3]: 1 + alpha m in [0.5, 2.5]
    m[0, :3] = -1.0 / alpha  # factor exactly zero: an exact zero write
    return m


@pytest.mark.parametrize("dtype", [torch.float32, BF16])
def test_the_write_strength_matches_the_oracle_and_the_reference_vectors(dtype):
    from conftest import frac_tensor, reference_vectors
    from oracle.delta import write_strength as oracle_strength
    from vesper.kernels.delta_scan import write_strength

    g = torch.Generator().manual_seed(4)
    logits = (3 * torch.randn(3, 50, 4, generator=g)).to(dtype)
    tol = 1e-6 if dtype == torch.float32 else 2 ** -8
    got = write_strength(logits.to(GPU))
    torch.testing.assert_close(got.cpu().double(), oracle_strength(logits.double()), rtol=tol, atol=1e-7)
    m = _modulator(3, 50, 5)
    got = write_strength(logits.to(GPU), m.to(GPU), 0.5)
    want = oracle_strength(logits.double(), m.double(), 0.5)
    torch.testing.assert_close(got.cpu().double(), want, rtol=tol, atol=1e-7)
    assert bool((got[0, :3] == 0).all())  # exact zeros where 1 + alpha m = 0
    c = reference_vectors()["write_strength"]
    ends = write_strength(frac_tensor(c["logits"], torch.float32).to(GPU))
    assert torch.equal(ends.cpu(), frac_tensor(c["want"], torch.float32))
    o = c["odds_case"]
    beta0 = float(frac_tensor([o["beta"]])[0])
    logit = torch.tensor([[[math.log(beta0 / (1 - beta0))]]], dtype=torch.float32)
    odds = write_strength(logit.to(GPU), torch.tensor([[float(frac_tensor([o["m"]])[0])]], device=GPU),
                          float(frac_tensor([o["alpha"]])[0]))
    assert abs(float(odds) - float(frac_tensor([o["want"]])[0])) < 1e-6


def test_the_write_strength_refusals_and_gradients():
    from oracle.delta import write_strength as oracle_strength
    from vesper.kernels.delta_scan import write_strength

    logits = torch.randn(2, 6, 3, device=GPU)
    m = torch.rand(2, 6, device=GPU)
    with pytest.raises(ValueError, match="alpha must be given"):
        write_strength(logits, m)
    with pytest.raises(ValueError, match="non-negative"):
        write_strength(logits, m, -0.5)
    with pytest.raises(ValueError, match="must not be negative"):
        write_strength(logits, m - 3.0, 1.0)
    g = torch.Generator().manual_seed(6)
    lg = torch.randn(2, 9, 3, generator=g, dtype=torch.float64)
    mm = _modulator(2, 9, 7).double()
    up = torch.randn(2, 9, 3, generator=g, dtype=torch.float64)
    lg_ref, m_ref = lg.clone().requires_grad_(), mm.clone().requires_grad_()
    (oracle_strength(lg_ref, m_ref, 0.5) * up).sum().backward()
    lg_gpu, m_gpu = lg.float().to(GPU).requires_grad_(), mm.float().to(GPU).requires_grad_()
    (write_strength(lg_gpu, m_gpu, 0.5) * up.float().to(GPU)).sum().backward()
    torch.testing.assert_close(lg_gpu.grad.cpu().double(), lg_ref.grad, rtol=1e-5, atol=1e-6)
    torch.testing.assert_close(m_gpu.grad.cpu().double(), m_ref.grad, rtol=1e-5, atol=1e-6)


def test_bf16_logits_with_a_modulator_give_float32_beta_and_gradients():
    """bf16 logits plus the float32 shift ln(1 + alpha m) promote to float32 in the reference
    (recurrence.py:84-88): beta comes out float32, and its gradient is taken from the unrounded
    beta, so saturated logits (where a bf16 beta would round to 1) keep their nonzero slope."""
    from oracle.delta import write_strength as oracle_strength
    from vesper.kernels.delta_scan import write_strength

    g = torch.Generator().manual_seed(11)
    lg = (3 * torch.randn(2, 40, 3, generator=g)).to(BF16)
    # saturating logits (tokens 0-2 of row 0 have 1 + alpha m = 0, an exact zero write)
    lg[0, 3:11, 0] = torch.tensor([6.5, 7.0, 8.0, 9.0, 10.0, 12.0, 4.0, 5.5], dtype=BF16)
    mm = _modulator(2, 40, 12)
    up = torch.randn(2, 40, 3, generator=g)
    lg_ref = lg.double().requires_grad_()
    m_ref = mm.double().requires_grad_()
    want = oracle_strength(lg_ref, m_ref, 0.5)
    (want * up.double()).sum().backward()
    lg_gpu, m_gpu = lg.to(GPU).requires_grad_(), mm.to(GPU).requires_grad_()
    beta = write_strength(lg_gpu, m_gpu, 0.5)
    assert beta.dtype == torch.float32
    torch.testing.assert_close(beta.detach().cpu().double(), want.detach(), rtol=1e-6, atol=1e-7)
    (beta * up.to(GPU)).sum().backward()
    assert lg_gpu.grad.dtype == BF16
    # the logits' gradient is rounded to bf16 once (the reference casts the float32 gradient back);
    # the absolute term is an ulp of a float32 beta near 1 (~6e-8) times |up|, which 1 - beta carries
    torch.testing.assert_close(lg_gpu.grad.cpu().double(), lg_ref.grad, rtol=2 ** -8, atol=3e-7)
    assert bool((lg_gpu.grad[0, 3:11, 0] != 0).all())  # saturated logits keep a slope
    assert not bool(lg_gpu.grad[0, :3].any())  # a zero write has a zero gradient
    torch.testing.assert_close(m_gpu.grad.cpu().double(), m_ref.grad, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("fp32", [False, True])
@pytest.mark.parametrize("with_m", [False, True])
def test_the_scan_from_logits_gives_the_same_outputs_with_and_without_autograd(fp32, with_m):
    """The no-grad path computes beta inside the scan's loads, the autograd path through
    write_strength and delta_scan_fused; both round beta to the inputs' dtype, so both see the
    same beta and their forward outputs agree bitwise."""
    from vesper.kernels.delta_scan import delta_scan_fused_logits

    b, n, h, dk = 2, 200, 3, 64
    q, k, v, _, h0 = scan_inputs(b, n, h, dk, seed=13)
    logits = 2 * torch.randn(b, n, h, generator=torch.Generator().manual_seed(14))
    dtype = torch.float32 if fp32 else BF16
    q, k, v, logits = (t.to(dtype).to(GPU) for t in (q, k, v, logits))
    h0 = h0.to(GPU)
    kw = {"m": _modulator(b, n, 15).to(GPU), "alpha": 0.5} if with_m else {}
    with torch.no_grad():
        o_plain, s_plain = delta_scan_fused_logits(q, k, v, logits, h0, **kw)
    o_grad, s_grad = delta_scan_fused_logits(q, k, v, logits.clone().requires_grad_(), h0, **kw)
    assert torch.equal(o_grad.detach(), o_plain)
    assert torch.equal(s_grad.detach(), s_plain)


@pytest.mark.parametrize("fp32", [False, True])
@pytest.mark.parametrize(("b", "n", "h", "dk"), [(2, 9, 3, 64), (2, 130, 3, 64), (1, 200, 2, 16)])
def test_the_scan_with_the_write_strength_in_its_loads_matches_the_oracle(fp32, b, n, h, dk):
    from oracle.delta import write_strength as oracle_strength
    from vesper.kernels.delta_scan import delta_scan_fused_logits

    q, k, v, _, h0 = scan_inputs(b, n, h, dk, seed=8)
    logits = torch.randn(b, n, h, generator=torch.Generator().manual_seed(9))
    m = _modulator(b, n, 10)
    dtype = torch.float32 if fp32 else BF16
    q, k, v, logits = (t.to(dtype) for t in (q, k, v, logits))
    beta = oracle_strength(logits.double(), m.double(), 0.5)
    o_ref, s_ref = delta_scan_chunked(q.double(), k.double(), v.double(), beta, h0.double(), 64)
    dev = [t.to(GPU) for t in (q, k, v, logits, h0)]
    o, s = delta_scan_fused_logits(*dev, m=m.to(GPU), alpha=0.5)
    tol = TOL_FP32 if fp32 else TOL
    assert relative_error(o, o_ref) < tol and relative_error(s, s_ref) < tol
    # no modulator: beta = sigmoid(logits)
    o, s = delta_scan_fused_logits(*dev)
    o_ref, s_ref = delta_scan_chunked(q.double(), k.double(), v.double(), torch.sigmoid(logits.double()),
                                      h0.double(), 64)
    assert relative_error(o, o_ref) < tol and relative_error(s, s_ref) < tol


# ---- the forward's records of the chunks' starting states, and the backward that reads them ----

def _unpack_records(rec: torch.Tensor, b: int, h: int, nc: int, dk: int) -> torch.Tensor:
    """The records' [D x D] blocks as states [b, h, nc, D, D]: element ((s (NT/2) + rt/2) 64 + l) 8 +
    (rt % 2) 4 + r of a block is row 16 rt + 4 (l / 16) + r, column 16 s + l % 16 (NT = D / 16)."""
    nt = dk // 16
    x = rec.view(BF16).float().cpu().view(b * h * nc, nt, nt // 2, 4, 16, 2, 4)  # s, rt/2, g, j, rt%2, r
    # rows 16 (2 p + e) + 4 g + r, columns 16 s + j
    x = x.permute(0, 2, 5, 3, 6, 1, 4).reshape(b * h * nc, dk, dk)
    return x.view(b, h, nc, dk, dk)


def _record_forward(q, k, v, beta, h0):
    from vesper.kernels import _lib

    b, n, h, dk = q.shape
    lib = _lib.library()
    nbytes = int(lib.vsp_delta_scan_records_bytes(b, n, h, dk))
    wbytes = int(lib.vsp_delta_scan_workspace_bytes(b, n, h, dk, 0))
    rec = torch.empty(nbytes, dtype=torch.uint8, device=GPU)
    ws = torch.empty(wbytes, dtype=torch.uint8, device=GPU)
    o, s = torch.empty_like(q), torch.empty_like(h0)
    _lib.call("vsp_delta_scan_record_bf16", *(_lib.ptr(t) for t in (q, k, v, beta, h0, o, s, ws)), wbytes, None,
              _lib.ptr(rec), nbytes, b, n, h, dk, _lib.stream_of(GPU))
    return o, s, rec


@pytest.mark.parametrize("dk", [32, 64])
def test_the_forward_records_each_chunks_starting_state(dk):
    """The records hold the state before chunk c: the oracle's final state over the first 64 c tokens
    (the initial state itself, rounded to bf16, for chunk 0), to bf16 precision; the forward's
    outputs are the plain forward's bit for bit."""
    from vesper.kernels.delta_scan import delta_scan_fused

    b, n, h = 2, 200, 3
    q, k, v, beta, h0 = _bf16_inputs(b, n, h, dk, seed=dk + 5)
    o, s, rec = _record_forward(q, k, v, beta, h0)
    o_plain, s_plain = delta_scan_fused(q, k, v, beta, h0)
    assert torch.equal(o, o_plain) and torch.equal(s, s_plain)
    nc = (n + 63) // 64
    states = _unpack_records(rec, b, h, nc, dk)
    assert torch.equal(states[:, :, 0], h0.cpu().to(BF16).float())
    for c in range(1, nc):
        _, want = _oracle(q[:, : 64 * c], k[:, : 64 * c], v[:, : 64 * c], beta[:, : 64 * c], h0)
        assert relative_error(states[:, :, c], want) < 1e-2, c


@pytest.mark.parametrize("dk", [32, 64])
def test_the_backward_from_the_records_and_the_backward_alone_agree(dk):
    """vsp_delta_scan_backward_recorded_bf16 (the autograd path at widths 32 and 64) and
    vsp_delta_scan_backward_bf16 (which recomputes the states) on one input with an active mask: dv
    and the initial state's gradient do not read the states and are equal bit for bit; both sets of
    gradients match the oracle's."""
    from oracle.delta import delta_scan_chunked
    from vesper.kernels import _lib

    b, n, h = 2, 300, 3
    q, k, v, beta, h0 = _bf16_inputs(b, n, h, dk, seed=dk + 9)
    active = torch.rand(b, n, generator=torch.Generator().manual_seed(4)) < 0.7
    mask = active.to(GPU).view(torch.uint8)
    g = torch.Generator().manual_seed(5)
    d_o = torch.randn(b, n, h, dk, generator=g).to(BF16)
    d_s = torch.randn(b, h, dk, dk, generator=g)
    lib = _lib.library()
    nbytes = int(lib.vsp_delta_scan_records_bytes(b, n, h, dk))
    wbytes = int(lib.vsp_delta_scan_workspace_bytes(b, n, h, dk, 0))
    rec = torch.empty(nbytes, dtype=torch.uint8, device=GPU)
    ws = torch.empty(wbytes, dtype=torch.uint8, device=GPU)
    o, s = torch.empty_like(q), torch.empty_like(h0)
    _lib.call("vsp_delta_scan_record_bf16", *(_lib.ptr(t) for t in (q, k, v, beta, h0, o, s, ws)), wbytes,
              _lib.ptr(mask), _lib.ptr(rec), nbytes, b, n, h, dk, _lib.stream_of(GPU))
    go, gs = d_o.to(GPU), d_s.to(GPU)
    bbytes = int(lib.vsp_delta_scan_backward_workspace_bytes(b, n, h, dk))
    bws = torch.empty(bbytes, dtype=torch.uint8, device=GPU)
    grads = {}
    for name in ("recorded", "alone"):
        out = [torch.empty_like(t) for t in (q, k, v, beta, h0)]
        head = [_lib.ptr(t) for t in (q, k, v, beta, h0, go, gs, mask)]
        tail = [_lib.ptr(t) for t in out] + [_lib.ptr(bws), bbytes, b, n, h, dk, _lib.stream_of(GPU)]
        if name == "recorded":
            _lib.call("vsp_delta_scan_backward_recorded_bf16", *head, _lib.ptr(rec), nbytes, *tail)
        else:
            _lib.call("vsp_delta_scan_backward_bf16", *head, *tail)
        grads[name] = out
    torch.cuda.synchronize()
    assert torch.equal(grads["recorded"][2], grads["alone"][2])
    assert torch.equal(grads["recorded"][4], grads["alone"][4])
    ref_in = [t.cpu().double().requires_grad_() for t in (q, k, v, beta, h0)]
    o_ref, s_ref = delta_scan_chunked(*ref_in, 64, active=active)
    torch.autograd.backward([(o_ref * d_o.double() * active[..., None, None]).sum() + (s_ref * d_s.double()).sum()])
    for name, got in grads.items():
        for what, x, want in zip(["q", "k", "v", "beta", "state"], got, ref_in):
            assert relative_error(x, want.grad) < TOL, (name, what, relative_error(x, want.grad))


def test_record_refusals():
    from vesper.kernels import _lib
    from vesper.kernels._lib import KernelLibraryError

    lib = _lib.library()
    assert int(lib.vsp_delta_scan_records_bytes(1, 200, 2, 16)) == 0  # widths 32 and 64 only
    assert int(lib.vsp_delta_scan_records_bytes(1, 8, 2, 64)) == 0    # the serial path keeps none
    assert int(lib.vsp_delta_scan_records_bytes(1, 200, 2, 64)) == 4 * 2 * 64 * 64 * 2
    q, k, v, beta, h0 = _bf16_inputs(1, 200, 2, 16)
    o, s = torch.empty_like(q), torch.empty_like(h0)
    ws = torch.empty(int(lib.vsp_delta_scan_workspace_bytes(1, 200, 2, 16, 0)), dtype=torch.uint8, device=GPU)
    with pytest.raises(KernelLibraryError, match="no records"):
        _lib.call("vsp_delta_scan_record_bf16", *(_lib.ptr(t) for t in (q, k, v, beta, h0, o, s, ws)), ws.numel(),
                  None, _lib.ptr(ws), ws.numel(), 1, 200, 2, 16, _lib.stream_of(GPU))
