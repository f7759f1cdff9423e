"""The HIP ring attention (``vesper.kernels.ring_attn``) against the CPU oracle, through the C ABI."""

from __future__ import annotations

import pytest
import torch

from conftest import frac_tensor, needs_gpu, reference_vectors
from oracle import attention as oa
from oracle.delta import relative_error

pytestmark = [pytest.mark.gpu, needs_gpu]

GPU = torch.device("cuda")
BF16 = torch.bfloat16


def test_a_ring_attends_by_position_not_by_slot_order():
    # slots hold positions [3, 1, 2] with values [30, 10, 20]; the new token (position 4, value
    # 40) sees positions 2..4 with equal logits, so every output is 30 (tests/test_attention.py:150-172)
    from vesper.kernels.ring_attn import RingKVCache, ring_attention

    c = reference_vectors()["ring_by_position"]
    w, dk = c["window"], 16
    vals = frac_tensor(c["ring_values"]).reshape(1, w, 1, 1).expand(1, w, 1, dk).to(BF16)
    ring = RingKVCache(torch.zeros(1, w, 1, dk, dtype=BF16, device=GPU), vals.contiguous().to(GPU),
                       torch.tensor([c["ring_pos"]], device=GPU), torch.ones(1, w, dtype=torch.bool, device=GPU), w)
    q = torch.zeros(1, 1, 1, dk, dtype=BF16, device=GPU)
    v = torch.full((1, 1, 1, dk), float(frac_tensor([c["new_value"]])[0]), dtype=BF16, device=GPU)
    o, after = ring_attention(q, q, v, torch.tensor([[c["new_pos"]]], device=GPU), ring)
    assert torch.equal(o.float().cpu(), torch.full((1, 1, 1, dk), float(frac_tensor([c["want"]])[0])))
    assert after.pos.cpu().tolist() == [c["pos_after_write"]]
    assert bool(after.valid.all())
    assert torch.equal(ring.pos.cpu(), torch.tensor([c["ring_pos"]]))  # the functional form copied


def _random_ring(b, w, hkv, dk, seed, dtype=BF16):
    g = torch.Generator().manual_seed(seed)
    rk = torch.randn(b, w, hkv, dk, generator=g).to(dtype)
    rv = torch.randn(b, w, hkv, dk, generator=g).to(dtype)
    p = torch.randint(w, 3 * w, (b, 1), generator=g)
    # positions spread around the window: some visible, some too old, some in the future
    rpos = p - torch.randint(-3, w + 5, (b, w), generator=g)
    valid = torch.rand(b, w, generator=g) < 0.85
    return rk, rv, rpos, valid, p


@pytest.mark.parametrize("dtype", [BF16, torch.float16])
@pytest.mark.parametrize("dk", [16, 32, 64, 128])
@pytest.mark.parametrize(("h", "hkv"), [(8, 8), (8, 4), (8, 1), (12, 4)])
def test_random_rings_match_the_oracle(dtype, dk, h, hkv):
    from vesper.kernels.ring_attn import RingKVCache, ring_attention

    b, w = 3, 37
    rk, rv, rpos, valid, p = _random_ring(b, w, hkv, dk, seed=dk + h + hkv, dtype=dtype)
    g = torch.Generator().manual_seed(5)
    q = torch.randn(b, 1, h, dk, generator=g).to(dtype)
    k = torch.randn(b, 1, hkv, dk, generator=g).to(dtype)
    v = torch.randn(b, 1, hkv, dk, generator=g).to(dtype)
    want = oa.ring_attend(q.double(), k.double(), v.double(), p, rk.double(), rv.double(), rpos, valid, w)
    ring = RingKVCache(*(t.to(GPU) for t in (rk, rv, rpos, valid)), w)
    o, after = ring_attention(q.to(GPU), k.to(GPU), v.to(GPU), p.to(GPU), ring)
    assert relative_error(o, want) < 1e-2
    torch.testing.assert_close(o.float().cpu(), want.float(), rtol=3e-2, atol=3e-2)
    nk, nv, npos, nvalid = oa.kv_ring_write(rk, rv, rpos, valid, k, v, p)
    assert torch.equal(after.k.cpu(), nk) and torch.equal(after.v.cpu(), nv)
    assert torch.equal(after.pos.cpu(), npos) and torch.equal(after.valid.cpu(), nvalid)


@pytest.mark.parametrize("dtype", [BF16, torch.float16])
@pytest.mark.parametrize(("h", "hkv", "dk"), [(8, 8, 64), (8, 2, 128), (4, 4, 16)])
def test_a_float32_ring_reads_as_the_ring_cast_to_the_query_dtype(dtype, h, hkv, dk):
    """The reference decoder's rings are float32 (decode.py:81,85; column.py:492) and attend_ring
    casts them to the query dtype (attention.py:325): over a float32 ring the outputs equal, bitwise,
    those over the same ring rounded to q's dtype, and the new token lands in its slot widened to
    float32 (every other slot untouched)."""
    from vesper.kernels.ring_attn import RingKVCache, ring_attention

    b, w = 5, 40
    rk, rv, rpos, valid, p = _random_ring(b, w, hkv, dk, seed=71 + dk, dtype=torch.float32)
    g = torch.Generator().manual_seed(72)
    q = torch.randn(b, 1, h, dk, generator=g).to(dtype)
    k = torch.randn(b, 1, hkv, dk, generator=g).to(dtype)
    v = torch.randn(b, 1, hkv, dk, generator=g).to(dtype)
    wide = RingKVCache(*(t.to(GPU) for t in (rk, rv, rpos, valid)), w)
    narrow = RingKVCache(rk.to(GPU, dtype), rv.to(GPU, dtype), rpos.to(GPU), valid.to(GPU), w)
    dq, dk_, dv, dp = (t.to(GPU) for t in (q, k, v, p))
    o32, after32 = ring_attention(dq, dk_, dv, dp, wide)
    o16, after16 = ring_attention(dq, dk_, dv, dp, narrow)
    assert torch.equal(o32, o16)
    assert after32.k.dtype == torch.float32 and after32.v.dtype == torch.float32
    nk, nv, npos, nvalid = oa.kv_ring_write(rk, rv, rpos, valid, k.float(), v.float(), p)
    assert torch.equal(after32.k.cpu(), nk) and torch.equal(after32.v.cpu(), nv)
    assert torch.equal(after32.pos.cpu(), npos) and torch.equal(after32.valid.cpu(), nvalid)
    assert torch.equal(after16.pos, after32.pos)
    want = oa.ring_attend(q.double(), k.double(), v.double(), p, rk.to(dtype).double(), rv.to(dtype).double(),
                          rpos, valid, w)
    assert relative_error(o32, want) < 1e-2


@pytest.mark.parametrize("ring_dtype", [BF16, torch.float32])
@pytest.mark.parametrize("dk", [8, 24, 40, 96, 136, 200, 248, 256])
@pytest.mark.parametrize(("h", "hkv"), [(8, 8), (4, 2), (8, 1)])
def test_rings_of_every_width_up_to_256_match_the_oracle(ring_dtype, dk, h, hkv):
    """Head widths past the four first ones: 8 and 256 run their own shape; the widths that are not
    powers of two run the next power of two's lanes with the lanes past the width idle (nothing
    read or written there: the slots' neighbours in the ring row stay untouched)."""
    from vesper.kernels.ring_attn import RingKVCache, ring_attention

    b, w = 3, 45
    rk, rv, rpos, valid, p = _random_ring(b, w, hkv, dk, seed=3 * dk + h, dtype=ring_dtype)
    g = torch.Generator().manual_seed(dk)
    q = torch.randn(b, 1, h, dk, generator=g).to(BF16)
    k = torch.randn(b, 1, hkv, dk, generator=g).to(BF16)
    v = torch.randn(b, 1, hkv, dk, generator=g).to(BF16)
    want = oa.ring_attend(q.double(), k.double(), v.double(), p, rk.to(BF16).double(), rv.to(BF16).double(),
                          rpos, valid, w)
    ring = RingKVCache(*(t.to(GPU) for t in (rk, rv, rpos, valid)), w)
    o, after = ring_attention(q.to(GPU), k.to(GPU), v.to(GPU), p.to(GPU), ring)
    assert relative_error(o, want) < 1e-2
    torch.testing.assert_close(o.float().cpu(), want.float(), rtol=3e-2, atol=3e-2)
    nk, nv, npos, nvalid = oa.kv_ring_write(rk, rv, rpos, valid, k.to(ring_dtype), v.to(ring_dtype), p)
    assert torch.equal(after.k.cpu(), nk) and torch.equal(after.v.cpu(), nv)
    assert torch.equal(after.pos.cpu(), npos) and torch.equal(after.valid.cpu(), nvalid)


def test_widths_the_kernel_does_not_take_are_refused():
    from vesper.contracts import ContractError
    from vesper.kernels.ring_attn import kv_ring_empty, ring_attention

    for dk in (12, 264):
        ring = kv_ring_empty(1, 1, dk, 8, BF16, GPU)
        q = torch.zeros(1, 1, 1, dk, dtype=BF16, device=GPU)
        with pytest.raises(ContractError, match="multiples of 8"):
            ring_attention(q, q, q, torch.tensor([[1]], device=GPU), ring)


def test_a_ring_of_another_dtype_is_refused():
    from vesper.contracts import ContractError
    from vesper.kernels.ring_attn import kv_ring_empty, ring_attention

    ring = kv_ring_empty(1, 1, 16, 4, torch.float16, GPU)
    q = torch.zeros(1, 1, 1, 16, dtype=BF16, device=GPU)
    with pytest.raises(ContractError, match="dtype"):
        ring_attention(q, q, q, torch.ones(1, 1, dtype=torch.long, device=GPU), ring)


def test_decoding_steps_equal_the_whole_chunk_window():
    # 3w + 5 single-token steps from an empty ring equal the window attention over the whole chunk
    from vesper.kernels.ring_attn import kv_ring_empty, ring_attention

    b, h, hkv, dk, w, start = 2, 8, 2, 64, 16, 7
    steps = 3 * w + 5
    g = torch.Generator().manual_seed(4)
    q = torch.randn(b, steps, h, dk, generator=g).to(BF16)
    k = torch.randn(b, steps, hkv, dk, generator=g).to(BF16)
    v = torch.randn(b, steps, hkv, dk, generator=g).to(BF16)
    whole = oa.window_attention(q.double(), k.double(), v.double(), w)
    ring = kv_ring_empty(b, hkv, dk, w, BF16, GPU)
    pos = torch.arange(start, start + steps).expand(b, steps).contiguous()
    outs = []
    for i in range(steps):
        sl = slice(i, i + 1)
        o, ring = ring_attention(q[:, sl].to(GPU), k[:, sl].to(GPU), v[:, sl].to(GPU), pos[:, sl].to(GPU), ring,
                                 inplace=True)
        outs.append(o)
    got = torch.cat(outs, 1)
    assert relative_error(got, whole) < 1e-2
    torch.testing.assert_close(got.float().cpu(), whole.float(), rtol=3e-2, atol=3e-2)
    held = ring.valid[0].cpu()
    assert sorted(ring.pos[0].cpu()[held].tolist()) == list(range(start + steps - w, start + steps))


def test_captured_decoding_with_one_workspace_equals_eager_on_every_replay():
    # eight decoding steps captured in one graph, all sharing one counter workspace: every replay
    # from the same starting ring gives the eager outputs and ring bitwise, and leaves the counters zero
    from vesper.kernels.ring_attn import RingKVCache, ring_attention

    b, h, hkv, dk, w, steps = 6, 8, 8, 64, 32, 8
    rk, rv, rpos, valid, _ = _random_ring(b, w, hkv, dk, seed=11)
    g = torch.Generator().manual_seed(12)
    q = torch.randn(steps, b, 1, h, dk, generator=g).to(BF16).to(GPU)
    k = torch.randn(steps, b, 1, hkv, dk, generator=g).to(BF16).to(GPU)
    v = torch.randn(steps, b, 1, hkv, dk, generator=g).to(BF16).to(GPU)
    p0 = torch.randint(2 * w, 3 * w, (b, 1), generator=g)
    pos = torch.stack([p0 + i for i in range(steps)]).to(GPU)
    start = [t.to(GPU) for t in (rk, rv, rpos, valid)]
    counters = torch.zeros(b, dtype=torch.int32, device=GPU)

    def run(ring):
        return [ring_attention(q[i], k[i], v[i], pos[i], ring, inplace=True, check_positions=False,
                               workspace=counters)[0] for i in range(steps)]

    eager_ring = RingKVCache(*(t.clone() for t in start), w)
    eager = run(eager_ring)
    ring = RingKVCache(*(t.clone() for t in start), w)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        run(RingKVCache(*(t.clone() for t in start), w))
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        got = run(ring)
    for rep in range(3):
        for dst, src in zip((ring.k, ring.v, ring.pos, ring.valid), start):
            dst.copy_(src)
        graph.replay()
        torch.cuda.synchronize()
        for i in range(steps):
            assert torch.equal(got[i], eager[i]), (rep, i)
        for a, e in zip((ring.k, ring.v, ring.pos, ring.valid), (eager_ring.k, eager_ring.v, eager_ring.pos, eager_ring.valid)):
            assert torch.equal(a, e), rep
        assert int(counters.abs().sum()) == 0, rep
        run(RingKVCache(*(t.clone() for t in start), w))  # eager work between replays
        torch.cuda.synchronize()


def test_decode_config_b64_h8_d64_ring512_one_step():
    from vesper.kernels.ring_attn import RingKVCache, ring_attention

    b, h, dk, w = 64, 8, 64, 512
    g = torch.Generator().manual_seed(0)
    rk = torch.randn(b, w, h, dk, generator=g).to(BF16)
    rv = torch.randn(b, w, h, dk, generator=g).to(BF16)
    rpos = torch.arange(w).expand(b, w).contiguous()
    valid = torch.ones(b, w, dtype=torch.bool)
    q = torch.randn(b, 1, h, dk, generator=g).to(BF16)
    k = torch.randn(b, 1, h, dk, generator=g).to(BF16)
    v = torch.randn(b, 1, h, dk, generator=g).to(BF16)
    p = torch.full((b, 1), w)
    want = oa.ring_attend(q.float(), k.float(), v.float(), p, rk.float(), rv.float(), rpos, valid, w)
    ring = RingKVCache(*(t.to(GPU) for t in (rk, rv, rpos, valid)), w)
    o, after = ring_attention(q.to(GPU), k.to(GPU), v.to(GPU), p.to(GPU), ring, inplace=True)
    assert relative_error(o, want) < 1e-2
    assert after is ring and int(ring.pos[0, 0]) == w  # slot 512 % 512 = 0 took the new token


def test_an_inactive_row_reads_zero_and_still_writes():
    from vesper.kernels.ring_attn import RingKVCache, ring_attention

    rk, rv, rpos, valid, p = _random_ring(4, 20, 2, 64, seed=3)
    g = torch.Generator().manual_seed(6)
    q = torch.randn(4, 1, 4, 64, generator=g).to(BF16)
    k = torch.randn(4, 1, 2, 64, generator=g).to(BF16)
    v = torch.randn(4, 1, 2, 64, generator=g).to(BF16)
    act = torch.tensor([True, False, True, False])
    ring = RingKVCache(*(t.to(GPU) for t in (rk, rv, rpos, valid)), 20)
    o_all, _ = ring_attention(q.to(GPU), k.to(GPU), v.to(GPU), p.to(GPU), ring)
    o, after = ring_attention(q.to(GPU), k.to(GPU), v.to(GPU), p.to(GPU), ring, active=act.to(GPU))
    assert torch.equal(o[act.to(GPU)], o_all[act.to(GPU)]) and bool((o[~act.to(GPU)] == 0).all())
    _, _, npos, _ = oa.kv_ring_write(rk, rv, rpos, valid, k, v, p)
    assert torch.equal(after.pos.cpu(), npos)


def test_refusals():
    from vesper.contracts import ContractError
    from vesper.kernels.ring_attn import kv_ring_empty, ring_attention

    ring = kv_ring_empty(1, 1, 64, 8, BF16, GPU)
    q = torch.zeros(1, 1, 1, 64, dtype=BF16, device=GPU)
    with pytest.raises(ContractError, match="nonnegative"):
        ring_attention(q, q, q, torch.tensor([[-1]], device=GPU), ring)
    with pytest.raises(ContractError, match="dtype"):
        ring_attention(q.float(), q, q, torch.tensor([[1]], device=GPU), ring)
    with pytest.raises(ContractError, match="axis"):
        ring_attention(q, q, q, torch.tensor([[1, 2]], device=GPU), ring)


def test_decode_config_256_steps_delta_and_ring_against_the_chunked_oracles():
    """The decode workload at its full size: batch 64, H 8, d 64, 256 steps, each the delta rule's
    single step on the fp32 state [64, 8, 64, 64] (S0 ~ N(0, 0.02^2)) and attention over a bf16 KV
    ring of 512 entries prefilled at positions 0..511, the step at position 512 + s writing slot
    s (every slot of the first half is overwritten). The truth: the chunked delta scan over the 256
    tokens (the same recurrence) and window attention with the 512 prefilled rows as the cache
    (the ring's visible entries are the window's keys), both on the CPU."""
    from oracle.delta import delta_scan_chunked, normalize_keys
    from vesper.kernels.delta_scan import delta_scan_step_fused
    from vesper.kernels.ring_attn import RingKVCache, ring_attention

    b, h, dk, w, steps = 64, 8, 64, 512, 256
    g = torch.Generator().manual_seed(11)
    s0 = 0.02 * torch.randn(b, h, dk, dk, generator=g)
    q = torch.randn(b, steps, h, dk, generator=g)
    k = normalize_keys(torch.randn(b, steps, h, dk, generator=g))
    q = normalize_keys(q)
    v = torch.randn(b, steps, h, dk, generator=g)
    beta = torch.sigmoid(torch.randn(b, steps, h, generator=g))
    rk = torch.randn(b, w, h, dk, generator=g).to(BF16)
    rv = torch.randn(b, w, h, dk, generator=g).to(BF16)
    aq = torch.randn(b, steps, h, dk, generator=g).to(BF16)
    ak = torch.randn(b, steps, h, dk, generator=g).to(BF16)
    av = torch.randn(b, steps, h, dk, generator=g).to(BF16)

    state = s0.to(GPU)
    ring = RingKVCache(rk.to(GPU), rv.to(GPU), torch.arange(w).expand(b, w).contiguous().to(GPU),
                       torch.ones(b, w, dtype=torch.bool, device=GPU), w)
    dq, dkk, dv, db = (t.to(GPU) for t in (q, k, v, beta))
    daq, dak, dav = (t.to(GPU) for t in (aq, ak, av))
    outs, atts = [], []
    with torch.no_grad():
        for s in range(steps):
            o, _ = delta_scan_step_fused(dq[:, s], dkk[:, s], dv[:, s], db[:, s], state, out_state=state)
            a, _ = ring_attention(daq[:, s : s + 1], dak[:, s : s + 1], dav[:, s : s + 1],
                                  torch.full((b, 1), w + s, device=GPU), ring, inplace=True, check_positions=False)
            outs.append(o)
            atts.append(a)
    o_ref, s_ref = delta_scan_chunked(q.double(), k.double(), v.double(), beta.double(), s0.double(), 64)
    assert relative_error(torch.stack(outs, dim=1), o_ref) < 1e-5
    assert relative_error(state, s_ref) < 1e-5
    keys = torch.cat([rk, ak], dim=1).float()
    values = torch.cat([rv, av], dim=1).float()
    a_ref = oa.window_attention(aq.float(), keys, values, w)
    assert relative_error(torch.cat(atts, dim=1), a_ref) < 1e-2
    # the ring now holds positions 256..767: slots 0..255 rewritten with the new tokens
    assert torch.equal(ring.pos[:, :steps].cpu(), torch.arange(w, w + steps).expand(b, steps))
    assert torch.equal(ring.k[:, :steps].cpu(), ak) and torch.equal(ring.v[:, steps:].cpu(), rv[:, steps:])
