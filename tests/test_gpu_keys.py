"""The key filter kernel (``vsp_key_filter_*`` via ``vesper.kernels.keys`` / ``vesper.column``)
against the key-filter oracle.

Parity bar (the reference's own, ``tests/test_keys_fused.py:70-75``): 2e-5 for float32 key inputs,
8e-3 for bfloat16 (the key's own final rounding), element-wise against the oracle in float64, for
the keys, the next history and the gradients of the key input, the taps and the history. At the
prefill shape (B8 T4096, d 512 = 8 heads of 64, 4 taps) the same bound against the oracle in
float32, and exact size-independent properties: chunking does not change a key (bitwise), the
backward repeats bitwise, captured replays equal eager.
"""

from __future__ import annotations

import pytest
import torch

from conftest import needs_gpu
from oracle import keys as ok
from oracle.delta import normalize_keys

pytestmark = [pytest.mark.gpu, needs_gpu]

GPU = torch.device("cuda")
K = 4


def _taps(d: int, width: int = K) -> torch.Tensor:
    # asymmetric: every tap and channel differ (tests/test_keys_fused.py:38-43 of the reference)
    r = torch.arange(width, dtype=torch.float32)[:, None]
    j = torch.arange(d, dtype=torch.float32)[None, :]
    return (r + 1) * 0.5 - 0.003 * j + 0.01 * r * j


def _bound(dtype: torch.dtype) -> float:
    return 2e-5 if dtype == torch.float32 else 8e-3


def _check(z, history, taps, heads, dtype):
    from vesper.column import recurrent_keys

    keys, after = recurrent_keys(z.to(GPU), history.to(GPU), taps.to(GPU), heads)
    want, want_after = ok.filter_keys(z.double(), history.double(), taps.double(), heads)
    bound = _bound(dtype)
    torch.testing.assert_close(keys.double().cpu(), want, rtol=bound, atol=bound)
    assert keys.dtype == dtype
    torch.testing.assert_close(after.cpu().double(), want_after, rtol=0, atol=0)
    return keys


@pytest.mark.parametrize("n", [1, 2, 3, 257])  # shorter than the filter, and a long chunk
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_the_keys_match_the_oracle(n, dtype):
    g = torch.Generator().manual_seed(n)
    z = (torch.randn(3, n, 128, generator=g) * 2).to(dtype)
    z[0, 0] = 0.0  # a zero key input row: the floor
    history = torch.randn(3, K - 1, 128, generator=g)
    _check(z, history, _taps(128), 2, dtype)


@pytest.mark.parametrize("head_dim", [8, 16, 32, 64, 128, 256, 512])
@pytest.mark.parametrize("width", [1, 2, 4, 8])
def test_every_head_width_and_filter_width(head_dim, width):
    g = torch.Generator().manual_seed(head_dim + width)
    heads = max(1, 512 // head_dim)
    d = heads * head_dim
    z = torch.randn(2, 45, d, generator=g).to(torch.bfloat16)
    history = torch.randn(2, width - 1, d, generator=g)
    _check(z, history, _taps(d, width), heads, torch.bfloat16)


def test_the_prefill_shape_b8_t4096_d512_h8_k4():
    g = torch.Generator().manual_seed(11)
    z = torch.randn(8, 4096, 512, generator=g).to(torch.bfloat16)
    history = torch.randn(8, K - 1, 512, generator=g)
    from vesper.kernels.keys import fused_keys

    keys = fused_keys(z.to(GPU), history.to(GPU), _taps(512).to(GPU), 8)
    want, _ = ok.filter_keys(z.float(), history, _taps(512), 8)
    torch.testing.assert_close(keys.float().cpu(), want.float(), rtol=8e-3, atol=8e-3)
    again = fused_keys(z.to(GPU), history.to(GPU), _taps(512).to(GPU), 8)
    assert torch.equal(keys, again)


def test_chunking_does_not_change_a_key():
    from vesper.column import recurrent_keys

    g = torch.Generator().manual_seed(3)
    z = torch.randn(2, 300, 256, generator=g).to(GPU, torch.bfloat16)
    cold = torch.zeros(2, K - 1, 256, device=GPU)
    taps = _taps(256).to(GPU)
    whole, last = recurrent_keys(z, cold, taps, 4)
    for sizes in ((1,) * 7 + (293,), (2, 0, 3, 1, 294), (100, 100, 100), (0, 4, 296)):
        history, start, parts = cold, 0, []
        for size in sizes:
            keys, history = recurrent_keys(z[:, start:start + size], history, taps, 4)
            parts.append(keys)
            start += size
        assert torch.equal(torch.cat(parts, dim=1), whole), sizes
        assert torch.equal(history, last)


def test_no_filter_is_the_plain_normalization_and_keeps_the_history():
    from vesper.column import recurrent_keys

    g = torch.Generator().manual_seed(4)
    z = torch.randn(2, 33, 128, generator=g)
    none = torch.zeros(2, 0, 128, device=GPU)
    keys, after = recurrent_keys(z.to(GPU), none, None, 2)
    assert after is none
    torch.testing.assert_close(keys.cpu().double(), normalize_keys(z.double().view(2, 33, 2, 64)), rtol=2e-5, atol=2e-5)
    empty = z[:, :0].to(GPU)
    history = torch.randn(2, K - 1, 128, device=GPU)
    keys, after = recurrent_keys(empty, history, _taps(128).to(GPU), 2)
    assert keys.shape == (2, 0, 2, 64) and after is history


def test_the_reference_normalization_edge_rows_through_the_kernel():
    # tests/test_recurrence_review.py:37-87 of the reference, through the key kernel's path without
    # a filter (recurrent_keys with no taps): a row whose peak is a huge or tiny finite value
    # normalizes to exactly a unit vector in its own dtype; a row under the 1e-6 floor is exactly
    # u / 1e-6 (float32, as the oracle's division in float32 gives it); a zero row stays zero. Head
    # width 8 (the kernel's narrowest), the peak at several features and signs.
    from conftest import frac_tensor, reference_vectors
    from vesper.column import recurrent_keys

    c = reference_vectors()["normalize_keys"]
    for dtype_name, magnitude in c["magnitudes_by_dtype"]["rows"]:
        if dtype_name == "float64":
            continue  # no float64 kernel
        dtype = getattr(torch, dtype_name)
        z = torch.zeros(1, 4, 16, dtype=dtype)
        want = torch.zeros(1, 4, 2, 8, dtype=dtype)
        for t, (feature, sign) in enumerate([(0, 1.0), (5, -1.0), (9, 1.0), (15, -1.0)]):
            z[0, t, feature] = sign * float(magnitude)
            want[0, t, feature // 8, feature % 8] = sign
        keys, _ = recurrent_keys(z.to(GPU), torch.zeros(1, 0, 16, device=GPU), None, 2)
        assert torch.equal(keys.cpu(), want), dtype_name
    small = frac_tensor(c["small_floor"]["k"], torch.float32)  # [[3e-8, 4e-8]]
    z = torch.zeros(1, 2, 8)
    z[0, 0, :2] = small[0]
    z[0, 1, 6:] = -small[0]
    keys, _ = recurrent_keys(z.to(GPU), torch.zeros(1, 0, 8, device=GPU), None, 1)
    assert torch.equal(keys.cpu(), normalize_keys(z.view(1, 2, 1, 8)))
    want = frac_tensor(c["small_floor"]["want"])[0]
    torch.testing.assert_close(keys[0, 0, 0, :2].cpu().double(), want, rtol=1e-7, atol=0)
    zero = torch.zeros(1, 3, 8)
    keys, _ = recurrent_keys(zero.to(GPU), torch.zeros(1, 0, 8, device=GPU), None, 1)
    assert torch.equal(keys.cpu(), zero.view(1, 3, 1, 8))


def test_captured_replays_equal_eager():
    from vesper.kernels.keys import fused_keys

    g = torch.Generator().manual_seed(5)
    z = torch.randn(2, 64, 128, generator=g).to(GPU, torch.bfloat16)
    history = torch.randn(2, K - 1, 128, generator=g).to(GPU)
    taps = _taps(128).to(GPU)
    eager = fused_keys(z, history, taps, 2)
    out = torch.empty_like(eager)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        out.copy_(fused_keys(z, history, taps, 2))  # warm-up outside the capture
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out.copy_(fused_keys(z, history, taps, 2))
    for _ in range(3):
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)


def test_refusals():
    from vesper.contracts import ContractError
    from vesper.kernels.keys import fused_keys

    z = torch.randn(1, 4, 128, device=GPU)
    history = torch.zeros(1, K - 1, 128, device=GPU)
    taps = _taps(128).to(GPU)
    with pytest.raises(ContractError, match="dtype"):
        fused_keys(z.double(), history, taps, 2)
    with pytest.raises(ContractError, match="CUDA only"):
        fused_keys(z.cpu(), history.cpu(), taps.cpu(), 2)
    with pytest.raises(ContractError, match="taps"):
        fused_keys(z, torch.zeros(1, 8, 128, device=GPU), _taps(128, 9).to(GPU), 2)
    with pytest.raises(ContractError, match="head width"):
        fused_keys(z, history, taps, 32)  # head width 4
    with pytest.raises(ContractError, match="axis"):
        fused_keys(z, torch.zeros(1, K, 128, device=GPU), taps, 2)


def _grads(z, history, taps, heads, up):
    from vesper.column import recurrent_keys

    zs, hs, ts = (t.detach().clone().to(GPU).requires_grad_() for t in (z, history, taps))
    keys, _ = recurrent_keys(zs, hs, ts, heads)
    torch.autograd.backward([(keys.double() * up.to(GPU).double()).sum()])
    return zs.grad, hs.grad, ts.grad


def _check_grads(z, history, taps, heads, up, bound):
    got = _grads(z, history, taps, heads, up)
    # the key's gradient reaches the kernel in the key's dtype, as under the reference's autograd
    g = up.to(z.dtype).double()
    want = ok.filter_keys_grads(z.double(), history.double(), taps.double(), heads, g)
    for a, b, name in zip(got, want, ("dz", "dhistory", "dtaps")):
        assert a is not None, name
        torch.testing.assert_close(a.double().cpu(), b, rtol=bound, atol=bound, msg=name)
    return got


@pytest.mark.parametrize("n", [1, 2, 3, 257])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_the_gradients_match_the_oracle(n, dtype):
    g = torch.Generator().manual_seed(100 + n)
    z = (torch.randn(3, n, 128, generator=g) * 2).to(dtype)
    z[0, 0] = 0.0
    history = torch.randn(3, K - 1, 128, generator=g)
    up = torch.randn(3, n, 2, 64, generator=g)
    dz, dh, dt = _check_grads(z, history, _taps(128), 2, up, _bound(dtype))
    assert dz.dtype == dtype and dh.dtype == torch.float32 and dt.dtype == torch.float32


@pytest.mark.parametrize("head_dim", [8, 64, 512])
@pytest.mark.parametrize("width", [1, 2, 3, 4, 5, 8])
def test_the_gradients_for_every_filter_width(head_dim, width):
    g = torch.Generator().manual_seed(head_dim * 10 + width)
    heads = max(1, 512 // head_dim)
    z = torch.randn(2, 70, 512, generator=g)
    history = torch.randn(2, width - 1, 512, generator=g)
    up = torch.randn(2, 70, heads, head_dim, generator=g)
    _check_grads(z, history, _taps(512, width), heads, up, 2e-5)


def test_the_gradients_at_the_prefill_shape_and_they_repeat():
    from vesper.kernels.keys import fused_keys

    g = torch.Generator().manual_seed(12)
    z = torch.randn(8, 4096, 512, generator=g).to(torch.bfloat16)
    history = torch.randn(8, K - 1, 512, generator=g)
    taps = _taps(512)
    up = torch.randn(8, 4096, 8, 64, generator=g).to(torch.bfloat16)

    def run():
        zs, hs, ts = (t.to(GPU).requires_grad_() for t in (z, history, taps))
        keys = fused_keys(zs, hs, ts, 8)
        keys.backward(up.to(GPU))
        return zs.grad, hs.grad, ts.grad

    first = run()
    again = run()
    for a, b in zip(first, again):
        assert torch.equal(a, b)  # deterministic: the taps' sums run in a fixed order
    want = ok.filter_keys_grads(z.float(), history, taps, 8, up.float())
    for a, b, name in zip(first, want, ("dz", "dhistory", "dtaps")):
        torch.testing.assert_close(a.float().cpu(), b, rtol=8e-3, atol=8e-3, msg=name)


def test_captured_forward_and_backward_equal_eager():
    from vesper.kernels.keys import fused_keys

    g = torch.Generator().manual_seed(13)
    z = torch.randn(2, 100, 128, generator=g).to(GPU, torch.bfloat16).requires_grad_()
    history = torch.randn(2, K - 1, 128, generator=g).to(GPU).requires_grad_()
    taps = _taps(128).to(GPU).requires_grad_()
    up = torch.randn(2, 100, 2, 64, generator=g).to(GPU, torch.bfloat16)

    def step():
        keys = fused_keys(z, history, taps, 2)
        return (keys.detach(), *torch.autograd.grad((keys * up).sum(), (z, history, taps)))

    eager = [t.clone() for t in step()]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()  # warm-up outside the capture
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        static = step()
    for _ in range(3):
        for t in static:
            t.zero_()
        graph.replay()
        torch.cuda.synchronize()
        for a, b in zip(static, eager):
            assert torch.equal(a, b)


def test_an_empty_chunk_has_zero_gradients():
    from vesper.kernels.keys import fused_keys

    z = torch.randn(2, 0, 128, device=GPU, requires_grad=True)
    history = torch.randn(2, K - 1, 128, device=GPU, requires_grad=True)
    taps = _taps(128).to(GPU).requires_grad_()
    keys = fused_keys(z, history, taps, 2)
    gz, gh, gt = torch.autograd.grad(keys.sum(), (z, history, taps), allow_unused=True)
    assert gz.shape == z.shape
    assert torch.equal(gh, torch.zeros_like(gh)) and torch.equal(gt, torch.zeros_like(gt))


# ---- copy-forward inside the filter's loads (carried key inputs of inactive tokens) ----

@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize(("n", "width", "head_dim"), [(3, 4, 64), (40, 1, 16), (257, 4, 64), (300, 8, 128)])
def test_carried_key_inputs_equal_the_merged_ones_bitwise(dtype, n, width, head_dim):
    from vesper.column import recurrent_keys

    b, heads = 2, 2
    d = heads * head_dim
    g = torch.Generator().manual_seed(n + width)
    z = torch.randn(b, n, d, generator=g).to(GPU, dtype)
    zc = torch.randn(b, n, d, generator=g).to(GPU, dtype)
    history = torch.randn(b, width - 1, d, generator=g).to(GPU)
    taps = _taps(d, width).to(GPU)
    active = (torch.rand(b, n, generator=g) > 0.4).to(GPU)
    merged = torch.where(active[..., None], z, zc)
    poisoned = z.masked_fill(~active[..., None], float("nan"))  # fresh inputs of inactive tokens: never read
    keys, hist = recurrent_keys(poisoned, history, taps, heads, active=active, carried_z=zc)
    want_keys, want_hist = recurrent_keys(merged, history, taps, heads)
    torch.cuda.synchronize()
    assert torch.equal(keys, want_keys)
    assert torch.equal(hist, want_hist)


def test_carried_key_inputs_at_b8_t4096_d512_h8_k4():
    from vesper.kernels.keys import fused_keys

    b, n, d, heads = 8, 4096, 512, 8
    g = torch.Generator().manual_seed(5)
    z, zc = (torch.randn(b, n, d, generator=g).to(GPU, torch.bfloat16) for _ in range(2))
    history = torch.randn(b, K - 1, d, generator=g).to(GPU)
    taps = _taps(d).to(GPU)
    active = (torch.rand(b, n, generator=g) > 0.3).to(GPU)
    got = fused_keys(z, history, taps, heads, active=active, carried_z=zc)
    want = fused_keys(torch.where(active[..., None], z, zc), history, taps, heads)
    assert torch.equal(got, want)


def test_carried_key_inputs_under_autograd_reach_the_carried_tensor():
    from vesper.kernels.keys import fused_keys

    b, n, d, heads = 2, 50, 64, 1
    g = torch.Generator().manual_seed(6)
    z, zc = (torch.randn(b, n, d, generator=g).to(GPU).requires_grad_() for _ in range(2))
    history = torch.randn(b, K - 1, d, generator=g).to(GPU)
    active = (torch.rand(b, n, generator=g) > 0.4).to(GPU)
    fused_keys(z, history, _taps(d).to(GPU), heads, active=active, carried_z=zc).square().sum().backward()
    assert not bool(z.grad[~active].any()) and not bool(zc.grad[active].any()) and bool(zc.grad.any())


# ---- the key step: keys and the next history from one launch ----

@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize(("n", "width"), [(1, 4), (2, 4), (3, 4), (5, 4), (40, 8), (17, 2), (9, 1)])
@pytest.mark.parametrize("carry", [False, True])
def test_the_key_step_writes_the_next_history(dtype, n, width, carry):
    from vesper.kernels.keys import fused_keys, key_step

    b, heads, d = 2, 2, 128
    g = torch.Generator().manual_seed(n * 10 + width)
    z = torch.randn(b, n, d, generator=g).to(GPU, dtype)
    zc = torch.randn(b, n, d, generator=g).to(GPU, dtype)
    history = torch.randn(b, width - 1, d, generator=g).to(GPU)
    taps = _taps(d, width).to(GPU)
    active = (torch.rand(b, n, generator=g) > 0.4).to(GPU) if carry else None
    keys, nxt = key_step(z, history, taps, heads, active=active, carried_z=zc if carry else None)
    merged = torch.where(active[..., None], z, zc) if carry else z
    want = torch.cat([history, merged.float()], dim=1)[:, n:]  # the newest width - 1 inputs
    assert nxt.dtype == torch.float32 and nxt.shape == (b, width - 1, d)
    assert torch.equal(nxt, want)
    assert torch.equal(keys, fused_keys(merged, history, taps, heads))


_IN_PLACE = [(1, 4), (1, 2), (1, 8), (3, 4), (7, 8), (8, 4), (2, 1)]


@pytest.mark.parametrize(("dtype", "n", "width"), [(torch.float32, n, w) for n, w in _IN_PLACE]
                         + [(torch.bfloat16, n, w) for n, w in _IN_PLACE + [(16, 8)]])
@pytest.mark.parametrize("carry", [False, True])
def test_the_key_step_updates_a_history_in_place(dtype, n, width, carry):
    """A decode step's update: the next history written over the history it was computed from
    equals the out-of-place step's, keys included, bit for bit (chunks up to 8 tokens with float32
    inputs, 16 with bf16)."""
    from vesper.kernels.keys import key_step

    b, heads, d = 3, 2, 256
    g = torch.Generator().manual_seed(n * 100 + width)
    z = torch.randn(b, n, d, generator=g).to(GPU, dtype)
    zc = torch.randn(b, n, d, generator=g).to(GPU, dtype)
    history = torch.randn(b, width - 1, d, generator=g).to(GPU)
    taps = _taps(d, width).to(GPU)
    active = (torch.rand(b, n, generator=g) > 0.4).to(GPU) if carry else None
    want_keys, want_next = key_step(z, history, taps, heads, active=active, carried_z=zc if carry else None)
    inplace = history.clone()
    keys, nxt = key_step(z, inplace, taps, heads, active=active, carried_z=zc if carry else None, in_place=True)
    assert nxt is inplace
    assert torch.equal(inplace, want_next) and torch.equal(keys, want_keys)


def test_an_in_place_history_refuses_a_long_chunk():
    from vesper.contracts import ContractError
    from vesper.kernels.keys import key_step

    z = torch.zeros(1, 17, 64, dtype=torch.bfloat16, device=GPU)
    history = torch.zeros(1, 3, 64, device=GPU)
    with pytest.raises(ContractError, match="at most 16"):
        key_step(z, history, _taps(64, 4).to(GPU), 1, in_place=True)


@pytest.mark.parametrize("dk", [16, 32, 64, 128])
@pytest.mark.parametrize("width", [1, 2, 4, 8])
@pytest.mark.parametrize("inactive", [False, True])
def test_the_key_filter_inside_the_delta_step_equals_the_two_launches(dk, width, inactive):
    """vsp_delta_step_keys_bf16: the decode step's key formed inside the delta step's launch gives
    the key step's history and the delta step's output and state bit for bit."""
    from vesper.kernels.delta_scan import delta_scan_step_fused, delta_scan_step_keys
    from vesper.kernels.keys import key_step

    b, h = 3, 4
    g = torch.Generator().manual_seed(dk * 10 + width)
    q, v = (torch.randn(b, h, dk, generator=g).to(torch.bfloat16).to(GPU) for _ in range(2))
    z = torch.randn(b, 1, h * dk, generator=g).to(torch.bfloat16).to(GPU)
    beta = torch.rand(b, h, generator=g).to(torch.bfloat16).to(GPU)
    history = torch.randn(b, width - 1, h * dk, generator=g).to(GPU)
    taps = _taps(h * dk, width).to(GPU)
    state = (0.1 * torch.randn(b, h, dk, dk, generator=g)).to(GPU)
    active = torch.tensor([True, False, True], device=GPU) if inactive else None
    keys, want_hist = key_step(z, history, taps, h)
    want_o, want_state = delta_scan_step_fused(q, keys[:, 0], v, beta, state, active=active)
    hist, st = history.clone(), state.clone()
    o = delta_scan_step_keys(q, z[:, 0], v, beta, hist, taps, st, active=active)
    assert torch.equal(o, want_o) and torch.equal(st, want_state) and torch.equal(hist, want_hist)


# ---- normalize_keys alone, on rows of any width (vsp_normalize_keys_*) ---------------------------

@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("width", [1, 3, 64, 100, 513, 4096, 65536])
def test_normalize_keys_on_rows_of_any_width(width, dtype):
    from vesper.kernels.keys import normalize_keys as fused

    g = torch.Generator().manual_seed(width)
    rows = 3 if width >= 4096 else 37
    k = (torch.randn(rows, width, generator=g) * torch.logspace(-8, 3, rows)[:, None]).to(dtype)
    k[0] = 0  # a zero row stays zero
    got = fused(k.to(GPU))
    assert got.dtype == dtype and got.shape == k.shape
    bound = _bound(dtype)
    torch.testing.assert_close(got.cpu().double(), normalize_keys(k.double()), rtol=bound, atol=bound)
    assert torch.equal(fused(k.to(GPU)), got)  # repeatable
    # leading dimensions are rows: a [2, rows / 2 ...] view gives the same rows
    if rows % 2 == 0:
        assert torch.equal(fused(k.to(GPU).view(2, rows // 2, width)).view(rows, width), got)


def test_normalize_keys_reference_rows():
    # tests/test_recurrence_review.py:50-87 of the reference: 65536 float16 ones give exactly 1/256
    # each (the squared norm accumulated without overflow); a row whose peak is huge or tiny in its
    # dtype is exactly a unit vector; a row under the 1e-6 floor is u / 1e-6; a zero row stays zero
    from conftest import frac_tensor, reference_vectors
    from vesper.kernels.keys import normalize_keys as fused

    c = reference_vectors()["normalize_keys"]
    assert c["wide_ones_fp16"]["n"] == 65536 and c["wide_ones_fp16"]["want_each"] == "1/256"
    ones = torch.ones(1, 65536, dtype=torch.float16, device=GPU)
    assert torch.equal(fused(ones), torch.full_like(ones, 1 / 256))
    for dtype_name, magnitude in c["magnitudes_by_dtype"]["rows"]:
        if dtype_name == "float64":
            continue  # no float64 kernel
        dtype = getattr(torch, dtype_name)
        key = torch.tensor(((float(magnitude), 0.0),), dtype=dtype, device=GPU)
        assert torch.equal(fused(key), torch.tensor(((1.0, 0.0),), dtype=dtype, device=GPU)), dtype_name
    small = frac_tensor(c["small_floor"]["k"], torch.float32).to(GPU)
    torch.testing.assert_close(fused(small).cpu().double(), frac_tensor(c["small_floor"]["want"]), rtol=1e-7, atol=0)
    zero = torch.zeros(1, 3, device=GPU)
    assert torch.equal(fused(zero), zero)


def test_normalize_keys_gradients():
    # the reference's independent derivative (tests/test_recurrence_review.py:67-72): at (s, 2 s),
    # d((x + y) / sqrt(x^2 + y^2)) = (2, -1) / (5 sqrt 5) / s; then random rows at several widths
    # against the oracle's autograd in float64, and rows under the floor (gradient g / 1e-6)
    import math

    from vesper.kernels.keys import normalize_keys as fused

    for s in (1.0, 1e30):
        key = torch.tensor(((s, 2 * s),), device=GPU, requires_grad=True)
        (grad,) = torch.autograd.grad(fused(key).sum(), (key,))
        want = torch.tensor(((2.0, -1.0),), dtype=torch.float64) / (5 * math.sqrt(5)) / s
        torch.testing.assert_close(grad.cpu().double(), want, rtol=1e-6, atol=0)
    g = torch.Generator().manual_seed(3)
    for width, dtype, tol in ((7, torch.float32, 1e-5), (1000, torch.float32, 1e-5), (70000, torch.float32, 1e-5),
                              (600, torch.bfloat16, 2e-2), (600, torch.float16, 4e-3)):
        # rows under the floor, small, unit and large (float16: 1e-9 underflows to zero, whose
        # gradient g / 1e-6 would overflow it)
        tiny = 1e-4 if dtype == torch.float16 else 1e-9
        k = (torch.randn(5, width, generator=g) * torch.tensor([tiny, 1e-3, 1.0, 10.0, 1e4])[:, None]).to(dtype)
        up = torch.randn(5, width, generator=g).to(dtype)
        kg = k.to(GPU).requires_grad_()
        (grad,) = torch.autograd.grad((fused(kg).float() * up.to(GPU).float()).sum(), (kg,))
        kr = k.double().requires_grad_()
        (want,) = torch.autograd.grad((normalize_keys(kr) * up.double()).sum(), (kr,))
        assert grad.dtype == dtype
        for row in range(5):  # each row on its own scale
            scale = want[row].abs().max().item()
            torch.testing.assert_close(grad[row].cpu().double() / scale, want[row] / scale, rtol=tol, atol=tol)


def test_normalize_keys_empty_and_refusals():
    # tests/test_recurrence_review.py:81-87: empty arrays keep their shape, with a gradient
    from vesper.contracts import ContractError
    from vesper.kernels.keys import normalize_keys as fused

    for shape in ((0, 3), (2, 0)):
        key = torch.empty(shape, device=GPU, requires_grad=True)
        out = fused(key)
        assert out.shape == key.shape
        (grad,) = torch.autograd.grad(out.sum(), (key,))
        assert grad.shape == key.shape
    with pytest.raises(ContractError, match="CUDA only"):
        fused(torch.ones(2, 3))
    with pytest.raises(ContractError, match="dtype"):
        fused(torch.ones(2, 3, dtype=torch.float64, device=GPU))
