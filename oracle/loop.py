"""CPU oracle of the looped column with per-token halting (test infrastructure only; see ``oracle/__init__.py``).

Restated from the reference's pass loop and column:

- ``loop_forward`` follows ``Loop.forward`` (``vesper/loop.py:415-453``) with a given exit trace
  (``TraceRule``, ``vesper/loop.py:203-240``): every pass runs over every token; after a pass the
  column's outputs at inactive positions are zeroed (``:441-442``); the tokens halting now freeze
  the projections they wrote (``_merge``, ``:523-537``), which every later pass writes again in
  their place (copy-forward); a halted token's hidden state is carried forward unchanged
  (``:452``); the last pass halts every token still active.
- ``mixer_column_step`` is the column's two mixers as ``Column.step`` orders them
  (``vesper/column.py:709-812``): the pre-normalization (``RMSNorm`` with its gain at one), the
  recurrent projections, the carry merges of ``k, v, beta``
  (``:784-789``), the delta scan, the residual; the pre-normalization and the attention
  projections, the carry merges of the
  attention keys and values (``:795-796``), window attention, the residual; optionally the causal
  key filter before the keys' normalization (``RecurrentSublayer.keys``, ``:255-289``), its
  history carried per pass; optionally the rotary embedding of the attention's queries and keys
  at positions 0..n-1 (``WindowedAttention.project``, ``attention.py:292``). The FFN is not part
  of the mixer path and is left out;
  keys are L2-normalised (``normalize_keys``) as the scan requires, queries are not
  (``RecurrentSublayer.project``, ``column.py:236-253``; ``docs/model-card.md:26``).
- ``mixer_decode_step`` is the same column one token at a time over per-pass KV rings, at a fixed
  depth with every pass dense, as ``decode_step`` (``vesper/decode.py:29-46``) runs it.

Rounding points mirror the GPU path (``vesper/loop.py``): the residual stream stays in the wide
dtype; every matmul takes bf16-rounded operands and returns a bf16-rounded product; the mixers
take bf16 inputs and return bf16 outputs; the scan state stays in the wide dtype.
"""

from __future__ import annotations

from collections.abc import Callable, Sequence
from dataclasses import dataclass

import torch
from torch import Tensor

from oracle.attention import kv_ring_write, ring_attend, rotary, window_attention
from oracle.delta import delta_scan_chunked, delta_scan_step, normalize_keys
from oracle.keys import filter_keys

BF16 = torch.bfloat16


@dataclass(frozen=True)
class Written:
    """What a pass writes per token into its states (``Projections``, ``vesper/column.py:113-137``)."""

    k: Tensor  # [b, n, h, dk]
    v: Tensor  # [b, n, h, dk]
    beta: Tensor  # [b, n, h]
    attn_k: Tensor  # [b, n, hkv, dk]
    attn_v: Tensor  # [b, n, hkv, dk]
    z: Tensor | None = None  # [b, n, h*dk] the key filter's input (with a filter)


# step(x, pass_index, state, carry) -> (out, new_state, written); carry = (active, carried Written)
ColumnStep = Callable[[Tensor, int, Tensor, "tuple[Tensor, Written] | None"], "tuple[Tensor, Tensor, Written]"]


def _where_tokens(mask: Tensor, a: Tensor, b: Tensor) -> Tensor:
    m = mask.reshape(*mask.shape, *([1] * (a.dim() - mask.dim())))
    return torch.where(m, a, b)


def merge(halts: Tensor, fresh: Written, previous: Written) -> Written:
    """Tokens halting now freeze their fresh projections; the others keep the previous ones (``loop.py:523-537``)."""
    z = None if fresh.z is None or previous.z is None else _where_tokens(halts, fresh.z, previous.z)
    return Written(*(_where_tokens(halts, f, p) for f, p in zip(
        (fresh.k, fresh.v, fresh.beta, fresh.attn_k, fresh.attn_v),
        (previous.k, previous.v, previous.beta, previous.attn_k, previous.attn_v))), z=z)


def carry_in(active: Tensor, fresh: Tensor, carried: Tensor) -> Tensor:
    """``_carry`` (``vesper/column.py:140-143``): fresh where active, the carried value elsewhere."""
    return _where_tokens(active, fresh, carried)


@dataclass(frozen=True)
class LoopOutput:
    y: Tensor  # [b, n, d] the hidden state each token halted with
    states: tuple[Tensor, ...]  # one scan state per pass
    n_iters: Tensor  # int32 [b, n] passes each token was active in
    per_pass: tuple[Tensor, ...]  # each pass's column output, zero at inactive positions


def loop_forward(x0: Tensor, step: ColumnStep, states: Sequence[Tensor], exits: Sequence[Tensor]) -> LoopOutput:
    """Run ``len(states)`` passes of one column with exits given per pass (``exits[t]`` bool ``[b, n]``).

    A token that is active at pass ``t`` and has ``exits[t]`` set halts after that pass; the last
    pass halts every token (``loop.py:443``, ``last=t == runs - 1``).
    """
    passes = len(states)
    if len(exits) < passes:
        raise ValueError(f"{passes} passes need {passes} exit masks, got {len(exits)}")
    b, n = x0.shape[0], x0.shape[1]
    active = torch.ones(b, n, dtype=torch.bool)
    n_iters = torch.zeros(b, n, dtype=torch.int32)
    carried: Written | None = None
    x = x0
    new_states = list(states)
    per_pass = []
    for t in range(passes):
        carry = None if carried is None else (active, carried)
        h, new_states[t], written = step(x, t, new_states[t], carry)
        h = _where_tokens(active, h, torch.zeros_like(h))
        halts = active & (exits[t] | (t == passes - 1))
        n_iters = n_iters + active.to(torch.int32)
        per_pass.append(h)
        carried = written if carried is None else merge(halts, written, carried)
        x = _where_tokens(active, h, x)
        active = active & ~halts
    return LoopOutput(y=x, states=tuple(new_states), n_iters=n_iters, per_pass=tuple(per_pass))


RMS_EPS = 1e-6  # column.py:55
RMS_SCALE_FLOOR = 1e-3  # column.py:56


def rms_norm(x: Tensor) -> Tensor:
    """``RMSNorm`` with its gain at one (its initial value), ``column.py:146-188``: ``x / sqrt(mean(x^2)
    + 1e-6)``, computed scale-safely (each row divided by its peak magnitude floored at 1e-3 first),
    in the input's dtype or float32, whichever is wider. The pre-normalization of both sublayers in
    ``Column.step`` (``column.py:779``, ``:793``)."""
    wide = x.to(torch.promote_types(x.dtype, torch.float32))
    scale = wide.abs().amax(dim=-1, keepdim=True).clamp_min(RMS_SCALE_FLOOR)
    scaled = wide / scale
    rms = torch.sqrt(scaled.square().mean(dim=-1, keepdim=True) + RMS_EPS / (scale * scale))
    return (scaled / rms).to(x.dtype)


def _bf(t: Tensor) -> Tensor:
    """Round to bfloat16 and come back to the wide dtype."""
    return t.to(BF16).to(t.dtype)


def _mm(x: Tensor, w: Tensor) -> Tensor:
    """A bf16 matmul as the GPU path runs it: bf16 operands, a wide product, a bf16 result."""
    return _bf(_bf(x) @ _bf(w))


@dataclass(frozen=True)
class MixerWeights:
    """Per-pass projection weights ``[d, out]`` (``x @ w``)."""

    wq: Sequence[Tensor]
    wk: Sequence[Tensor]
    wv: Sequence[Tensor]
    wb: Sequence[Tensor]  # [d, h]: the write-strength logits
    waq: Sequence[Tensor]
    wak: Sequence[Tensor]
    wav: Sequence[Tensor]
    heads: int
    kv_heads: int
    head_dim: int
    window: int
    taps: Sequence[Tensor] | None = None  # per pass [K, h*dk]: the causal key filter, or none
    rotary_base: float | None = None  # the attention's rotary embedding of q and k, or none


def _keys(weights: MixerWeights, t: int, z: Tensor, history: Tensor | None, rnd: Callable[[Tensor], Tensor]
          ) -> tuple[Tensor, Tensor | None]:
    """``RecurrentSublayer.keys`` (``column.py:255-289``): the filter (if any), then ``normalize_keys``."""
    b, n, _ = z.shape
    h, dk = weights.heads, weights.head_dim
    if weights.taps is None:
        return rnd(normalize_keys(z.view(b, n, h, dk))), history
    assert history is not None
    keys, nxt = filter_keys(z, history, weights.taps[t], h)
    return rnd(keys), nxt


def mixer_column_step(weights: MixerWeights, masked: bool = True, bf16: bool = True) -> ColumnStep:
    """The config's column: delta scan then window attention, each with its residual (see module doc).

    With ``masked`` the mixers take the active mask (inactive outputs zero, their writes kept);
    without it they run densely over every token, as the reference's mixers do. With a key filter
    (``weights.taps``) a pass's state is ``(scan state, key history)`` and a halted token's key
    input is carried into the filter, its key after it (``column.py:779-789``). ``bf16`` False
    drops the bf16 rounding points (the arithmetic alone, in the inputs' dtype).
    """
    h, hkv, dk, w = weights.heads, weights.kv_heads, weights.head_dim, weights.window
    rnd = _bf if bf16 else (lambda t: t)

    def mm(x: Tensor, m: Tensor) -> Tensor:
        return _mm(x, m) if bf16 else x @ m

    def step(x: Tensor, t: int, state, carry: tuple[Tensor, Written] | None):
        b, n, _ = x.shape
        active = None if carry is None else carry[0]
        mask = active if masked else None
        scan_state, history = state if weights.taps is not None else (state, None)
        xn = rms_norm(x)
        q = mm(xn, weights.wq[t]).view(b, n, h, dk)
        z = mm(xn, weights.wk[t]).view(b, n, h * dk)
        if carry is not None and carry[1].z is not None:
            z = carry_in(active, z, carry[1].z)
        k, history = _keys(weights, t, z, history, rnd)
        v = mm(xn, weights.wv[t]).view(b, n, h, dk)
        beta = rnd(torch.sigmoid(mm(xn, weights.wb[t])))
        if carry is not None:
            k, v, beta = (carry_in(active, f, c) for f, c in zip((k, v, beta), (carry[1].k, carry[1].v, carry[1].beta)))
        r, new_state = delta_scan_chunked(q, k, v, beta, scan_state, 64, active=mask)
        x1 = x + rnd(r).reshape(b, n, h * dk)
        x1n = rms_norm(x1)
        aq = mm(x1n, weights.waq[t]).view(b, n, h, dk)
        ak = mm(x1n, weights.wak[t]).view(b, n, hkv, dk)
        av = mm(x1n, weights.wav[t]).view(b, n, hkv, dk)
        if weights.rotary_base is not None:  # WindowedAttention.project (attention.py:292), positions 0..n-1
            pos = torch.arange(n).expand(b, n)
            aq, ak = rnd(rotary(aq, pos, weights.rotary_base)), rnd(rotary(ak, pos, weights.rotary_base))
        if carry is not None:
            ak, av = (carry_in(active, f, c) for f, c in zip((ak, av), (carry[1].attn_k, carry[1].attn_v)))
        a = window_attention(aq, ak, av, w, active=mask)
        x2 = x1 + rnd(a).reshape(b, n, h * dk)
        written = Written(k=k, v=v, beta=beta, attn_k=ak, attn_v=av, z=z if weights.taps is not None else None)
        return x2, (new_state, history) if weights.taps is not None else new_state, written

    return step


# one pass's decoding state: (scan state, key history or None, (ring k, ring v, ring pos, ring valid))
DecodeState = tuple[Tensor, "Tensor | None", tuple[Tensor, Tensor, Tensor, Tensor]]


def cold_decode_states(weights: MixerWeights, b: int, dtype: torch.dtype) -> list[DecodeState]:
    """Zero scan states and key histories, unwritten rings (``init_column_state(..., ring=True)``,
    ``column.py:465-500``), one per pass."""
    h, hkv, dk, w = weights.heads, weights.kv_heads, weights.head_dim, weights.window
    out = []
    for t in range(len(weights.wq)):
        hist = None if weights.taps is None else torch.zeros(b, weights.taps[t].shape[0] - 1, h * dk, dtype=dtype)
        ring = (torch.zeros(b, w, hkv, dk, dtype=dtype), torch.zeros(b, w, hkv, dk, dtype=dtype),
                torch.zeros(b, w, dtype=torch.long), torch.zeros(b, w, dtype=torch.bool))
        out.append((torch.zeros(b, h, dk, dk, dtype=dtype), hist, ring))
    return out


def mixer_decode_step(weights: MixerWeights, depth: int, bf16: bool = True
                      ) -> Callable[[Tensor, Tensor, Sequence[DecodeState]], tuple[Tensor, list[DecodeState]]]:
    """One token per row through the first ``depth`` passes, every pass dense (``DenseRule``):
    the column's step with the delta rule's single step (``recurrence.py:143-163``) and attention
    over the pass's ring followed by the ring write (``attend_ring``, ``attention.py:298-338``),
    as ``decode_step`` (``vesper/decode.py:29-46``) runs the column. Returns ``(y [b, 1, d], states)``
    with new state objects for the first ``depth`` passes and the others unchanged."""
    h, hkv, dk, w = weights.heads, weights.kv_heads, weights.head_dim, weights.window
    rnd = _bf if bf16 else (lambda t: t)

    def mm(x: Tensor, m: Tensor) -> Tensor:
        return _mm(x, m) if bf16 else x @ m

    def step(x: Tensor, pos: Tensor, states: Sequence[DecodeState]) -> tuple[Tensor, list[DecodeState]]:
        b = x.shape[0]
        new = list(states)
        for t in range(depth):
            scan_state, history, (rk, rv, rp, rvalid) = states[t]
            xn = rms_norm(x)
            q = mm(xn, weights.wq[t]).view(b, 1, h, dk)
            z = mm(xn, weights.wk[t]).view(b, 1, h * dk)
            k, history = _keys(weights, t, z, history, rnd)
            v = mm(xn, weights.wv[t]).view(b, 1, h, dk)
            beta = rnd(torch.sigmoid(mm(xn, weights.wb[t])))
            o, scan_state = delta_scan_step(q[:, 0], k[:, 0], v[:, 0], beta[:, 0], scan_state)
            x1 = x + rnd(o).reshape(b, 1, h * dk)
            x1n = rms_norm(x1)
            aq = mm(x1n, weights.waq[t]).view(b, 1, h, dk)
            ak = mm(x1n, weights.wak[t]).view(b, 1, hkv, dk)
            av = mm(x1n, weights.wav[t]).view(b, 1, hkv, dk)
            if weights.rotary_base is not None:
                aq, ak = rnd(rotary(aq, pos, weights.rotary_base)), rnd(rotary(ak, pos, weights.rotary_base))
            a = ring_attend(aq, ak, av, pos, rk, rv, rp, rvalid, w)
            ring = kv_ring_write(rk, rv, rp, rvalid, ak, av, pos)
            x = x1 + rnd(a).reshape(b, 1, h * dk)
            new[t] = (scan_state, history, ring)
        return x, new

    return step
