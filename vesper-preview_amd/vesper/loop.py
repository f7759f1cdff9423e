"""The looped column with per-token halting, on MI355X: the caller of the mixers with an active mask.

This is the pass loop of the reference's ``Loop.forward`` (``vesper/loop.py:415-453``) driven by
a given exit trace (``TraceRule``, ``:203-240``), over a column reduced to its two mixers in the
order of ``Column.step`` (``vesper/column.py:709-812``):

- recurrent sublayer: the pre-normalization (``RMSNorm`` with its gain at one, ``column.py:146-188``),
  projections ``q, z, v, beta`` of the pass input (one ``vsp_project_bf16`` launch; the query
  is not normalized, ``column.py:247``; ``beta = sigmoid``), the key from the key input ``z`` (``normalize_keys``, after
  the causal key filter when the column has one, ``column.py:255-289``, with the pass's key
  history), the carry merges for halted tokens (their key input before the filter, ``k, v, beta``
  after, ``column.py:779-789``), the delta scan (``vsp_delta_scan_bf16`` with the active mask),
  the residual;
- attention sublayer: the pre-normalization, projections (one launch), the rotary embedding of the queries and
  keys at positions 0..n-1 (``attention.py:178-217, 292``; one launch, ``vsp_rotary_qk_bf16``), the
  carry merges of the attention keys and values
  (``column.py:795-796``), window attention over the chunk (``vsp_window_attn_bf16`` with the
  active mask), the residual.

The loop zeroes inactive outputs, freezes the projections of tokens as they halt and writes them
into every later pass's state (copy-forward), and carries halted tokens' hidden states forward
unchanged (``loop.py:441-453``, ``:523-537``). By default (``copy_forward="fused"``) the kernels read
the carried rows of inactive tokens inside their loads (the key filter's ``carried_z``, the scan's
``carried``, the attention's ``carried``) and one launch per pass (``copy_rows_where``) freezes the
halting tokens' projections into the carried buffers and carries the hidden state, in place of the
reference's ``where`` merges; ``copy_forward="where"`` runs those merges as torch selects.

All passes run even when no token is active any more. The FFN is not part of the mixer path and
is left out. The residual stream stays in float32 (autocast's convention); matmuls and mixers run
in bfloat16 with the scan state in float32. Forward only.
"""

from __future__ import annotations

from collections.abc import Sequence
from dataclasses import dataclass

import torch
from torch import Tensor

from vesper.attention import rotary_qk
from vesper.column import recurrent_keys
from vesper.contracts import ContractError, Dims, check_shape
from vesper.kernels.carry import copy_rows_where, halt_step, residual_rows_where
from vesper.kernels.delta_scan import delta_scan_fused
from vesper.kernels.keys import fused_keys
from vesper.kernels.norm import projection, rms_norm_bf16
from vesper.kernels.window_attn import window_attention

BF16 = torch.bfloat16


_ONES: dict[tuple[int, torch.device], Tensor] = {}


def _normalize(x: Tensor, heads: int) -> Tensor:
    """``normalize_keys`` (``vesper/recurrence.py:91-115``) per head of ``x [b, n, heads * dk]``
    (bfloat16, on the GPU): divide by the head's peak magnitude (floored at 1e-6), then by the norm
    of the scaled head floored at one, in float32, returned as bfloat16 ``[b, n, heads, dk]``. One
    launch of the key kernel with a single tap of ones (its filter then passes the input through)
    instead of a chain of elementwise kernels."""
    d = x.shape[-1]
    key = (d, x.device)
    if key not in _ONES:
        _ONES[key] = torch.ones(1, d, dtype=torch.float32, device=x.device)
    return fused_keys(x, x.new_empty(x.shape[0], 0, d, dtype=torch.float32), _ONES[key], heads)


def _where_tokens(mask: Tensor, a: Tensor, b: Tensor) -> Tensor:
    return torch.where(mask.reshape(*mask.shape, *([1] * (a.dim() - mask.dim()))), a, b)


@dataclass(frozen=True)
class Written:
    """What a pass writes per token into its states (the mixer part of ``Projections``)."""

    k: Tensor
    v: Tensor
    beta: Tensor
    attn_k: Tensor
    attn_v: Tensor
    z: Tensor | None = None  # the key filter's input, with a filter

    def merged(self, halts: Tensor, previous: Written) -> Written:
        """Tokens halting now freeze these projections; the others keep ``previous`` (``loop.py:523-537``)."""
        z = None if self.z is None or previous.z is None else _where_tokens(halts, self.z, previous.z)
        return Written(*(_where_tokens(halts, a, b) for a, b in zip(
            (self.k, self.v, self.beta, self.attn_k, self.attn_v),
            (previous.k, previous.v, previous.beta, previous.attn_k, previous.attn_v))), z=z)


@dataclass(frozen=True)
class LoopResult:
    y: Tensor  # [b, n, d] float32: the hidden state each token halted with
    states: tuple[Tensor, ...]  # the scan state of every pass, [b, h, dk, dk] float32
    n_iters: Tensor  # int32 [b, n]: passes each token was active in
    histories: tuple[Tensor, ...] | None = None  # each pass's next key history, with a filter


class LoopedColumn:
    """One column's mixers run for ``passes`` passes with per-pass projection weights.

    Weights are ``[d, out]`` bfloat16 tensors per pass (``x @ w``): ``wq, wk, wv [d, h*dk]``,
    ``wb [d, h]``, ``waq [d, h*dk]``, ``wak, wav [d, hkv*dk]``; optional ``taps`` are the key
    filter's ``[K, h*dk]`` float32 taps per pass (``wk`` then gives the filter's input).
    """

    def __init__(self, weights: dict[str, Sequence[Tensor]], heads: int, kv_heads: int, head_dim: int,
                 window: int, taps: Sequence[Tensor] | None = None, copy_forward: str = "fused",
                 rotary_base: float | None = 10000.0) -> None:
        names = ("wq", "wk", "wv", "wb", "waq", "wak", "wav")
        missing = [n for n in names if n not in weights]
        if missing:
            raise ValueError(f"missing weights: {missing}")
        self.passes = len(weights["wq"])
        if any(len(weights[n]) != self.passes for n in names):
            raise ValueError("every weight needs one tensor per pass")
        self.w = {n: list(weights[n]) for n in names}
        self.heads, self.kv_heads, self.head_dim, self.window = heads, kv_heads, head_dim, window
        if taps is not None and len(taps) != self.passes:
            raise ValueError("the key filter needs one set of taps per pass")
        self.taps = None if taps is None else list(taps)
        if copy_forward not in ("fused", "where"):
            raise ValueError(f"copy_forward is 'fused' or 'where', got {copy_forward!r}")
        self.copy_forward = copy_forward
        self.rotary_base = rotary_base
        self._positions: dict[tuple[int, int, torch.device], Tensor] = {}
        # Each sublayer's projections stacked into one [p, d, h*dk] weight per pass (narrower ones
        # zero-padded), so one batched GEMM gives each projection as its own contiguous block
        # instead of one GEMM launch per projection. Built once from ``weights``.
        hd = heads * head_dim

        def padded(w: Tensor) -> Tensor:
            return w if w.shape[1] == hd else torch.nn.functional.pad(w, (0, hd - w.shape[1]))

        self.w_rec = [torch.stack([padded(self.w[n][t]) for n in ("wq", "wk", "wv", "wb")]) for t in range(self.passes)]
        self.w_attn = [torch.stack([padded(self.w[n][t]) for n in ("waq", "wak", "wav")]) for t in range(self.passes)]
        self._decode_w: dict[int, tuple[Tensor, Tensor]] = {}

    def project_rec(self, t: int, xb: Tensor) -> tuple[Tensor, Tensor, Tensor, Tensor]:
        """Pass ``t``'s recurrent projections of ``xb [b, n, d]`` (bf16), one launch:
        ``q_in [b, n, h*dk]`` (before normalization), ``z [b, n, h*dk]`` (the key input),
        ``v [b, n, h, dk]``, ``beta = sigmoid [b, n, h]``."""
        b, n, d = xb.shape
        h, dk = self.heads, self.head_dim
        hd = h * dk
        q_in, z, v, beta = self._project(xb.reshape(b * n, d), t, 0, (hd, hd, hd, h), sigmoid_block=3)
        return q_in.view(b, n, hd), z.view(b, n, hd), v.view(b, n, h, dk), beta.view(b, n, h)

    def _project(self, xb: Tensor, t: int, which: int, used: tuple[int, ...],
                 sigmoid_block: int | None = None) -> list[Tensor]:
        """The blocks of pass ``t``'s stacked weight (``which``: 0 recurrent, 1 attention) applied
        to ``xb [M, d]``, each as its own ``[M, used_j]`` tensor: one ``vsp_project_bf16`` launch
        when ``d`` is a multiple of 64, else the batched library GEMM over the padded stack."""
        if xb.shape[1] % 64 == 0:
            return projection(xb, self.decode_weights(t)[which], used, sigmoid_block=sigmoid_block)
        y = torch.matmul(xb, (self.w_rec if which == 0 else self.w_attn)[t])
        outs = [y[j][:, :u].contiguous() for j, u in enumerate(used)]
        if sigmoid_block is not None:  # bf16 in and out, float32 inside
            outs[sigmoid_block] = torch.sigmoid(outs[sigmoid_block])
        return outs

    def decode_weights(self, t: int) -> tuple[Tensor, Tensor]:
        """Pass ``t``'s stacked recurrent and attention weights with each block transposed
        (``[p, h*dk, d]``), the operand layout of the decode step's fused projection; made once."""
        if t not in self._decode_w:
            self._decode_w[t] = (self.w_rec[t].transpose(1, 2).contiguous(),
                                 self.w_attn[t].transpose(1, 2).contiguous())
        return self._decode_w[t]

    def project_attn(self, t: int, xb: Tensor, pos: Tensor | None = None) -> tuple[Tensor, Tensor, Tensor]:
        """Pass ``t``'s attention projections of ``xb [b, n, d]`` (bf16), one launch, with the
        queries and keys rotated at positions ``pos [b, n]`` (default ``0..n-1``) in one launch
        when the column has a rotary base (``WindowedAttention.project``, ``attention.py:269-292``)."""
        b, n, d = xb.shape
        h, hkv, dk = self.heads, self.kv_heads, self.head_dim
        yq, yk, yv = self._project(xb.reshape(b * n, d), t, 1, (h * dk, hkv * dk, hkv * dk))
        aq, ak = yq.view(b, n, h, dk), yk.view(b, n, hkv, dk)
        if self.rotary_base is not None:
            if pos is None:
                key = (b, n, xb.device)
                pos = self._positions.get(key)
                if pos is None:
                    pos = torch.arange(n, device=xb.device).expand(b, n).contiguous()
                    self._positions[key] = pos
            aq, ak = rotary_qk(aq, ak, pos, self.rotary_base)
        return aq, ak, yv.view(b, n, hkv, dk)

    @property
    def key_history(self) -> int:
        """Key inputs a pass carries across a chunk boundary: ``K - 1`` (``column.py:75-77``)."""
        return 0 if self.taps is None else int(self.taps[0].shape[0]) - 1

    @classmethod
    def random(cls, d: int, heads: int, kv_heads: int, head_dim: int, window: int, passes: int, seed: int,
               device: torch.device, key_conv: int = 0, copy_forward: str = "fused",
               rotary_base: float | None = 10000.0) -> LoopedColumn:
        """Fixed random weights ~ N(0, 1/d) from a CPU generator (the same values on any device);
        with ``key_conv`` a filter of that width, taps ~ U(-1/sqrt(K), 1/sqrt(K)) as the
        reference draws them (``column.py:231-233``)."""
        g = torch.Generator().manual_seed(seed)
        shapes = {"wq": heads * head_dim, "wk": heads * head_dim, "wv": heads * head_dim, "wb": heads,
                  "waq": heads * head_dim, "wak": kv_heads * head_dim, "wav": kv_heads * head_dim}
        weights: dict[str, list[Tensor]] = {n: [] for n in shapes}
        for _ in range(passes):
            for name, out in shapes.items():
                weights[name].append((torch.randn(d, out, generator=g) / d**0.5).to(device, BF16))
        taps = None
        if key_conv:
            bound = 1.0 / key_conv**0.5
            taps = [(torch.rand(key_conv, heads * head_dim, generator=g) * (2 * bound) - bound).to(device)
                    for _ in range(passes)]
        return cls(weights, heads, kv_heads, head_dim, window, taps, copy_forward, rotary_base)

    def keys(self, t: int, z: Tensor, history: Tensor | None, active: Tensor | None = None,
             carried_z: Tensor | None = None) -> tuple[Tensor, Tensor | None]:
        """Pass ``t``'s keys of key inputs ``z [b, n, h*dk]`` (bf16) and the next key history
        (with ``carried_z``, inactive tokens' inputs come from it)."""
        b, n, _ = z.shape
        if self.taps is None:
            return _normalize(z, self.heads), history
        assert history is not None
        return recurrent_keys(z, history, self.taps[t], self.heads, active=active, carried_z=carried_z)

    def _step(self, x: Tensor, t: int, state: Tensor, history: Tensor | None, active: Tensor | None,
              carried: Written | None) -> tuple[tuple[Tensor, Tensor], Tensor, Tensor | None, Written]:
        """One pass over ``x``; returns ``(x1, a)`` (the hidden state after the recurrent sublayer
        and the attention's output: the pass's output is ``x1 + a``), the new state and history, and
        the projections the pass wrote."""
        b, n, d = x.shape
        h, dk = self.heads, self.head_dim
        xb = rms_norm_bf16(x)
        q_in, z, v, beta = self.project_rec(t, xb)
        q = q_in.view(b, n, h, dk)  # the scan's query is not normalized (column.py:247)
        fused = self.copy_forward == "fused" and carried is not None and active is not None
        where = self.copy_forward == "where" and carried is not None and active is not None
        if where and carried is not None and active is not None and carried.z is not None:
            z = _where_tokens(active, z, carried.z)  # a halted token's frozen key input, before the filter
        if fused and carried is not None and carried.z is not None:
            k, history = self.keys(t, z, history, active, carried.z)  # the filter reads carried inputs
        else:
            k, history = self.keys(t, z, history)
        if where and carried is not None and active is not None:
            k = _where_tokens(active, k, carried.k)
            v = _where_tokens(active, v, carried.v)
            beta = _where_tokens(active, beta, carried.beta)
        if fused and carried is not None:  # the scan reads inactive tokens' k, v, beta from the carried ones
            r, new_state = delta_scan_fused(q, k, v, beta, state, active=active,
                                            carried=(carried.k, carried.v, carried.beta))
        else:
            r, new_state = delta_scan_fused(q, k, v, beta, state, active=active)
        # x1 = x + r (float32, promoted in the add) and its norm, in one launch
        x1 = torch.empty_like(x)
        aq, ak, av = self.project_attn(t, rms_norm_bf16(x, residual=r.reshape(b, n, h * dk), sum_out=x1))
        if where and carried is not None and active is not None:
            ak = _where_tokens(active, ak, carried.attn_k)
            av = _where_tokens(active, av, carried.attn_v)
        if fused and carried is not None:
            a = window_attention(aq, ak, av, self.window, active=active, carried=(carried.attn_k, carried.attn_v))
        else:
            a = window_attention(aq, ak, av, self.window, active=active)
        written = Written(k=k, v=v, beta=beta, attn_k=ak, attn_v=av, z=z if self.taps is not None else None)
        return (x1, a.reshape(b, n, h * dk)), new_state, history, written

    def forward(self, x0: Tensor, states: Sequence[Tensor], exits: Sequence[Tensor],
                histories: Sequence[Tensor] | None = None) -> LoopResult:
        """All passes over ``x0 [b, n, d]`` (float32, on the GPU).

        Args:
            x0: the chunk's input hidden states.
            states: one float32 scan state ``[b, h, dk, dk]`` per pass.
            exits: per pass a bool ``[b, n]``: an active token with its exit set halts after the
                pass; the last pass halts every token still active.
            histories: with a key filter, one float32 key history ``[b, K-1, h*dk]`` per pass.

        Raises:
            ContractError: on shapes or dtypes outside that contract.
        """
        dims: Dims = {"d": self.heads * self.head_dim, "h": self.heads, "dk": self.head_dim}
        check_shape("x0", x0, ("b", "n", "d"), dims, torch.float32)
        if len(states) != self.passes or len(exits) < self.passes:
            raise ContractError(f"{self.passes} passes need {self.passes} states and exit masks")
        for t in range(self.passes):
            check_shape(f"states[{t}]", states[t], ("b", "h", "dk", "dk"), dims, torch.float32)
            check_shape(f"exits[{t}]", exits[t], ("b", "n"), dims, torch.bool)
        if self.taps is not None:
            if histories is None or len(histories) != self.passes:
                raise ContractError(f"a column with a key filter needs {self.passes} key histories")
            dims["w"] = self.key_history
            for t in range(self.passes):
                check_shape(f"histories[{t}]", histories[t], ("b", "w", "d"), dims, torch.float32)
        b, n = dims["b"], dims["n"]
        with torch.no_grad():
            active = torch.ones(b, n, dtype=torch.bool, device=x0.device)
            n_iters = torch.zeros(b, n, dtype=torch.int32, device=x0.device)
            carried: Written | None = None
            x = x0
            new_states = list(states)
            new_histories: list[Tensor | None] = list(histories) if histories is not None else [None] * self.passes
            for t in range(self.passes):
                # pass 0 runs with every token active: the unmasked kernels, as the reference's
                # carry-free first pass
                mask = None if carried is None else active
                (x1, a), new_states[t], new_histories[t], written = self._step(x, t, new_states[t],
                                                                               new_histories[t], mask, carried)
                # halts = active & exit (all active on the last pass), n_iters += active, and the
                # next pass's active & ~halts: one launch
                halts, next_active = halt_step(active, exits[t] if t < self.passes - 1 else None, n_iters)
                if carried is None:  # pass 0: every token active, the fresh projections are the carried ones
                    carried = written
                    x = torch.empty_like(x1)  # this loop's own buffer from here on
                    residual_rows_where(x1, a, x, None)
                elif self.copy_forward == "where":
                    h = x1 + a
                    h = _where_tokens(active, h, torch.zeros_like(h))
                    carried = written.merged(halts, carried)
                    x = _where_tokens(active, h, x)
                else:
                    # one launch: the tokens halting now freeze their fresh projections into the
                    # carried buffers (none after the last pass); then the active tokens' hidden
                    # states x1 + a go straight into x (this loop's own buffer from pass 1 on)
                    items: list[tuple[Tensor, Tensor, Tensor]] = []
                    if t < self.passes - 1:
                        items = [(written.k, carried.k, halts), (written.v, carried.v, halts),
                                 (written.beta, carried.beta, halts), (written.attn_k, carried.attn_k, halts),
                                 (written.attn_v, carried.attn_v, halts)]
                        if written.z is not None and carried.z is not None:
                            items.append((written.z, carried.z, halts))
                    copy_rows_where(items)
                    residual_rows_where(x1, a, x, active)
                active = next_active
        hist_out = tuple(t for t in new_histories if t is not None) if self.taps is not None else None
        return LoopResult(y=x, states=tuple(new_states), n_iters=n_iters, histories=hist_out)
