"""Single-token decoding of the looped column on MI355X, captured as one HIP graph.

The reference decodes greedily through ``CapturedDecoder`` (``vesper/decode.py:49-97``): every new
token runs one single-token step at a fixed depth, every pass dense (``DenseRule``), each pass
carrying its recurrent state, key history and ``RingKVCache`` (``init_column_state(...,
ring=True)``, ``vesper/column.py:465-500``), so the step's shapes never change and one captured
graph serves every token (``WarmedGraph``, ``vesper/graphs.py:180-240``: a few eager warm-up
calls, one capture, replays). This module is that decoder for the column's two mixers
(``vesper.loop.LoopedColumn``): per pass the projections, the key filter
(``vsp_key_filter_*``) over the pass's key history, the delta rule's single step
(``vsp_delta_step_*``, state in place) and attention over the pass's ring with the new token
written into its slot by the same launch (``vsp_ring_attn_*``, in place).

Differences from the reference's decoder, both for throughput on one GPU: a batch of rows decodes
together (each row at its own position; the ring kernel writes one slot per row), and the state
is updated in place: ``decode_step`` writes the new states into the tensors it was given and
returns them, and ``CapturedDecoder.step`` copies only those inputs that are not already its
graph's own buffers (a loop that passes each step's states on copies nothing).
"""

from __future__ import annotations

from collections.abc import Sequence

import torch
from torch import Tensor

from vesper.attention import rotary_inv_freq
from vesper.contracts import ContractError, Dims, check_shape
from vesper.kernels.delta_scan import delta_scan_step_fused, delta_scan_step_keys
from vesper.kernels.norm import decode_projection
from vesper.kernels.ring_attn import RingKVCache, ring_attention
from vesper.loop import BF16, LoopedColumn, _normalize

WARM_STEPS = 3  # eager calls before the capture (vesper/graphs.py:99)
PER_PASS = 6  # flat tensors per pass: scan state, key history, ring keys, values, positions, valid


def cold_states(column: LoopedColumn, b: int, device: torch.device) -> list[Tensor]:
    """A new generation's flat state: per pass a zero float32 scan state ``[b, h, dk, dk]``, a zero
    float32 key history ``[b, K-1, h*dk]`` (``K - 1 = 0`` without a filter) and an unwritten ring
    (bf16 keys and values ``[b, window, hkv, dk]`` of zeros, positions 0, ``valid`` False)."""
    h, hkv, dk, w = column.heads, column.kv_heads, column.head_dim, column.window
    flat: list[Tensor] = []
    for _ in range(column.passes):
        flat += [torch.zeros(b, h, dk, dk, device=device),
                 torch.zeros(b, column.key_history, h * dk, device=device),
                 torch.zeros(b, w, hkv, dk, dtype=BF16, device=device),
                 torch.zeros(b, w, hkv, dk, dtype=BF16, device=device),
                 torch.zeros(b, w, dtype=torch.long, device=device),
                 torch.zeros(b, w, dtype=torch.bool, device=device)]
    return flat


def _check(column: LoopedColumn, x: Tensor, position: Tensor, flat: Sequence[Tensor]) -> None:
    h, hkv, dk, w = column.heads, column.kv_heads, column.head_dim, column.window
    dims: Dims = {"one": 1, "d": h * dk, "h": h, "hkv": hkv, "dk": dk, "w": w, "kh": column.key_history}
    check_shape("x", x, ("b", "one", "d"), dims, torch.float32)
    check_shape("position", position, ("b", "one"), dims, torch.long)
    if len(flat) != PER_PASS * column.passes:
        raise ContractError(f"{column.passes} passes carry {PER_PASS * column.passes} state tensors, got {len(flat)}")
    for t in range(column.passes):
        s, hist, rk, rv, rp, rvalid = flat[PER_PASS * t: PER_PASS * (t + 1)]
        check_shape(f"state[{t}]", s, ("b", "h", "dk", "dk"), dims, torch.float32)
        check_shape(f"key_history[{t}]", hist, ("b", "kh", "d"), dims, torch.float32)
        check_shape(f"ring_k[{t}]", rk, ("b", "w", "hkv", "dk"), dims, BF16)
        check_shape(f"ring_v[{t}]", rv, ("b", "w", "hkv", "dk"), dims, BF16)
        check_shape(f"ring_pos[{t}]", rp, ("b", "w"), dims, torch.long)
        check_shape(f"ring_valid[{t}]", rvalid, ("b", "w"), dims, torch.bool)
    if x.device.type != "cuda":
        raise ContractError(f"the decoder runs on CUDA, x is on {x.device}")


def decode_step(column: LoopedColumn, depth: int, values: Sequence[Tensor],
                workspace: Tensor | None = None) -> list[Tensor]:
    """One token per row through the first ``depth`` passes, every pass dense, eager.

    ``values`` are ``x [b, 1, d]`` float32 (the token's hidden state), its position ``int64
    [b, 1]`` and the flat states (``cold_states``); the result is ``[y [b, 1, d], *flat]`` with the
    flat states updated in place (the same tensor objects). Passes at or past ``depth`` are left
    alone. ``workspace`` is an optional int32 ``[b]`` zero tensor for the ring kernel's arrival
    counters (left zero).

    Raises:
        ContractError: on shapes, dtypes or devices outside that contract, or ``depth`` outside
            ``1..passes``.
    """
    x, position, *flat = values
    _check(column, x, position, flat)
    if not 1 <= depth <= column.passes:
        raise ContractError(f"depth {depth} is outside 1..{column.passes}")
    b, d = x.shape[0], x.shape[2]
    h, hkv, dk = column.heads, column.kv_heads, column.head_dim
    hd = h * dk
    with torch.no_grad():
        # the residual stream between the sublayers: each projection adds the previous mixer's
        # output to it, normalizes and projects in one launch (vsp_decode_proj_bf16)
        xs = x.reshape(b, d)
        pending = None  # the previous pass's attention output, added by the next projection
        rotary = None
        if column.rotary_base is not None:
            rotary = (position.reshape(b), rotary_inv_freq(column.rotary_base, dk, x.device), dk, (0, 1))
        for t in range(depth):
            state, history, rk, rv, rp, rvalid = flat[PER_PASS * t: PER_PASS * (t + 1)]
            w_rec, w_attn = column.decode_weights(t)
            if pending is None:
                q_in, z, v, beta = decode_projection(xs, w_rec, (hd, hd, hd, h), sigmoid_block=3)
            else:
                nxt_x = torch.empty_like(xs)
                q_in, z, v, beta = decode_projection(xs, w_rec, (hd, hd, hd, h), residual=pending, sum_out=nxt_x,
                                                     sigmoid_block=3)
                xs = nxt_x
            q = q_in.view(b, h, dk)  # the scan's query is not normalized (column.py:247)
            if column.taps is None:
                k = _normalize(z.view(b, 1, hd), h)
                o, _ = delta_scan_step_fused(q, k[:, 0], v.view(b, h, dk), beta, state, out_state=state)
            else:  # the key filter inside the step's launch, the history updated in place
                o = delta_scan_step_keys(q, z, v.view(b, h, dk), beta, history, column.taps[t], state)
            x1 = torch.empty_like(xs)
            aq, ak, av = decode_projection(xs, w_attn, (hd, hkv * dk, hkv * dk), residual=o.reshape(b, hd),
                                           sum_out=x1, rotary=rotary)  # q and k rotated as stored
            xs = x1
            aq, ak = aq.view(b, 1, h, dk), ak.view(b, 1, hkv, dk)
            ring = RingKVCache(rk, rv, rp, rvalid, column.window)
            a, _ = ring_attention(aq, ak, av.view(b, 1, hkv, dk), position, ring, inplace=True, check_positions=False,
                                  workspace=workspace)
            pending = a.reshape(b, hd)
        x = (xs + pending).view(b, 1, d)  # float32 (promoted in the add)
    return [x, *flat]


class CapturedDecoder:
    """The column's single-token step at ``depth`` passes, captured on the GPU after warm-up.

    ``start(b)`` gives cold flat states for ``b`` rows; ``step(x, position, flat)`` advances them by
    one token and returns ``(y, flat)``. The first ``WARM_STEPS`` calls run eagerly (on the caller's
    tensors, updated in place), the next one captures the step over the decoder's own copies and
    replays it, every later call replays. After a replay ``y`` and ``flat`` are the graph's own
    buffers: read or pass them on before the next step (passing them back costs no copy). A new
    generation starts from ``start()``'s cold states, copied into the same buffers, so nothing of
    an earlier prompt survives. The shapes (``b`` and the column) are fixed by the capture.

    Raises:
        ContractError: if the column's weights are not on a GPU, or ``depth`` is outside
            ``1..passes``.
    """

    def __init__(self, column: LoopedColumn, depth: int) -> None:
        device = column.w["wq"][0].device
        if device.type != "cuda":
            raise ContractError(f"CapturedDecoder runs on CUDA, the column is on {device}")
        if not 1 <= depth <= column.passes:
            raise ContractError(f"depth {depth} is outside 1..{column.passes}")
        self.column, self.depth, self.device = column, depth, device
        self.eager = 0
        self.captures = 0
        self.replays = 0
        self._graph: torch.cuda.CUDAGraph | None = None
        self._static: list[Tensor] = []
        self._out: list[Tensor] = []
        self._workspace: Tensor | None = None

    def start(self, b: int = 1) -> list[Tensor]:
        """Cold states for a new generation of ``b`` rows, as flat state tensors."""
        return cold_states(self.column, b, self.device)

    def _run(self, values: Sequence[Tensor]) -> list[Tensor]:
        assert self._workspace is not None
        return decode_step(self.column, self.depth, values, self._workspace)

    def step(self, x: Tensor, position: Tensor, flat: Sequence[Tensor]) -> tuple[Tensor, list[Tensor]]:
        """One token per row (``x [b, 1, d]`` float32 at ``position`` int64 ``[b, 1]``): ``(y, flat)``."""
        values = [x, position, *flat]
        _check(self.column, x, position, flat)
        if self._graph is not None:
            # the graph holds the captured workspace and buffers: a call of another shape is refused
            # before anything the graph uses is touched
            for mine, given in zip(self._static, values):
                if mine.shape != given.shape or mine.dtype != given.dtype:
                    raise ContractError(f"the decoder was captured for {tuple(mine.shape)} {mine.dtype}, "
                                        f"got {tuple(given.shape)} {given.dtype}")
        elif self._workspace is None or self._workspace.shape[0] != x.shape[0]:
            self._workspace = torch.zeros(x.shape[0], dtype=torch.int32, device=self.device)
        if self.eager < WARM_STEPS:
            self.eager += 1
            side = torch.cuda.Stream()
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side):
                out = self._run(values)
            torch.cuda.current_stream().wait_stream(side)
            return out[0], out[1:]
        if self._graph is None:
            self._static = [v.clone() for v in values]  # owned buffers, never the caller's
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                self._out = self._run(self._static)
            self._graph = graph
            self.captures += 1
        for mine, given in zip(self._static, values):
            if mine.data_ptr() != given.data_ptr():
                mine.copy_(given)
        self._graph.replay()
        self.replays += 1
        return self._out[0], self._out[1:]
