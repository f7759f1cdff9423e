"""The delta-rule scan on MI355X: hand-written HIP kernels behind the reference's contract.

``delta_scan_fused`` and ``delta_scan_fused_fp32`` keep the signatures, tensor contracts and
refusals of the reference's ``vesper/kernels/delta_scan.py:132-187`` (registry rows
``docs/registry.md:29-30``): ``q, k, v [b, n, h, dk]``, ``beta [b, n, h]``, the state
``[b, h, dk, dk]`` in float32 read as ``H^T q`` after the token's own write, no query scaling, keys
already normalised. Where the reference calls fla-core's Triton kernels, these call
``libvesper_kernels.so`` through its C ABI (``include/vesper_kernels.h``) on torch's current stream:

- ``delta_scan_fused``: bfloat16 inputs and output, float32 state; the chunked WY/UT scan with
  bf16 MFMA contractions (``vsp_delta_scan_bf16``).
- ``delta_scan_fused_fp32``: float32 throughout, fp32 MFMA (``vsp_delta_scan_f32``).
- ``delta_scan_step_fused``: one token per row, the contract of ``vesper/recurrence.py:143-163``
  (``delta_scan_step``), for decoding (``vsp_delta_step_f32`` / ``vsp_delta_step_bf16``).

Each takes an optional keyword ``active`` (bool ``[b, n]``, ``[b]`` for the step): inactive tokens
still write the state; their outputs are zero (``vesper/loop.py:24-26``, ``:441-442``). ``None`` is
exactly the reference behaviour. With ``active``, the chunked scans also take ``carried = (k, v,
beta)``: the copy-forward of halted tokens (``vesper/column.py:779-789``), read inside the kernels'
loads (``vsp_delta_scan_carried_*``) where a token is inactive, in place of the ``where`` merges
before the call. The two chunked scans are autograd functions: their backward
(``vsp_delta_scan_backward_*``) gives the gradients of ``q, k, v, beta`` and the initial state at
every width up to ``MAX_HEAD_DIM``, as the reference's kernels do. Its chunked kernels tile widths
16, 32, 64 and, on the bf16 entry, 128; wider heads run a wide backward (state checkpoints from the
token-serial forward, then chunk and value-group kernels) that takes multiples of 16. A width in
between runs zero-padded to the next width taken, which leaves every output and gradient unchanged.
The single step is forward only (inputs that require a gradient are refused while grad mode is on).
"""

from __future__ import annotations

from typing import Any

import torch
from torch import Tensor

from vesper.contracts import ContractError, Dims, check_shape
from vesper.kernels import _lib

MAX_HEAD_DIM = 256  # delta_scan.py:41 in the reference; the HIP kernels take any width up to it
# the widths the tiled backward kernels take, on the bf16 and on the fp32 entry; wider heads take
# the wide backward at any multiple of 16 up to MAX_HEAD_DIM
BACKWARD_HEAD_DIMS = {False: (16, 32, 64, 128), True: (16, 32, 64)}


def backward_width(dk: int, fp32: bool) -> int:
    """The width the backward runs a head of width ``dk`` at (zero-padded up to it): the next tiled
    width, else the next multiple of 16."""
    tiled = next((w for w in BACKWARD_HEAD_DIMS[fp32] if w >= dk), None)
    return tiled if tiled is not None else -(-dk // 16) * 16
INPUT_DTYPE = torch.bfloat16  # delta_scan_fused's q, k, v, beta
FP32_INPUT_DTYPE = torch.float32  # delta_scan_fused_fp32's q, k, v, beta
STATE_DTYPE = torch.float32


def fused_scan_available() -> bool:
    """Whether the fused scans can run here: a HIP device and the built kernel library."""
    return torch.cuda.is_available() and _lib.available()


def _checked_length(q: Tensor, k: Tensor, v: Tensor, beta: Tensor, state: Tensor, input_dtype: torch.dtype) -> int:
    """Shape, dtype, device and width checks shared by both scan entries (the contract of the
    reference's ``delta_scan.py:93-119``, with its error texts); returns the token count ``n``.

    Raises:
        ContractError: on a shape or dtype mismatch, a tensor off the GPU or on another device than
            ``q``, or a head dimension above ``MAX_HEAD_DIM``.
    """
    dims: Dims = {}
    check_shape("q", q, ("b", "n", "h", "dk"), dims, input_dtype)
    check_shape("k", k, ("b", "n", "h", "dk"), dims, input_dtype)
    check_shape("v", v, ("b", "n", "h", "dk"), dims, input_dtype)
    check_shape("beta", beta, ("b", "n", "h"), dims, input_dtype)
    check_shape("state", state, ("b", "h", "dk", "dk"), dims, STATE_DTYPE)
    if q.device.type != "cuda":
        raise ContractError(f"the fused scan runs on CUDA only, got q on {q.device}")
    for name, tensor in (("k", k), ("v", v), ("beta", beta), ("state", state)):
        if tensor.device != q.device:
            raise ContractError(f"{name} is on {tensor.device}, q on {q.device}")
    if dims["dk"] > MAX_HEAD_DIM:
        raise ContractError(f"head dimension {dims['dk']} exceeds the kernel's {MAX_HEAD_DIM}")
    return dims["n"]


def _refuse_grad(*tensors: Tensor) -> None:
    if torch.is_grad_enabled() and any(t.requires_grad for t in tensors):
        raise ContractError(
            "the HIP delta step is forward only (no backward kernel): call it under torch.no_grad() "
            "or on detached inputs"
        )


def _active_mask(active: Tensor | None, lead: tuple[str, ...], dims: Dims, device: torch.device) -> Tensor | None:
    if active is None:
        return None
    check_shape("active", active, lead, dims, torch.bool)
    if active.device != device:
        raise ContractError(f"active is on {active.device}, q on {device}")
    return active.contiguous().view(torch.uint8)


def _aligned(t: Tensor) -> Tensor:
    """Contiguous and 16-byte aligned (the kernels move rows in 16-byte pieces)."""
    t = t.contiguous()
    return t if t.data_ptr() % 16 == 0 else t.clone()


def _scan(entry: str, q: Tensor, k: Tensor, v: Tensor, beta: Tensor, state: Tensor, active: Tensor | None,
          fp32: bool, mask: Tensor | None = None, carried: tuple[Tensor, Tensor, Tensor] | None = None,
          records: Tensor | None = None) -> tuple[Tensor, Tensor]:
    b, n, h, dk = q.shape
    q, k, v, beta, state = (_aligned(t) for t in (q, k, v, beta, state))
    if mask is None:
        mask = _active_mask(active, ("b", "n"), {"b": b, "n": n}, q.device)
    o = torch.empty_like(q)
    s_out = torch.empty_like(state)
    lib = _lib.library()
    ws_bytes = int(lib.vsp_delta_scan_workspace_bytes(b, n, h, dk, int(fp32)))
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=q.device) if ws_bytes else None
    with torch.cuda.device(q.device):
        if records is not None:  # the bf16 forward that also keeps the chunks' starting states
            _lib.call("vsp_delta_scan_record_bf16", q.data_ptr(), k.data_ptr(), v.data_ptr(), beta.data_ptr(),
                      state.data_ptr(), o.data_ptr(), s_out.data_ptr(), _lib.ptr(ws), ws_bytes, _lib.ptr(mask),
                      records.data_ptr(), records.numel(), b, n, h, dk, _lib.stream_of(q.device))
        elif carried is None:
            _lib.call(entry, q.data_ptr(), k.data_ptr(), v.data_ptr(), beta.data_ptr(), state.data_ptr(), o.data_ptr(),
                      s_out.data_ptr(), _lib.ptr(ws), ws_bytes, _lib.ptr(mask), b, n, h, dk, _lib.stream_of(q.device))
        else:
            kc, vc, bc = (_aligned(t) for t in carried)
            _lib.call(entry.replace("vsp_delta_scan_", "vsp_delta_scan_carried_"), q.data_ptr(), k.data_ptr(),
                      v.data_ptr(), beta.data_ptr(), kc.data_ptr(), vc.data_ptr(), bc.data_ptr(), state.data_ptr(),
                      o.data_ptr(), s_out.data_ptr(), _lib.ptr(ws), ws_bytes, _lib.ptr(mask), b, n, h, dk,
                      _lib.stream_of(q.device))
    return o, s_out


def _checked_carried(carried: tuple[Tensor, Tensor, Tensor], k: Tensor, v: Tensor, beta: Tensor,
                     active: Tensor | None) -> tuple[Tensor, Tensor, Tensor]:
    if active is None:
        raise ContractError("carried inputs need the active mask that says which tokens read them")
    if len(carried) != 3:
        raise ContractError(f"carried holds k, v and beta, got {len(carried)} tensors")
    for name, held, fresh in zip(("k", "v", "beta"), carried, (k, v, beta)):
        if held.shape != fresh.shape or held.dtype != fresh.dtype or held.device != fresh.device:
            raise ContractError(f"carried {name}: {tuple(held.shape)} {held.dtype} on {held.device}, "
                                f"{name} is {tuple(fresh.shape)} {fresh.dtype} on {fresh.device}")
    return carried


class _DeltaScan(torch.autograd.Function):
    @staticmethod
    def forward(ctx: Any, q: Tensor, k: Tensor, v: Tensor, beta: Tensor, state: Tensor, mask: Tensor | None,
                fp32: bool) -> tuple[Tensor, Tensor]:  # noqa: D102
        entry = "vsp_delta_scan_f32" if fp32 else "vsp_delta_scan_bf16"
        tensors = [t.detach() for t in (q, k, v, beta, state)]
        grad = any(ctx.needs_input_grad[:5])
        # the bf16 forward at widths 32 and 64 keeps the chunks' starting states for the backward,
        # which then runs only the state gradient's chain
        b, n, h, dk = q.shape
        nrec = 0 if fp32 or not grad else int(_lib.library().vsp_delta_scan_records_bytes(b, n, h, dk))
        records = torch.empty(nrec, dtype=torch.uint8, device=q.device) if nrec else None
        o, s_out = _scan(entry, *tensors, None, fp32, mask=mask, records=records)
        if grad:
            ctx.save_for_backward(*(_aligned(t) for t in tensors), *(() if mask is None else (mask,)),
                                  *(() if records is None else (records,)))
            ctx.fp32 = fp32
            ctx.masked = mask is not None
            ctx.recorded = records is not None
        return o, s_out

    @staticmethod
    def backward(ctx: Any, d_o: Tensor | None, d_state: Tensor | None) -> tuple[Tensor | None, ...]:  # noqa: D102
        saved = ctx.saved_tensors
        q, k, v, beta, state = saved[:5]
        mask = saved[5] if ctx.masked else None
        records = saved[-1] if ctx.recorded else None
        b, n, h, dk = q.shape
        go = torch.zeros_like(q) if d_o is None else _aligned(d_o.to(q.dtype))
        gs = None if d_state is None else _aligned(d_state.to(STATE_DTYPE))
        dq, dk_, dv, db = (torch.empty_like(t) for t in (q, k, v, beta))
        d_state_in = torch.empty_like(state)
        lib = _lib.library()
        ws_bytes = int(lib.vsp_delta_scan_backward_workspace_bytes(b, n, h, dk))
        ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device=q.device)
        entry = "vsp_delta_scan_backward_f32" if ctx.fp32 else "vsp_delta_scan_backward_bf16"
        with torch.cuda.device(q.device):
            if records is not None:
                _lib.call("vsp_delta_scan_backward_recorded_bf16", q.data_ptr(), k.data_ptr(), v.data_ptr(),
                          beta.data_ptr(), state.data_ptr(), go.data_ptr(), _lib.ptr(gs), _lib.ptr(mask),
                          records.data_ptr(), records.numel(), dq.data_ptr(), dk_.data_ptr(), dv.data_ptr(),
                          db.data_ptr(), d_state_in.data_ptr(), ws.data_ptr(), ws_bytes, b, n, h, dk,
                          _lib.stream_of(q.device))
            else:
                _lib.call(entry, q.data_ptr(), k.data_ptr(), v.data_ptr(), beta.data_ptr(), state.data_ptr(),
                          go.data_ptr(), _lib.ptr(gs), _lib.ptr(mask), dq.data_ptr(), dk_.data_ptr(), dv.data_ptr(),
                          db.data_ptr(), d_state_in.data_ptr(), ws.data_ptr(), ws_bytes, b, n, h, dk,
                          _lib.stream_of(q.device))
        need = ctx.needs_input_grad
        return (dq if need[0] else None, dk_ if need[1] else None, dv if need[2] else None,
                db if need[3] else None, d_state_in if need[4] else None, None, None)


def _autograd_scan(q: Tensor, k: Tensor, v: Tensor, beta: Tensor, state: Tensor, active: Tensor | None,
                   fp32: bool, carried: tuple[Tensor, Tensor, Tensor] | None = None) -> tuple[Tensor, Tensor]:
    b, n, _, dk = q.shape
    mask = _active_mask(active, ("b", "n"), {"b": b, "n": n}, q.device)
    if carried is not None:
        carried = _checked_carried(carried, k, v, beta, active)
    grad = torch.is_grad_enabled() and any(t.requires_grad for t in (q, k, v, beta, state, *(carried or ())))
    if grad and carried is not None and active is not None:
        # under autograd the merge is explicit, so the gradient reaches the carried tensors
        keep = active.reshape(b, n, 1, 1)
        k, v = torch.where(keep, k, carried[0]), torch.where(keep, v, carried[1])
        beta = torch.where(keep[..., 0], beta, carried[2])
        carried = None
    if grad:
        width = backward_width(dk, fp32)
        if width == dk:
            out: tuple[Tensor, Tensor] = _DeltaScan.apply(q, k, v, beta, state, mask, fp32)
            return out
        # zero features of q and k and zero value columns add exact zeros to every product, so the
        # padded scan's outputs and gradients are the unpadded ones (the padding's are dropped)
        pad = width - dk
        qp, kp, vp = (torch.nn.functional.pad(t, (0, pad)) for t in (q, k, v))
        sp = torch.nn.functional.pad(state, (0, pad, 0, pad))
        o, s = _DeltaScan.apply(qp, kp, vp, beta, sp, mask, fp32)
        return o[..., :dk].contiguous(), s[..., :dk, :dk].contiguous()
    entry = "vsp_delta_scan_f32" if fp32 else "vsp_delta_scan_bf16"
    return _scan(entry, q, k, v, beta, state, None, fp32, mask=mask, carried=carried)


def delta_scan_fused(q: Tensor, k: Tensor, v: Tensor, beta: Tensor, state: Tensor, *,
                     active: Tensor | None = None,
                     carried: tuple[Tensor, Tensor, Tensor] | None = None) -> tuple[Tensor, Tensor]:
    """Run the delta rule over a block of ``n`` tokens on the bf16 HIP kernels (chunked WY/UT form,
    fp32 state), the drop-in for ``vesper/kernels/delta_scan.py:132-153``.

    Args:
        q: the queries ``[b, n, h, dk]`` in bfloat16, resident on the GPU.
        k: the keys, same shape and dtype; the caller normalizes them (norm at most one).
        v: the values, same shape and dtype.
        beta: per token and head ``[b, n, h]``, bfloat16, each in [0, 1].
        state: the fp32 state ``[b, h, dk, dk]`` the block starts from, read as ``H^T q``.
        active: optional bool ``[b, n]``: a token marked False still updates the state, but its
            output row is zero.
        carried: optional ``(k, v, beta)`` with the shapes of ``k, v, beta`` (requires ``active``):
            rows that an inactive token writes in place of its fresh ones, the same result as
            merging with ``where(active, fresh, carried)`` first.

    Returns:
        ``(o, state_n)``: the outputs ``[b, n, h, dk]`` in bfloat16 and the fp32 state after the
        block; for ``n == 0`` the (empty) ``q`` tensor itself and the same ``state`` object.

    Under autograd the gradients of ``q, k, v, beta`` (bfloat16) and ``state`` (float32) come from
    the backward kernels.

    Raises:
        ContractError: on a dtype, shape, device or width outside the contract, before any kernel
            runs.
    """
    if _checked_length(q, k, v, beta, state, INPUT_DTYPE) == 0:
        return q, state
    return _autograd_scan(q, k, v, beta, state, active, fp32=False, carried=carried)


def delta_scan_fused_fp32(q: Tensor, k: Tensor, v: Tensor, beta: Tensor, state: Tensor, *,
                          active: Tensor | None = None,
                          carried: tuple[Tensor, Tensor, Tensor] | None = None) -> tuple[Tensor, Tensor]:
    """Apply ``n`` tokens to the state with float32 inputs, state and arithmetic.

    As ``delta_scan_fused`` with every tensor float32; ``o`` is float32.
    """
    if _checked_length(q, k, v, beta, state, FP32_INPUT_DTYPE) == 0:
        return q, state
    return _autograd_scan(q, k, v, beta, state, active, fp32=True, carried=carried)


def delta_scan_step_fused(q: Tensor, k: Tensor, v: Tensor, beta: Tensor, state: Tensor, *,
                          active: Tensor | None = None, out_state: Tensor | None = None) -> tuple[Tensor, Tensor]:
    """One token per row written then read: ``(H'^T q, H')`` (``vesper/recurrence.py:143-163``).

    Args:
        q, k, v: ``[b, h, dk]`` float32 or bfloat16 (all three alike, ``beta [b, h]`` too).
        state: ``[b, h, dk, dk]`` float32.
        active: optional bool ``[b]``; an inactive row writes the state and reads zero.
        out_state: optional float32 tensor shaped like ``state`` that receives the new state; it
            may be ``state`` itself (an in-place decode step).

    Returns:
        ``(o [b, h, dk], state')`` with ``o`` in the inputs' dtype.
    """
    dtype = q.dtype
    if dtype not in (torch.float32, torch.bfloat16):
        raise ContractError(f"q: dtype must be torch.float32 or torch.bfloat16, got {dtype}")
    dims: Dims = {}
    check_shape("q", q, ("b", "h", "dk"), dims, dtype)
    check_shape("k", k, ("b", "h", "dk"), dims, dtype)
    check_shape("v", v, ("b", "h", "dk"), dims, dtype)
    check_shape("beta", beta, ("b", "h"), dims, dtype)
    check_shape("state", state, ("b", "h", "dk", "dk"), dims, STATE_DTYPE)
    if q.device.type != "cuda":
        raise ContractError(f"the fused scan runs on CUDA only, got q on {q.device}")
    for name, tensor in (("k", k), ("v", v), ("beta", beta), ("state", state)):
        if tensor.device != q.device:
            raise ContractError(f"{name} is on {tensor.device}, q on {q.device}")
    if dims["dk"] > MAX_HEAD_DIM:
        raise ContractError(f"head dimension {dims['dk']} exceeds the kernel's {MAX_HEAD_DIM}")
    _refuse_grad(q, k, v, beta, state)
    b, h, dk = q.shape
    q, k, v, beta = (t.contiguous() for t in (q, k, v, beta))
    if not state.is_contiguous():
        raise ContractError("state must be contiguous")
    if out_state is None:
        out_state = torch.empty_like(state)
    else:
        check_shape("out_state", out_state, ("b", "h", "dk", "dk"), dims, STATE_DTYPE)
        if out_state.device != q.device or not out_state.is_contiguous():
            raise ContractError("out_state must be a contiguous tensor on q's device")
    mask = _active_mask(active, ("b",), dims, q.device)
    o = torch.empty_like(q)
    entry = "vsp_delta_step_f32" if dtype == torch.float32 else "vsp_delta_step_bf16"
    with torch.cuda.device(q.device):
        _lib.call(entry, q.data_ptr(), k.data_ptr(), v.data_ptr(), beta.data_ptr(), state.data_ptr(),
                  out_state.data_ptr(), o.data_ptr(), _lib.ptr(mask), b, h, dk, _lib.stream_of(q.device))
    return o, out_state


def delta_scan_step_keys(q: Tensor, z: Tensor, v: Tensor, beta: Tensor, history: Tensor, taps: Tensor, state: Tensor,
                         *, active: Tensor | None = None, out_state: Tensor | None = None) -> Tensor:
    """A decode step's key filter and delta step in one launch (``vsp_delta_step_keys_bf16``): each
    head's key is the normalized filter of the key inputs ``z`` over the key ``history``
    (``vesper/column.py:255-289``), formed and rounded as ``key_step`` forms it, the next history
    is written over ``history``, and the step runs as ``delta_scan_step_fused`` with that key:
    bitwise the two launches' results.

    Args:
        q, v: ``[b, h, dk]`` bfloat16; ``beta [b, h]`` bfloat16.
        z: ``[b, h * dk]`` bfloat16 key inputs of the token.
        history: ``[b, K-1, h * dk]`` contiguous float32, updated in place.
        taps: ``[K, h * dk]`` float32 (``K`` in 1..8, tap 0 on the token).
        state: ``[b, h, dk, dk]`` float32; ``out_state`` may be ``state`` itself.
        active: optional bool ``[b]``; an inactive row writes the state and reads zero.

    Returns:
        ``o [b, h, dk]`` bfloat16 (the new state is in ``out_state``, by default ``state``).

    Raises:
        ContractError: on shapes, dtypes or devices outside that contract, or a head width other
            than 16, 32, 64 or 128.
    """
    dims: Dims = {}
    check_shape("q", q, ("b", "h", "dk"), dims, torch.bfloat16)
    check_shape("v", v, ("b", "h", "dk"), dims, torch.bfloat16)
    check_shape("beta", beta, ("b", "h"), dims, torch.bfloat16)
    check_shape("state", state, ("b", "h", "dk", "dk"), dims, STATE_DTYPE)
    b, h, dk = q.shape
    dims["hd"] = h * dk
    check_shape("z", z, ("b", "hd"), dims, torch.bfloat16)
    check_shape("taps", taps, ("K", "hd"), dims, torch.float32)
    width = dims["K"]
    dims["hist"] = width - 1
    check_shape("history", history, ("b", "hist", "hd"), dims, torch.float32)
    if dk not in (16, 32, 64, 128) or not 1 <= width <= 8:
        raise ContractError(f"head dimension {dk} (16, 32, 64, 128) or filter width {width} (1..8) not taken")
    for name, t in (("z", z), ("v", v), ("beta", beta), ("history", history), ("taps", taps), ("state", state)):
        if t.device != q.device or t.device.type != "cuda":
            raise ContractError(f"{name} is on {t.device}, q on {q.device} (CUDA only)")
    _refuse_grad(q, z, v, beta, history, taps, state)
    if out_state is None:
        out_state = state
    for name, t in (("history", history), ("state", state), ("out_state", out_state)):
        if not t.is_contiguous() or t.data_ptr() % 16:
            raise ContractError(f"{name} must be contiguous and 16-byte aligned")
    if out_state.shape != state.shape or out_state.dtype != STATE_DTYPE or out_state.device != q.device:
        raise ContractError("out_state must be shaped, typed and placed like state")
    q, v, beta = (t.contiguous() for t in (q, v, beta))
    zc, tc = z.contiguous(), taps.contiguous()
    for name, t in (("z", zc), ("taps", tc)):
        if t.data_ptr() % 16:
            raise ContractError(f"{name} must be 16-byte aligned")
    mask = _active_mask(active, ("b",), dims, q.device)
    o = torch.empty_like(q)
    with torch.cuda.device(q.device):
        _lib.call("vsp_delta_step_keys_bf16", q.data_ptr(), zc.data_ptr(), v.data_ptr(), beta.data_ptr(),
                  history.data_ptr() if width > 1 else None, tc.data_ptr(), width, state.data_ptr(),
                  out_state.data_ptr(), o.data_ptr(), _lib.ptr(mask), b, h, dk, _lib.stream_of(q.device))
    return o


# ---- the write strength (vesper/recurrence.py:34-88), alone and inside the scan's loads ----------

def _checked_modulator(logits: Tensor, m: Tensor | None, alpha: float | None) -> float:
    """The reference's refusals of a modulator (``recurrence.py:68-84``); returns alpha (0 without m)."""
    if m is None:
        return 0.0
    if alpha is None:
        raise ValueError("alpha must be given with a modulator (configs/*.yaml: learning.alpha)")
    if not 0.0 <= alpha < float("inf"):
        raise ValueError(f"alpha must be finite and non-negative, got {alpha}")
    dims: Dims = {}
    check_shape("logits", logits, ("b", "n", "h"), dims)
    check_shape("m", m, ("b", "n"), dims, torch.float32)
    if m.device != logits.device:
        raise ContractError(f"m is on {m.device}, logits on {logits.device}")
    factor = 1.0 + alpha * m
    if bool((factor < 0).any().item()):
        raise ValueError(f"1 + alpha m must not be negative; alpha {alpha}, smallest m {m.min().item()}")
    return float(alpha)


class _WriteStrength(torch.autograd.Function):
    @staticmethod
    def forward(ctx: Any, logits: Tensor, m: Tensor | None, alpha: float) -> Tensor:  # noqa: D102
        ctx.logits_dtype = logits.dtype
        lg = _aligned(logits.detach())
        mm = None if m is None else m.detach().contiguous()
        if mm is not None:
            # logits + ln(1 + alpha m) promotes to float32 in the reference (recurrence.py:84-88), so
            # beta and its gradient are float32 there: the fp32 kernel on the exactly widened logits
            lg = lg.float()
        beta = torch.empty_like(lg)
        rows = lg.numel() // lg.shape[-1] if lg.dim() else 1
        entry = "vsp_write_strength_f32" if lg.dtype == torch.float32 else "vsp_write_strength_bf16"
        with torch.cuda.device(lg.device):
            _lib.call(entry, lg.data_ptr(), _lib.ptr(mm), float(alpha), beta.data_ptr(), rows, lg.shape[-1],
                      _lib.stream_of(lg.device))
        ctx.save_for_backward(beta, *(() if mm is None else (mm,)))
        ctx.alpha = alpha
        return beta

    @staticmethod
    def backward(ctx: Any, g: Tensor) -> tuple[Tensor | None, ...]:  # noqa: D102
        beta, *rest = ctx.saved_tensors
        b32 = beta.float()
        slope = g.float() * b32 * (1.0 - b32)  # d sigmoid; zero where the factor is zero (beta = 0)
        d_logits = slope.to(ctx.logits_dtype)
        d_m = None
        if rest and ctx.needs_input_grad[1]:
            factor = 1.0 + ctx.alpha * rest[0]
            d_m = torch.where(factor > 0, (slope * ctx.alpha / factor.clamp_min(torch.finfo(torch.float32).tiny)[..., None]
                                           ).sum(dim=-1), torch.zeros_like(factor))
        return d_logits if ctx.needs_input_grad[0] else None, d_m, None


def write_strength(logits: Tensor, m: Tensor | None = None, alpha: float | None = None) -> Tensor:
    """``beta`` in [0, 1] from the write-strength logits, modulated when ``m`` is given
    (``vesper/recurrence.py:34-88``): ``sigmoid(logits)``, or ``sigmoid(logits + ln(1 + alpha m))``
    with an exact zero where ``1 + alpha m`` is zero. On the GPU (``vsp_write_strength_*``):
    without ``m`` in ``logits``' dtype (bfloat16 or float32), with the float32 ``m`` in float32, as
    the reference's sum with the float32 shift promotes it; under autograd the gradients of
    ``logits`` (in its dtype) and ``m``.

    Args:
        logits: ``[b, n, h]`` (any shape without ``m``), bfloat16 or float32, on the GPU.
        m: optional float32 ``[b, n]`` modulator, broadcast over heads.
        alpha: the modulation strength, required with ``m``, finite and non-negative.

    Raises:
        ContractError: on a dtype, shape or device outside that; ValueError: as the reference
            (``m`` without ``alpha``, a negative or non-finite ``alpha``, ``1 + alpha m < 0``).
    """
    if logits.dtype not in (torch.float32, torch.bfloat16):
        raise ContractError(f"logits: dtype must be torch.float32 or torch.bfloat16, got {logits.dtype}")
    if logits.device.type != "cuda":
        raise ContractError(f"the write strength kernel runs on CUDA only, got logits on {logits.device}")
    a = _checked_modulator(logits, m, alpha)
    if logits.numel() == 0:
        return torch.empty_like(logits)
    return _WriteStrength.apply(logits, m, a)


def delta_scan_fused_logits(q: Tensor, k: Tensor, v: Tensor, logits: Tensor, state: Tensor, *,
                            m: Tensor | None = None, alpha: float | None = None,
                            active: Tensor | None = None) -> tuple[Tensor, Tensor]:
    """``delta_scan_fused(q, k, v, write_strength(logits, m, alpha), state)`` with the write strength
    computed inside the scan's beta loads (``vsp_delta_scan_logits_*``): ``beta`` is never
    written to memory. bfloat16 inputs run the bf16 scan, float32 inputs the fp32 scan; ``beta``
    is computed in float32 and rounded to the inputs' dtype, as the reference column casts it
    before its scan (``column.py:313``), so with and without autograd the scan sees the same beta.

    Under autograd it is the composition above (the write strength's gradient and the scan's
    backward kernels).

    Raises:
        ContractError / ValueError: as ``delta_scan_fused`` and ``write_strength``.
    """
    fp32 = q.dtype == torch.float32
    if _checked_length(q, k, v, logits, state, FP32_INPUT_DTYPE if fp32 else INPUT_DTYPE) == 0:
        return q, state
    a = _checked_modulator(logits, m, alpha)
    if torch.is_grad_enabled() and any(t.requires_grad for t in (q, k, v, logits, state, *(() if m is None else (m,)))):
        beta = write_strength(logits, m, alpha).to(q.dtype)
        return (delta_scan_fused_fp32 if fp32 else delta_scan_fused)(q, k, v, beta, state, active=active)
    b, n, h, dk = q.shape
    q, k, v, logits, state = (_aligned(t) for t in (q, k, v, logits, state))
    mm = None if m is None else m.contiguous()
    mask = _active_mask(active, ("b", "n"), {"b": b, "n": n}, q.device)
    o = torch.empty_like(q)
    s_out = torch.empty_like(state)
    lib = _lib.library()
    ws_bytes = int(lib.vsp_delta_scan_workspace_bytes(b, n, h, dk, int(fp32)))
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=q.device) if ws_bytes else None
    entry = "vsp_delta_scan_logits_f32" if fp32 else "vsp_delta_scan_logits_bf16"
    with torch.cuda.device(q.device):
        _lib.call(entry, q.data_ptr(), k.data_ptr(), v.data_ptr(), logits.data_ptr(), _lib.ptr(mm), a,
                  state.data_ptr(), o.data_ptr(), s_out.data_ptr(), _lib.ptr(ws), ws_bytes, _lib.ptr(mask),
                  b, n, h, dk, _lib.stream_of(q.device))
    return o, s_out
