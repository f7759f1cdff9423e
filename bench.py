#!/usr/bin/env python3
"""Benchmark of Vesper's column sequence mixers on one MI355X.

A step is one prefill pass of both mixers over one batch of synthetic input: the delta-rule scan
(B=8, T=4096, H=8, d=64; bf16 q/k/v/beta, fp32 state with S0 ~ N(0, 0.02^2), chunk 64) followed by
sliding-window causal attention over the same batch shape (window 512, bf16). ``value`` is prefill
tokens/s = B*T / (time of one step), inputs resident in HBM, the timed steps run as one captured HIP
graph (the eager loop's time, with the host's gaps between launches, is reported beside it). Beside it the line carries each
kernel's own rate at its own configuration (attention alone at B=4), the key filter that feeds the
scan (B8 T4096 d512 = 8 heads of 64, 4 taps, bf16), the decode rate (256
single-token steps of batch 64: fp32 delta update of S [64,8,64,64] then attention over a 512-entry
bf16 KV ring, captured as one HIP graph), the looped column with per-token halting (B4 T2048 d512,
8 passes, 4-tap key filter), the column's captured single-token decoder (batch 64, 8 passes), the
roofline of the dominant kernel measured with HIP events on the launch stream inside the timed
region, per-launch medians warm and cold (input sets rotated past the 256 MB MALL) for the scan
(bf16 and fp32), attention and decode, forward plus backward at the shapes the reference quotes its
kernels on, and the CPU oracle timed on bounded samples of the same workloads on all of this host's
cores.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
"""

from __future__ import annotations

import argparse
import json
import math
import os
import platform
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "vesper-preview_amd"))

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0

B, T, H, D, WINDOW = 8, 4096, 8, 64, 512
ATTN_B = 4
DEC_B, DEC_W, DEC_STEPS = 64, 512, 256
LOOP_B, LOOP_T, LOOP_D, LOOP_PASSES = 4, 2048, 512, 8
KEY_D, KEY_TAPS = H * D, 4  # the key filter over the prefill batch: d = 8 heads of 64, 4 taps
COPY_BYTES = 256 << 20  # the calibration copy of --traffic-probe


def log(*a: object) -> None:
    print(*a, file=sys.stderr, flush=True)


# ---- algorithmic work (per launch) ---------------------------------------------------------------
def scan_flops(b: int, t: int, h: int, d: int, chunk: int = 64) -> float:
    units = b * h * math.ceil(t / chunk)
    return units * (8 * 2 * chunk * d * d + chunk**3 / 3)


def scan_bytes(b: int, t: int, h: int, d: int) -> float:
    return 4 * b * t * h * d * 2 + b * t * h * 2 + 2 * b * h * d * d * 4  # q,k,v,o bf16; beta; S0, S_n


def window_pairs(t: int, w: int) -> int:
    return sum(min(i + 1, w) for i in range(t))


def attn_flops(b: int, t: int, h: int, d: int, w: int) -> float:
    return 4.0 * d * b * h * window_pairs(t, w)


def attn_bytes(b: int, t: int, h: int, hkv: int, d: int) -> float:
    return 2 * b * t * h * d * 2 + 2 * b * t * hkv * d * 2  # q, o; k, v


def key_filter_bytes(b: int, t: int, d: int, taps: int, elem: int = 2) -> float:
    """Key inputs read once, keys written once, plus the history rows and the taps (float32)."""
    return 2.0 * b * t * d * elem + 4.0 * d * (b * (taps - 1) + taps)


def key_filter_backward_bytes(b: int, t: int, d: int, taps: int, elem: int = 2) -> float:
    """Key inputs and the keys' gradient read once, the inputs' gradient written once; taps, history
    and their gradients (float32)."""
    return 3.0 * b * t * d * elem + 4.0 * d * 2 * (b * (taps - 1) + taps)


def decode_step_bytes(b: int, h: int, d: int, w: int) -> float:
    state = 2 * b * h * d * d * 4  # read + write
    delta_io = 4 * b * h * d * 4 + b * h * 4  # q, k, v, o fp32; beta
    ring = 2 * b * w * h * d * 2  # K and V rows read
    attn_io = 4 * b * h * d * 2 + b * 8  # q, k, v, o bf16; positions
    ring_write = 2 * b * h * d * 2 + b * 9
    return state + delta_io + ring + attn_io + ring_write


# ---- inputs -------------------------------------------------------------------------------------
def scan_inputs(torch, dev, b=B, t=T, h=H, d=D, seed=0):
    from vesper.kernels.delta_scan import INPUT_DTYPE

    g = torch.Generator().manual_seed(seed)
    q = torch.randn(b, t, h, d, generator=g)
    k = torch.randn(b, t, h, d, generator=g)
    q = q / q.norm(dim=-1, keepdim=True).clamp_min(1e-6)
    k = k / k.norm(dim=-1, keepdim=True).clamp_min(1e-6)
    v = torch.randn(b, t, h, d, generator=g)
    beta = torch.sigmoid(torch.randn(b, t, h, generator=g))
    s0 = 0.02 * torch.randn(b, h, d, d, generator=g)
    return [x.to(dev, INPUT_DTYPE) for x in (q, k, v, beta)] + [s0.to(dev)]


def attn_inputs(torch, dev, b=B, t=T, h=H, d=D, seed=1):
    g = torch.Generator().manual_seed(seed)
    return [torch.randn(b, t, h, d, generator=g).to(dev, torch.bfloat16) for _ in range(3)]


# ---- GPU legs -------------------------------------------------------------------------------------
def captured_ms(torch, fn, count: int, replays: int = 1) -> float:
    """Milliseconds per call of ``fn`` with ``count`` calls captured in one HIP graph: the graph is
    replayed once untimed, then ``replays`` times back to back between two events on the stream
    (median per-call time when ``replays`` > 1 is taken over single replays)."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(count):
            fn()
    graph.replay()
    torch.cuda.synchronize()
    times = []
    for _ in range(replays):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        graph.replay()
        e1.record()
        torch.cuda.synchronize()
        times.append(e0.elapsed_time(e1) / count)
    return statistics.median(times)


def time_prefill(torch, steps: int, warmup: int) -> dict:
    """The prefill step (the scan, then window attention, over the bench batch). The timed steps
    run as one HIP graph of ``steps`` steps (each step's kernels launched back to back by the
    device, as a captured training or serving loop runs them), between a synchronize and events on
    the stream; the scan and the attention alone are timed the same way (graphs of 10 launches,
    median of 5 replays). The eager loop (one Python call per mixer, events around each) is timed
    too: its gaps between launches are the host's."""
    from vesper.kernels.delta_scan import delta_scan_fused
    from vesper.kernels.window_attn import window_attention

    dev = torch.device("cuda:0")
    q, k, v, beta, s0 = scan_inputs(torch, dev)
    aq, ak, av = attn_inputs(torch, dev)

    def scan():
        delta_scan_fused(q, k, v, beta, s0)

    def attn():
        window_attention(aq, ak, av, WINDOW)

    def step():
        scan()
        attn()

    with torch.no_grad():
        for _ in range(warmup):
            step()
        torch.cuda.synchronize()
        # eager: events around each call
        ev = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(steps)]
        for i in range(steps):
            ev[i][0].record()
            scan()
            ev[i][1].record()
            attn()
            ev[i][2].record()
        torch.cuda.synchronize()
        # captured: exactly `steps` steps in one graph, timed over one replay
        t0 = time.perf_counter()
        step_ms = captured_ms(torch, step, steps)
        wall = time.perf_counter() - t0
        scan_ms = captured_ms(torch, scan, 10, 5)
        attn_ms = captured_ms(torch, attn, 10, 5)
    e_scan = [e[0].elapsed_time(e[1]) for e in ev]
    e_attn = [e[1].elapsed_time(e[2]) for e in ev]
    e_step = [e[0].elapsed_time(e[2]) for e in ev]
    return {"wall_s": wall, "step_ms": step_ms, "scan_ms": scan_ms, "attn_ms": attn_ms,
            "eager_step_ms": statistics.median(e_step), "eager_scan_ms": statistics.median(e_scan),
            "eager_attn_ms": statistics.median(e_attn)}


def time_attention_config(torch) -> float:
    """Milliseconds per launch of window attention at B4 T4096 H8 D64 w512 (bf16), in a HIP graph
    of 10 launches (median of 5 replays)."""
    from vesper.kernels.window_attn import window_attention

    dev = torch.device("cuda:0")
    aq, ak, av = attn_inputs(torch, dev, b=ATTN_B, seed=2)
    with torch.no_grad():
        for _ in range(3):
            window_attention(aq, ak, av, WINDOW)
        return captured_ms(torch, lambda: window_attention(aq, ak, av, WINDOW), 10, 5)


def time_key_filter(torch, reps: int = 50) -> tuple[float, float]:
    """Milliseconds per launch of the key filter, forward and backward, at B8 T4096 d512 (8 heads of
    64), 4 taps, bf16.

    The launches are captured in one HIP graph each and timed on replay: one launch (13 us) is about
    as long as the host's per-call checks, so a timed loop of eager calls would measure the host.
    The backward is the library's entry point (d z, d taps, d history) with its workspace.
    """
    from vesper.kernels import _lib
    from vesper.kernels.keys import fused_keys

    dev = torch.device("cuda:0")
    g = torch.Generator().manual_seed(4)
    z = torch.randn(B, T, KEY_D, generator=g).to(dev, torch.bfloat16)
    history = torch.randn(B, KEY_TAPS - 1, KEY_D, generator=g).to(dev)
    taps = torch.randn(KEY_TAPS, KEY_D, generator=g).to(dev)
    up = torch.randn(B, T, KEY_D, generator=g).to(dev, torch.bfloat16)
    grad_z = torch.empty_like(z)
    grad_taps = torch.empty(KEY_TAPS, KEY_D, device=dev)
    grad_history = torch.empty_like(history)
    nbytes = int(_lib.library().vsp_key_filter_backward_workspace_bytes(B, T, KEY_D, KEY_TAPS))
    workspace = torch.empty(nbytes, dtype=torch.uint8, device=dev)

    def forward():
        fused_keys(z, history, taps, H)

    def backward():
        _lib.call("vsp_key_filter_backward_bf16", _lib.ptr(z), _lib.ptr(history), _lib.ptr(taps), _lib.ptr(up),
                  _lib.ptr(grad_z), _lib.ptr(grad_taps), _lib.ptr(grad_history), _lib.ptr(workspace), nbytes,
                  B, T, KEY_D, H, KEY_TAPS, _lib.stream_of(dev))

    out = []
    with torch.no_grad():
        for fn in (forward, backward):
            side = torch.cuda.Stream()
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side):
                for _ in range(3):
                    fn()
            torch.cuda.current_stream().wait_stream(side)
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                for _ in range(reps):
                    fn()
            graph.replay()  # warm
            times = []
            for _ in range(5):
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                torch.cuda.synchronize()
                e0.record()
                graph.replay()
                e1.record()
                torch.cuda.synchronize()
                times.append(e0.elapsed_time(e1) / reps)
            out.append(statistics.median(times))
    return out[0], out[1]


def time_scan_backward(torch, reps: int = 10) -> dict:
    """The delta scan's backward at B8 T4096 H8 d64 bf16 through the C ABI, 10 launches in one HIP
    graph (median milliseconds of 3 replays): as autograd runs it (``recorded_ms``: the forward
    recorded each chunk's starting state, so only the state gradient's chain runs; the forward
    with the records is timed the same way, ``forward_recording_ms``), and the backward that
    recomputes the states itself (``alone_ms``)."""
    from vesper.kernels import _lib

    dev = torch.device("cuda:0")
    q, k, v, beta, s0 = scan_inputs(torch, dev)
    up = torch.randn(q.shape, generator=torch.Generator().manual_seed(8)).to(dev, torch.bfloat16)
    ds = torch.randn(s0.shape, generator=torch.Generator().manual_seed(9)).to(dev)
    dq, dk, dv, db = (torch.empty_like(t) for t in (q, k, v, beta))
    d0 = torch.empty_like(s0)
    lib = _lib.library()
    nbytes = int(lib.vsp_delta_scan_backward_workspace_bytes(B, T, H, D))
    ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    fbytes = int(lib.vsp_delta_scan_workspace_bytes(B, T, H, D, 0))
    fws = torch.empty(fbytes, dtype=torch.uint8, device=dev)
    rbytes = int(lib.vsp_delta_scan_records_bytes(B, T, H, D))
    rec = torch.empty(rbytes, dtype=torch.uint8, device=dev)
    o, s1 = torch.empty_like(q), torch.empty_like(s0)
    p = _lib.ptr
    # (the stream is looked up at each call: under capture it is the capturing one)
    grads = lambda: [p(dq), p(dk), p(dv), p(db), p(d0), p(ws), nbytes, B, T, H, D, _lib.stream_of(dev)]  # noqa: E731

    def forward():
        _lib.call("vsp_delta_scan_record_bf16", p(q), p(k), p(v), p(beta), p(s0), p(o), p(s1), p(fws), fbytes, None,
                  p(rec), rbytes, B, T, H, D, _lib.stream_of(dev))

    def recorded():
        _lib.call("vsp_delta_scan_backward_recorded_bf16", p(q), p(k), p(v), p(beta), p(s0), p(up), p(ds), None,
                  p(rec), rbytes, *grads())

    def alone():
        _lib.call("vsp_delta_scan_backward_bf16", p(q), p(k), p(v), p(beta), p(s0), p(up), p(ds), None, *grads())

    def timed(run):
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            run()
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for _ in range(reps):
                run()
        graph.replay()
        times = []
        for _ in range(3):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            torch.cuda.synchronize()
            e0.record()
            graph.replay()
            e1.record()
            torch.cuda.synchronize()
            times.append(e0.elapsed_time(e1) / reps)
        return statistics.median(times)

    out = {"forward_recording_ms": timed(forward)}  # (also leaves the records the backward reads)
    out["recorded_ms"] = timed(recorded)
    out["alone_ms"] = timed(alone)
    return out


def time_attention_backward(torch, reps: int = 20) -> float:
    """Milliseconds per backward of window attention at B4 T4096 H8 D64 w512 bf16 (the dq and the
    dk/dv kernels, from a forward's o and log-sum-exp), 20 launches in one HIP graph."""
    from vesper.kernels import _lib

    dev = torch.device("cuda:0")
    aq, ak, av = attn_inputs(torch, dev, b=ATTN_B, seed=5)
    b, n, h, dk = aq.shape
    o = torch.empty_like(aq)
    lse = torch.empty(b, h, n, device=dev)
    up = torch.randn(aq.shape, generator=torch.Generator().manual_seed(6)).to(dev, torch.bfloat16)
    dq, dkk, dv = torch.empty_like(aq), torch.empty_like(ak), torch.empty_like(av)
    ws = torch.empty(b * h * n, device=dev)
    scale = 1.0 / math.sqrt(dk)
    _lib.call("vsp_window_attn_lse_bf16", _lib.ptr(aq), _lib.ptr(ak), _lib.ptr(av), _lib.ptr(o), _lib.ptr(lse), None,
              b, n, 0, h, h, dk, WINDOW, scale, _lib.stream_of(dev))

    def run():
        _lib.call("vsp_window_attn_backward_bf16", _lib.ptr(aq), _lib.ptr(ak), _lib.ptr(av), _lib.ptr(o), _lib.ptr(up),
                  _lib.ptr(lse), _lib.ptr(ws), _lib.ptr(dq), _lib.ptr(dkk), _lib.ptr(dv), b, n, 0, h, h, dk, WINDOW,
                  scale, _lib.stream_of(dev))

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            run()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(reps):
            run()
    graph.replay()
    times = []
    for _ in range(3):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record()
        graph.replay()
        e1.record()
        torch.cuda.synchronize()
        times.append(e0.elapsed_time(e1) / reps)
    return statistics.median(times)


def time_decode(torch, reps: int = 5) -> dict:
    from vesper.kernels.delta_scan import delta_scan_step_fused
    from vesper.kernels.ring_attn import RingKVCache, ring_attention

    dev = torch.device("cuda:0")
    g = torch.Generator().manual_seed(3)
    b, h, d, w, n = DEC_B, H, D, DEC_W, DEC_STEPS
    state = (0.02 * torch.randn(b, h, d, d, generator=g)).to(dev)
    ring = RingKVCache(torch.randn(b, w, h, d, generator=g).to(dev, torch.bfloat16),
                       torch.randn(b, w, h, d, generator=g).to(dev, torch.bfloat16),
                       torch.arange(w).expand(b, w).contiguous().to(dev),
                       torch.ones(b, w, dtype=torch.bool, device=dev), w)
    pos0, valid0 = ring.pos.clone(), ring.valid.clone()
    dq = torch.randn(n, b, h, d, generator=g)
    dk = torch.randn(n, b, h, d, generator=g)
    dq = (dq / dq.norm(dim=-1, keepdim=True)).to(dev)
    dk = (dk / dk.norm(dim=-1, keepdim=True)).to(dev)
    dv = torch.randn(n, b, h, d, generator=g).to(dev)
    dbeta = torch.sigmoid(torch.randn(n, b, h, generator=g)).to(dev)
    aq = torch.randn(n, b, 1, h, d, generator=g).to(dev, torch.bfloat16)
    ak = torch.randn(n, b, 1, h, d, generator=g).to(dev, torch.bfloat16)
    av = torch.randn(n, b, 1, h, d, generator=g).to(dev, torch.bfloat16)
    pos = (w + torch.arange(n)).view(n, 1, 1).expand(n, b, 1).contiguous().to(dev)
    counters = torch.zeros(b, dtype=torch.int32, device=dev)  # the ring write's arrival counters

    def run_all():
        for s in range(n):
            delta_scan_step_fused(dq[s], dk[s], dv[s], dbeta[s], state, out_state=state)
            ring_attention(aq[s], ak[s], av[s], pos[s], ring, inplace=True, check_positions=False,
                           workspace=counters)

    with torch.no_grad():
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            run_all()
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            run_all()
        times = []
        for _ in range(reps):
            ring.pos.copy_(pos0)
            ring.valid.copy_(valid0)
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            torch.cuda.synchronize()
            e0.record()
            graph.replay()
            e1.record()
            torch.cuda.synchronize()
            times.append(e0.elapsed_time(e1))
    ms = statistics.median(times)
    return {"ms_256_steps": ms, "tok_s": b * n / (ms / 1e3), "us_per_step": 1e3 * ms / n}


def time_looped(torch, reps: int = 3) -> dict:
    """The looped column with halting: B4 T2048 d512 H8 d64, 8 passes, window 512, 4-tap key filter,
    p_halt 0.3; the copy-forward fused into the kernels' loads (the default) and, for comparison,
    as where merges."""
    from vesper.loop import LoopedColumn

    dev = torch.device("cuda:0")
    b, n, d, h, dk, passes = LOOP_B, LOOP_T, LOOP_D, H, D, LOOP_PASSES
    g = torch.Generator().manual_seed(12)
    x0 = torch.randn(b, n, d, generator=g).to(dev)
    exits = [(torch.rand(b, n, generator=g) < 0.3).to(dev) for _ in range(passes)]
    states = [torch.zeros(b, h, dk, dk, device=dev) for _ in range(passes)]
    histories = [torch.zeros(b, KEY_TAPS - 1, d, device=dev) for _ in range(passes)]
    result = {}
    for mode in ("fused", "where"):
        column = LoopedColumn.random(d, h, h, dk, WINDOW, passes, seed=11, device=dev, key_conv=KEY_TAPS,
                                     copy_forward=mode)
        for _ in range(2):  # warm-up (the first call also sets up the GEMM kernels)
            column.forward(x0, states, exits, histories)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record()
        for _ in range(reps):
            out = column.forward(x0, states, exits, histories)
        e1.record()
        torch.cuda.synchronize()
        result[mode] = e0.elapsed_time(e1) / reps
    # the fused forward captured in one HIP graph (as a training or serving loop would run it):
    # the device time without the host's per-launch cost; the replay must equal the eager result
    column = LoopedColumn.random(d, h, h, dk, WINDOW, passes, seed=11, device=dev, key_conv=KEY_TAPS)
    eager = column.forward(x0, states, exits, histories).y.clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        column.forward(x0, states, exits, histories)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        captured = column.forward(x0, states, exits, histories)
    times = []
    for _ in range(reps):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record()
        graph.replay()
        e1.record()
        torch.cuda.synchronize()
        times.append(e0.elapsed_time(e1))
        if not torch.equal(captured.y, eager):
            raise RuntimeError("a replay of the captured looped column differs from the eager forward")
    ms = result["fused"]
    return {"ms": ms, "ms_where": result["where"], "ms_captured": statistics.median(times),
            "tok_s": b * n / (ms / 1e3), "mean_passes": float(out.n_iters.float().mean())}


def time_column_decode(torch, steps: int = 64) -> dict:
    """The column's captured single-token decoder: batch 64, d512 (8 heads of 64, 8 KV heads),
    window 512, 4-tap key filter, all 8 passes dense; rings full (positions 0..511 written), the
    timed tokens at positions 512 onwards; one step = one HIP graph replay."""
    from vesper.decode import PER_PASS, CapturedDecoder
    from vesper.loop import LoopedColumn

    dev = torch.device("cuda:0")
    b, d, h, dk, passes = DEC_B, LOOP_D, H, D, LOOP_PASSES
    column = LoopedColumn.random(d, h, h, dk, DEC_W, passes, seed=21, device=dev, key_conv=KEY_TAPS)
    decoder = CapturedDecoder(column, passes)
    flat = decoder.start(b)
    g = torch.Generator().manual_seed(22)
    for t in range(passes):
        flat[PER_PASS * t + 2].copy_(torch.randn(b, DEC_W, h, dk, generator=g).to(torch.bfloat16))
        flat[PER_PASS * t + 3].copy_(torch.randn(b, DEC_W, h, dk, generator=g).to(torch.bfloat16))
        flat[PER_PASS * t + 4].copy_(torch.arange(DEC_W).expand(b, DEC_W))
        flat[PER_PASS * t + 5].fill_(True)
    xs = torch.randn(steps + 8, b, 1, d, generator=g).to(dev)
    pos = (DEC_W + torch.arange(steps + 8)).view(-1, 1, 1).expand(-1, b, 1).contiguous().to(dev)
    with torch.no_grad():
        for i in range(8):  # warm-up, then the capture, then replays
            _, flat = decoder.step(xs[i], pos[i], flat)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record()
        for i in range(8, steps + 8):
            _, flat = decoder.step(xs[i], pos[i], flat)
        e1.record()
        torch.cuda.synchronize()
    us = e0.elapsed_time(e1) / steps * 1e3
    return {"us_per_step": us, "tok_s": b / (us / 1e6), "captures": decoder.captures, "replays": decoder.replays}


# ---- per-launch medians, warm and cold ---------------------------------------------------------------
def _medians(torch, calls, reps: int) -> list[float]:
    """GPU milliseconds of each of ``reps`` calls (``calls(i)`` runs call i), median-ready: the
    device is first held busy by a spin kernel long enough for the host to enqueue every call with
    its events, so no event pair times the host."""
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(reps)]
    torch.cuda.synchronize()
    torch.cuda._sleep(50_000_000)  # tens of ms of device time ahead of the host
    for i in range(reps):
        ev[i][0].record()
        calls(i)
        ev[i][1].record()
    torch.cuda.synchronize()
    return [a.elapsed_time(b) for a, b in ev]


def time_cold_warm(torch, reps: int = 52) -> dict:
    """Median milliseconds per launch over ``reps`` launches after 10 warm-ups, warm (one resident
    input set) and cold (input sets rotated so that more than 512 MB lie between two uses of a
    set, beyond the 256 MB MALL): the bf16 scan at B8 T4096 H8 d64, window attention at B8 and B4
    T4096 H8 D64 w512, and the float32 scan at B2 T512 H4 d64 and B8 T4096 H8 d64."""
    from vesper.kernels.delta_scan import delta_scan_fused, delta_scan_fused_fp32
    from vesper.kernels.window_attn import window_attention

    dev = torch.device("cuda:0")
    out: dict = {}
    with torch.no_grad():
        sets = [scan_inputs(torch, dev, seed=10 + i) for i in range(4)]  # 4 x 137 MB
        fn = lambda i, s=sets: delta_scan_fused(*s[i % len(s)])  # noqa: E731
        for i in range(10):
            fn(i)
        out["delta_scan_bf16_b8_warm_ms"] = statistics.median(_medians(torch, lambda i: fn(0), reps))
        out["delta_scan_bf16_b8_cold_ms"] = statistics.median(_medians(torch, fn, reps))
        del sets
        for b, name in ((B, "b8"), (ATTN_B, "b4")):
            asets = [attn_inputs(torch, dev, b=b, seed=20 + i) for i in range(8 if b == ATTN_B else 5)]
            afn = lambda i, s=asets: window_attention(*s[i % len(s)], WINDOW)  # noqa: E731
            for i in range(10):
                afn(i)
            out[f"window_attn_{name}_warm_ms"] = statistics.median(_medians(torch, lambda i: afn(0), reps))
            out[f"window_attn_{name}_cold_ms"] = statistics.median(_medians(torch, afn, reps))
            del asets
        for (b, t, h), name in (((2, 512, 4), "c1_b2_t512_h4"), ((B, T, H), "b8_t4096_h8")):
            s32 = [x.float() for x in scan_inputs(torch, dev, b=b, t=t, h=h, seed=30)]
            for _ in range(10):
                delta_scan_fused_fp32(*s32)
            out[f"delta_scan_fp32_{name}_warm_ms"] = statistics.median(
                _medians(torch, lambda i: delta_scan_fused_fp32(*s32), reps))
            del s32
    return out


def time_decode_cold(torch, sets: int = 8) -> float:
    """Microseconds per decode step (delta step + ring attention, batch 64) with ``sets``
    independent states and rings (72 MiB each, 576 MB in all) used in turn, so consecutive uses of
    one set are 504 MB apart: the 256 MB MALL cannot serve them. 256 steps in one HIP graph."""
    from vesper.kernels.delta_scan import delta_scan_step_fused
    from vesper.kernels.ring_attn import RingKVCache, ring_attention

    dev = torch.device("cuda:0")
    g = torch.Generator().manual_seed(31)
    b, h, d, w, n = DEC_B, H, D, DEC_W, DEC_STEPS
    states = [(0.02 * torch.randn(b, h, d, d, generator=g)).to(dev) for _ in range(sets)]
    rings = [RingKVCache(torch.randn(b, w, h, d, generator=g).to(dev, torch.bfloat16),
                         torch.randn(b, w, h, d, generator=g).to(dev, torch.bfloat16),
                         torch.arange(w).expand(b, w).contiguous().to(dev),
                         torch.ones(b, w, dtype=torch.bool, device=dev), w) for _ in range(sets)]
    counters = [torch.zeros(b, dtype=torch.int32, device=dev) for _ in range(sets)]
    dq = torch.randn(n, b, h, d, generator=g)
    dq = (dq / dq.norm(dim=-1, keepdim=True)).to(dev)
    dbeta = torch.sigmoid(torch.randn(n, b, h, generator=g)).to(dev)
    aq = torch.randn(n, b, 1, h, d, generator=g).to(dev, torch.bfloat16)
    pos = (w + torch.arange(n) // sets).view(n, 1, 1).expand(n, b, 1).contiguous().to(dev)

    def run_all():
        for s in range(n):
            j = s % sets
            delta_scan_step_fused(dq[s], dq[s], dq[s], dbeta[s], states[j], out_state=states[j])
            ring_attention(aq[s], aq[s], aq[s], pos[s], rings[j], inplace=True, check_positions=False,
                           workspace=counters[j])

    with torch.no_grad():
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            run_all()
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            run_all()
        times = []
        for _ in range(5):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            torch.cuda.synchronize()
            e0.record()
            graph.replay()
            e1.record()
            torch.cuda.synchronize()
            times.append(e0.elapsed_time(e1))
    return 1e3 * statistics.median(times) / n


def time_published_shapes(torch, reps: int = 20) -> dict:
    """Forward plus backward at the shapes the reference quotes its kernels on (context only, taken
    on other GPUs): window attention at b16, chunk 1024 after a 512-row cache, 8 heads over 2 KV
    heads, dk 64, window 512 (vesper/kernels/window_attn.py:10-13: 1.46 ms on an RTX 5090); the
    scan at b32 n88 h2 dk16 in bf16 and in fp32 (vesper/kernels/delta_scan.py:22-24: about 2 and
    1 ms on an RTX 5060 Ti). Eager autograd calls, median milliseconds of ``reps``."""
    from vesper.kernels.delta_scan import delta_scan_fused, delta_scan_fused_fp32
    from vesper.kernels.window_attn import window_attention

    dev = torch.device("cuda:0")
    g = torch.Generator().manual_seed(41)
    out = {}
    b, n, m, h, hkv, dk = 16, 1024, 512, 8, 2, 64
    q = torch.randn(b, n, h, dk, generator=g).to(dev, torch.bfloat16).requires_grad_()
    keys = torch.randn(b, m + n, hkv, dk, generator=g).to(dev, torch.bfloat16).requires_grad_()
    vals = torch.randn(b, m + n, hkv, dk, generator=g).to(dev, torch.bfloat16).requires_grad_()
    up = torch.randn(b, n, h, dk, generator=g).to(dev, torch.bfloat16)

    def attn():
        window_attention(q, keys, vals, m).backward(up)

    def timed(fn) -> float:
        for _ in range(3):
            fn()
        times = []
        for _ in range(reps):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            fn()
            torch.cuda.synchronize()
            times.append(1e3 * (time.perf_counter() - t0))
        return statistics.median(times)

    out["window_attn_fwd_bwd_b16_n1024_m512_h8_hkv2_dk64_ms"] = round(timed(attn), 4)
    for fp32, name in ((False, "bf16"), (True, "fp32")):
        dtype = torch.float32 if fp32 else torch.bfloat16
        sb, sn, sh, sd = 32, 88, 2, 16
        qs = torch.randn(sb, sn, sh, sd, generator=g)
        ks = torch.randn(sb, sn, sh, sd, generator=g)
        ks = ks / ks.norm(dim=-1, keepdim=True)
        ins = [t.to(dev, dtype).requires_grad_() for t in (qs, ks, torch.randn(sb, sn, sh, sd, generator=g),
                                                             torch.sigmoid(torch.randn(sb, sn, sh, generator=g)))]
        s0 = torch.zeros(sb, sh, sd, sd, device=dev, requires_grad=True)
        kernel = delta_scan_fused_fp32 if fp32 else delta_scan_fused

        def scan():
            o, s = kernel(*ins, s0)
            (o.float().sum() + s.sum()).backward()

        out[f"delta_scan_{name}_fwd_bwd_b32_n88_h2_dk16_ms"] = round(timed(scan), 4)
    return out


# ---- CPU baseline ---------------------------------------------------------------------------------
def probe_library():
    """``libvesper_probe.so`` (bench.py's HBM streaming probes, built beside the kernel library)."""
    import ctypes

    from vesper.kernels import build as kbuild

    if not kbuild.PROBE_LIBRARY.exists():
        raise RuntimeError(f"{kbuild.PROBE_LIBRARY} is not built: run __graft_entry__.build()")
    lib = ctypes.CDLL(str(kbuild.PROBE_LIBRARY))
    lib.vsp_probe_stream.restype = ctypes.c_int
    lib.vsp_probe_stream.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int,
                                     ctypes.c_void_p]
    return lib


PROBE_MODES = {"read": 0, "copy": 1, "fill": 2, "read_nt": 3, "copy_nt": 4, "fill_nt": 5}


def time_hbm_ceiling(torch, sweep: bool = False) -> dict:
    """What HBM gives to the simplest access patterns, from hand-written streaming kernels
    (``libvesper_probe.so``: 16-byte pieces, a grid-stride loop with several pieces in flight per
    thread). Cold: 1 GiB buffers (four times the 256 MB MALL, so every pass misses it), read,
    copied and filled, per launch in a HIP graph of 5 (median of 3 replays); TB/s counts bytes read
    plus bytes written. Then the decode step's own pattern: its 8.39 MB fp32 state (b64 H8 64x64)
    read and written back in place, warm (one buffer) and cold (64 buffers rotated, 537 MB). With
    ``sweep`` every mode and workgroup count; otherwise the counts the sweep found best."""
    lib = probe_library()
    dev = torch.device("cuda:0")
    gib = 1 << 30
    a = torch.empty(gib, dtype=torch.uint8, device=dev)
    b = torch.empty(gib, dtype=torch.uint8, device=dev)
    a.fill_(1)
    b.fill_(2)
    sink = torch.zeros(16384 * 256, dtype=torch.int32, device=dev)

    def launch(mode: str, src, dst, nbytes: int, blocks: int) -> None:
        # torch's current stream at each call: under capture that is the capturing stream
        st = lib.vsp_probe_stream(PROBE_MODES[mode], src, dst, nbytes, blocks, torch.cuda.current_stream(dev).cuda_stream)
        if st != 0:
            raise RuntimeError(f"vsp_probe_stream({mode}, {nbytes}, {blocks}) returned {st}")

    out: dict = {}
    block_counts = (1024, 2048, 4096, 8192, 16384) if sweep else (4096,)
    modes = ("read", "copy", "fill", "read_nt", "copy_nt", "fill_nt") if sweep else ("read", "copy", "fill")
    for mode in modes:
        best = None
        for blocks in block_counts:
            if mode.startswith("read"):
                fn = lambda: launch(mode, a.data_ptr(), sink.data_ptr(), gib, blocks)  # noqa: E731
                moved = gib
            elif mode.startswith("copy"):
                fn = lambda: launch(mode, a.data_ptr(), b.data_ptr(), gib, blocks)  # noqa: E731
                moved = 2 * gib
            else:
                fn = lambda: launch(mode, None, b.data_ptr(), gib, blocks)  # noqa: E731
                moved = gib
            ms = captured_ms(torch, fn, 5, 3)
            tbs = moved / (ms / 1e3) / 1e12
            if sweep:
                out[f"{mode}_1GiB_blocks{blocks}_tbs"] = round(tbs, 3)
            if best is None or tbs > best[0]:
                best = (tbs, blocks, ms)
        out[f"{mode}_1GiB_cold_tbs"] = round(best[0], 3)
        out[f"{mode}_1GiB_cold_blocks"] = best[1]
    del b
    # the decode step's state: 8.39 MB read and written in place (copy onto itself)
    state_bytes = 64 * 8 * 64 * 64 * 4
    nbuf = 64
    bufs = a[: nbuf * state_bytes].view(nbuf, state_bytes)
    for blocks in ((256, 512, 1024, 2048) if sweep else (1024,)):
        warm = captured_ms(torch, lambda: launch("copy", bufs[0].data_ptr(), bufs[0].data_ptr(), state_bytes, blocks),
                           20, 3)
        it = iter(range(10**9))
        cold = captured_ms(torch, lambda: (lambda i: launch("copy", bufs[i % nbuf].data_ptr(), bufs[i % nbuf].data_ptr(),
                                                             state_bytes, blocks))(next(it)), nbuf, 3)
        key = f"state_8p39MB_inplace_blocks{blocks}" if sweep else "state_8p39MB_inplace"
        out[f"{key}_warm_us"] = round(warm * 1e3, 3)
        out[f"{key}_cold_us"] = round(cold * 1e3, 3)
        out[f"{key}_warm_tbs"] = round(2 * state_bytes / (warm / 1e3) / 1e12, 3)
        out[f"{key}_cold_tbs"] = round(2 * state_bytes / (cold / 1e3) / 1e12, 3)
    return out


def cpu_info(torch) -> dict:
    """The host the CPU legs ran on: logical CPUs, the model name lscpu reports, torch's threading."""
    model = platform.processor() or "unknown"
    try:
        import subprocess

        text = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10, check=False).stdout
        for line in text.splitlines():
            if line.strip().startswith("Model name"):
                model = line.split(":", 1)[1].strip()
                break
    except (OSError, subprocess.SubprocessError):
        pass
    info = " ".join(torch.__config__.parallel_info().split())
    return {"cpu_count": os.cpu_count(), "model": model, "parallel_info": info[:400]}


def cpu_legs(torch) -> dict:
    """The oracle on the host for the decode workload (8 warm-up steps, then the 256 steps of batch
    64: delta step on the fp32 state + ring attention over 512 bf16-valued entries and the ring
    write) and the looped column (one batch row of B4 T2048 d512 H8, 8 passes, halting 0.3, in
    float32), on all of the host's cores."""
    from oracle import loop as ol
    from oracle.attention import kv_ring_write, ring_attend
    from oracle.delta import delta_scan_step

    torch.set_num_threads(os.cpu_count() or 1)
    g = torch.Generator().manual_seed(3)
    b, h, d, w, n = DEC_B, H, D, DEC_W, DEC_STEPS
    state = 0.02 * torch.randn(b, h, d, d, generator=g)
    rk = torch.randn(b, w, h, d, generator=g).to(torch.bfloat16).float()
    rv = torch.randn(b, w, h, d, generator=g).to(torch.bfloat16).float()
    rpos = torch.arange(w).expand(b, w).contiguous()
    valid = torch.ones(b, w, dtype=torch.bool)
    out = {}
    t0 = 0.0
    for s in range(n + 8):
        if s == 8:
            t0 = time.perf_counter()
        q = torch.randn(b, h, d, generator=g)
        q = q / q.norm(dim=-1, keepdim=True)
        beta = torch.sigmoid(torch.randn(b, h, generator=g))
        _, state = delta_scan_step(q, q, q, beta, state)
        aq = torch.randn(b, 1, h, d, generator=g).to(torch.bfloat16).float()
        p = torch.full((b, 1), w + s)
        ring_attend(aq, aq, aq, p, rk, rv, rpos, valid, w)
        rk, rv, rpos, valid = kv_ring_write(rk, rv, rpos, valid, aq, aq, p)
    dt = time.perf_counter() - t0
    out["decode"] = {"tok_s": round(b * n / dt, 1), "s_256_steps": round(dt, 3),
                     "sample": "the 256-step decode workload in full after 8 warm-up steps (oracle, fp32)"}
    lb, ln, ld, passes = 1, LOOP_T, LOOP_D, LOOP_PASSES
    gw = torch.Generator().manual_seed(11)
    mats = lambda o: [(torch.randn(ld, o, generator=gw) / ld**0.5).to(torch.bfloat16).float() for _ in range(passes)]  # noqa: E731
    weights = ol.MixerWeights(wq=mats(H * D), wk=mats(H * D), wv=mats(H * D), wb=mats(H), waq=mats(H * D),
                              wak=mats(H * D), wav=mats(H * D), heads=H, kv_heads=H, head_dim=D, window=WINDOW,
                              rotary_base=10000.0)
    gx = torch.Generator().manual_seed(12)
    x0 = torch.randn(lb, ln, ld, generator=gx)
    exits = [torch.rand(lb, ln, generator=gx) < 0.3 for _ in range(passes)]
    states = [torch.zeros(lb, H, D, D) for _ in range(passes)]
    t0 = time.perf_counter()
    ol.loop_forward(x0, ol.mixer_column_step(weights, bf16=False), states, exits)
    dt = time.perf_counter() - t0
    out["looped_column"] = {"tok_s": round(lb * ln / dt, 1), "s": round(dt, 3),
                            "sample": "one batch row of the looped-column workload (T2048 d512 H8, 8 passes, "
                                      "p_halt 0.3, no key filter), oracle in float32, one run"}
    return out


# ---- CPU baseline (the headline's) ----------------------------------------------------------------
def cpu_baseline(torch) -> dict:
    from oracle.attention import window_attention as oracle_window
    from oracle.delta import delta_scan_chunked

    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    sb = B  # the whole step's batch
    q, k, v, beta, s0 = scan_inputs(torch, torch.device("cpu"), b=sb)
    aq, ak, av = attn_inputs(torch, torch.device("cpu"), b=sb)
    q, k, v, beta = (x.float() for x in (q, k, v, beta))
    aq, ak, av = (x.float() for x in (aq, ak, av))
    times = []
    for i in range(6):
        t0 = time.perf_counter()
        delta_scan_chunked(q, k, v, beta, s0, 64)
        oracle_window(aq, ak, av, WINDOW)
        if i:  # the first run warms up
            times.append(time.perf_counter() - t0)
    t = statistics.median(times)
    host = cpu_info(torch)
    return {"value": sb * T / t, "unit": "tok/s", "cores": torch.get_num_threads(), "kind": "port",
            "sample": f"one full step on the CPU: oracle delta_scan_chunked + window_attention in fp32 on the "
                      f"same inputs (B={sb}, T={T}, H={H}, d={D}, w={WINDOW}), median of 5 after 1 warm-up, "
                      f"{host['model']}", **host}


def traffic_probe(torch) -> None:
    """One launch of each bench kernel plus a plain copy of known size, for `rocprofv3 --pmc` runs.

    The copy (torch's `copy_` of COPY_BYTES) reads and writes exactly COPY_BYTES: the ratio of that
    to what FETCH_SIZE / WRITE_SIZE report for it scales the counters of the other kernels.
    """
    from vesper.kernels.delta_scan import delta_scan_fused, delta_scan_step_fused
    from vesper.kernels.keys import fused_keys
    from vesper.kernels.ring_attn import RingKVCache, ring_attention
    from vesper.kernels.window_attn import window_attention

    dev = torch.device("cuda:0")
    src = torch.ones(COPY_BYTES // 4, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    q, k, v, beta, s0 = scan_inputs(torch, dev)
    aq, ak, av = attn_inputs(torch, dev)  # the prefill step's shape, B8
    g = torch.Generator().manual_seed(3)
    b, h, d, w = DEC_B, H, D, DEC_W
    state = (0.02 * torch.randn(b, h, d, d, generator=g)).to(dev)
    ring = RingKVCache(torch.randn(b, w, h, d, generator=g).to(dev, torch.bfloat16),
                       torch.randn(b, w, h, d, generator=g).to(dev, torch.bfloat16),
                       torch.arange(w).expand(b, w).contiguous().to(dev),
                       torch.ones(b, w, dtype=torch.bool, device=dev), w)
    dq = torch.randn(b, h, d, generator=g).to(dev)
    dbeta = torch.rand(b, h, generator=g).to(dev)
    rq = torch.randn(b, 1, h, d, generator=g).to(dev, torch.bfloat16)
    pos = torch.full((b, 1), w, device=dev)
    kz = torch.randn(B, T, KEY_D, generator=g).to(dev, torch.bfloat16)
    khist = torch.randn(B, KEY_TAPS - 1, KEY_D, generator=g).to(dev)
    ktaps = torch.randn(KEY_TAPS, KEY_D, generator=g).to(dev)
    with torch.no_grad():
        dst.copy_(src)
        delta_scan_fused(q, k, v, beta, s0)
        window_attention(aq, ak, av, WINDOW)
        delta_scan_step_fused(dq, dq, dq, dbeta, state, out_state=state)
        ring_attention(rq, rq, rq, pos, ring, inplace=True, check_positions=False)
        fused_keys(kz, khist, ktaps, H)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes": COPY_BYTES}), flush=True)


def traffic_probe_backward(torch) -> None:
    """The copy of known size, then one training step of each mixer under autograd at its bench
    shape (the scan at B8 T4096 H8 d64 bf16: the forward recording the chunks' starting states and
    the backward reading them; window attention at B4 T4096 H8 D64 w512), for `rocprofv3 --pmc`."""
    from vesper.kernels.delta_scan import delta_scan_fused
    from vesper.kernels.window_attn import window_attention

    dev = torch.device("cuda:0")
    src = torch.ones(COPY_BYTES // 4, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    inputs = [t.requires_grad_() for t in scan_inputs(torch, dev)]
    g = torch.Generator().manual_seed(8)
    d_o = torch.randn(inputs[0].shape, generator=g).to(dev, torch.bfloat16)
    d_s = torch.randn(inputs[4].shape, generator=g).to(dev)
    aq, ak, av = (t.requires_grad_() for t in attn_inputs(torch, dev, b=ATTN_B))
    d_a = torch.randn(aq.shape, generator=g).to(dev, torch.bfloat16)
    with torch.no_grad():
        dst.copy_(src)
    o, s = delta_scan_fused(*inputs)
    torch.autograd.backward([o, s], [d_o, d_s])
    a = window_attention(aq, ak, av, WINDOW)
    torch.autograd.backward([a], [d_a])
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes": COPY_BYTES}), flush=True)


def traffic_from_profiles(kernel: str) -> float | None:
    path = ROOT / "profiles" / "hbm_traffic.json"
    if not path.exists():
        return None
    try:
        data = json.loads(path.read_text())
        return float(data[kernel]["bytes_per_launch"])
    except (KeyError, ValueError, TypeError):
        return None


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-decode", action="store_true")
    ap.add_argument("--no-loop", action="store_true")
    ap.add_argument("--traffic-probe-backward", action="store_true",
                    help="one training step of each mixer after a copy of known size, for rocprofv3 --pmc")
    ap.add_argument("--traffic-probe", action="store_true",
                    help="launch each kernel once plus a calibration copy, for rocprofv3 --pmc runs")
    ap.add_argument("--hbm-ceiling", action="store_true",
                    help="only the HBM streaming probes, every mode and workgroup count (one JSON line)")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU: the mixers shard over (batch, head) with no exchange, and this build "
              f"runs no multi-GPU path (asked for --gpus {args.gpus}, WORLD_SIZE {world})", file=sys.stderr)
        return 2

    import torch

    if not torch.cuda.is_available():
        log("no HIP device")
        return 1
    from vesper.kernels import _lib

    _lib.library()  # fail loudly if the kernels are not built
    if args.traffic_probe:
        traffic_probe(torch)
        return 0
    if args.traffic_probe_backward:
        traffic_probe_backward(torch)
        return 0
    if args.hbm_ceiling:
        print(json.dumps({"hbm_ceiling": time_hbm_ceiling(torch, sweep=True)}), flush=True)
        return 0

    def leg(fn, *a):
        """A leg's result, once every kernel it queued (graph replays included) has completed with no
        bounded wait giving up: a replay whose scan hand-over gave up writes NaN and must not pass
        as a timing."""
        out = fn(torch, *a)
        _lib.check_faults(synchronize=True)
        return out

    pre = leg(time_prefill, args.steps, args.warmup)
    tok_s = B * T / (pre["step_ms"] / 1e3)
    s_bytes, s_flops = scan_bytes(B, T, H, D), scan_flops(B, T, H, D)
    a_bytes, a_flops = attn_bytes(B, T, H, H, D), attn_flops(B, T, H, D, WINDOW)
    attn4_ms = leg(time_attention_config)
    attn4_bwd_ms = leg(time_attention_backward)
    scan_bwd = leg(time_scan_backward)
    keys_ms, keys_bwd_ms = leg(time_key_filter)
    dec = None if args.no_decode else leg(time_decode)
    dec_cold_us = None if args.no_decode else leg(time_decode_cold)
    cold_warm = leg(time_cold_warm)
    published = leg(time_published_shapes)
    looped = None if args.no_loop else leg(time_looped)
    col_dec = None if args.no_decode else leg(time_column_decode)

    # the dominant kernel by its time per launch in a graph of 10 launches (median of 5 replays)
    scan_dominant = pre["scan_ms"] >= pre["attn_ms"]
    if scan_dominant:
        name, ms, nbytes, flops = "delta_scan (prep + chain kernels)", pre["scan_ms"], s_bytes, s_flops
        traffic = traffic_from_profiles("delta_scan")
    else:
        name, ms, nbytes, flops = "window_attn_kernel", pre["attn_ms"], a_bytes, a_flops
        traffic = traffic_from_profiles("window_attn")
    achieved = nbytes / (ms / 1e3) / 1e9
    roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic, "kernel": name,
                "algorithmic_bytes": nbytes, "algorithmic_flops": flops,
                "mfma_frac_bf16": round(flops / (ms / 1e3) / 1e12 / BF16_PEAK_TFLOPS, 4),
                "avg_launch_ms": round(ms, 4),
                "launch_ms_statistic": "per launch in a HIP graph of 10, median of 5 replays"}
    # both prefill kernels, whichever dominates this run (their times are close)
    roofline["per_kernel"] = {
        "delta_scan": {"ms": round(pre["scan_ms"], 4),
                       "hbm_frac": round(s_bytes / (pre["scan_ms"] / 1e3) / 1e9 / HBM_PEAK_GBS, 4),
                       "mfma_frac_bf16": round(s_flops / (pre["scan_ms"] / 1e3) / 1e12 / BF16_PEAK_TFLOPS, 4),
                       "traffic": traffic_from_profiles("delta_scan")},
        "window_attn": {"ms": round(pre["attn_ms"], 4),
                        "hbm_frac": round(a_bytes / (pre["attn_ms"] / 1e3) / 1e9 / HBM_PEAK_GBS, 4),
                        "mfma_frac_bf16": round(a_flops / (pre["attn_ms"] / 1e3) / 1e12 / BF16_PEAK_TFLOPS, 4),
                        "traffic": traffic_from_profiles("window_attn")},
    }

    result = {
        "metric": "delta-scan+window-attn prefill tok/s @T=4096; decode tok/s; % of roofline",
        "value": round(tok_s, 1),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(pre["step_ms"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1); q, k L2-normalised; beta = sigmoid(N(0,1)); S0 ~ N(0, 0.02^2))",
        "config": {
            "workload": "column mixers prefill: delta scan B8 T4096 H8 d64 chunk 64 (bf16 in, fp32 state) + "
                        "window attention B8 T4096 H8 D64 w512 (bf16)",
            "global_batch": B, "seq_len": T, "heads": H, "head_dim": D, "window": WINDOW, "parallelism": "none",
        },
        "kernels": {
            "delta_scan_ms": round(pre["scan_ms"], 4),
            "prefill_step_eager_ms": round(pre["eager_step_ms"], 4),
            "delta_scan_eager_ms": round(pre["eager_scan_ms"], 4),
            "window_attn_b8_eager_ms": round(pre["eager_attn_ms"], 4),
            "delta_scan_tok_s": round(B * T / (pre["scan_ms"] / 1e3), 1),
            "delta_scan_hbm_frac": round(s_bytes / (pre["scan_ms"] / 1e3) / 1e9 / HBM_PEAK_GBS, 4),
            "delta_scan_mfma_frac_bf16": round(s_flops / (pre["scan_ms"] / 1e3) / 1e12 / BF16_PEAK_TFLOPS, 4),
            "delta_scan_backward_ms": round(scan_bwd["recorded_ms"], 4),
            "delta_scan_backward_note": "autograd's path: the states at the chunks' starts recorded by the forward",
            "delta_scan_forward_recording_ms": round(scan_bwd["forward_recording_ms"], 4),
            "delta_scan_backward_recomputing_states_ms": round(scan_bwd["alone_ms"], 4),
            "window_attn_b8_ms": round(pre["attn_ms"], 4),
            "window_attn_b4_ms": round(attn4_ms, 4),
            "window_attn_b4_tok_s": round(ATTN_B * T / (attn4_ms / 1e3), 1),
            "window_attn_b4_hbm_frac": round(attn_bytes(ATTN_B, T, H, H, D) / (attn4_ms / 1e3) / 1e9 / HBM_PEAK_GBS, 4),
            "window_attn_b4_mfma_frac_bf16": round(attn_flops(ATTN_B, T, H, D, WINDOW) / (attn4_ms / 1e3) / 1e12 / BF16_PEAK_TFLOPS, 4),
            "window_attn_b4_backward_ms": round(attn4_bwd_ms, 4),
            # algorithmic backward work: 2.5x the forward's (QK^T again, dP, dQ, dK, dV)
            "window_attn_b4_backward_mfma_frac_bf16": round(2.5 * attn_flops(ATTN_B, T, H, D, WINDOW) / (attn4_bwd_ms / 1e3) / 1e12 / BF16_PEAK_TFLOPS, 4),
        },
        "roofline": roofline,
    }
    k_bytes = key_filter_bytes(B, T, KEY_D, KEY_TAPS)
    kb_bytes = key_filter_backward_bytes(B, T, KEY_D, KEY_TAPS)
    result["key_filter"] = {
        "workload": "causal key filter + per-head key normalization: B8 T4096 d512 (8 heads of 64), 4 taps, bf16 "
                    "keys, float32 history and taps; backward = d z, d taps, d history from the keys' gradient",
        "us": round(keys_ms * 1e3, 3), "tok_s": round(B * T / (keys_ms / 1e3), 1),
        "hbm_frac": round(k_bytes / (keys_ms / 1e3) / 1e9 / HBM_PEAK_GBS, 4), "algorithmic_bytes": k_bytes,
        "backward_us": round(keys_bwd_ms * 1e3, 3),
        "backward_hbm_frac": round(kb_bytes / (keys_bwd_ms / 1e3) / 1e9 / HBM_PEAK_GBS, 4),
        "backward_algorithmic_bytes": kb_bytes,
    }
    if dec is not None:
        step_bytes = decode_step_bytes(DEC_B, H, D, DEC_W)
        result["decode"] = {
            "workload": "256 steps, batch 64, H8 d64: fp32 delta step on S [64,8,64,64] + attention over a 512-entry "
                        "bf16 KV ring, one HIP graph",
            "tok_s": round(dec["tok_s"], 1), "us_per_step": round(dec["us_per_step"], 3),
            "hbm_frac": round(step_bytes / (dec["us_per_step"] / 1e6) / 1e9 / HBM_PEAK_GBS, 4),
            "algorithmic_bytes_per_step": step_bytes,
        }
    if col_dec is not None:
        result["column_decode"] = {
            "workload": "captured single-token decode of the looped column: batch 64, d512 H8 d64, 8 passes dense, "
                        "each pass key filter (4 taps) + fp32 delta step + attention over a full 512-entry bf16 KV "
                        "ring, bf16 projections; one HIP graph replay per step",
            "tok_s": round(col_dec["tok_s"], 1), "us_per_step": round(col_dec["us_per_step"], 3),
            "us_per_pass": round(col_dec["us_per_step"] / LOOP_PASSES, 3),
        }
    if looped is not None:
        result["looped_column"] = {
            "workload": "looped column with per-token halting: B4 T2048 d512 H8 d64, 8 passes of key filter (4 taps) "
                        "+ delta scan + window attention (w512) with bf16 projections (fixed N(0, 1/512) weights), "
                        "p_halt 0.3, copy-forward of halted tokens",
            "tok_s": round(looped["tok_s"], 1), "ms": round(looped["ms"], 3),
            "copy_forward": "fused into the kernels' loads; one row-copy launch per pass",
            "ms_with_where_merges": round(looped["ms_where"], 3),
            "ms_captured": round(looped["ms_captured"], 3),
            "mean_active_passes": round(looped["mean_passes"], 3),
        }
    result["cold_warm"] = {
        "method": "median of 52 launches after 10 warm-ups; warm: one input set; cold: input sets rotated "
                  "so more than 512 MB lie between two uses of a set (the MALL is 256 MB)",
        **{k: round(v, 4) for k, v in cold_warm.items()},
        "delta_scan_bf16_b8_cold_hbm_frac": round(s_bytes / (cold_warm["delta_scan_bf16_b8_cold_ms"] / 1e3) / 1e9
                                                  / HBM_PEAK_GBS, 4),
    }
    result["kernels"]["delta_scan_fp32_c1_b2_t512_h4_ms"] = round(cold_warm["delta_scan_fp32_c1_b2_t512_h4_warm_ms"], 4)
    result["kernels"]["delta_scan_fp32_b8_t4096_h8_ms"] = round(cold_warm["delta_scan_fp32_b8_t4096_h8_warm_ms"], 4)
    result["published_shapes"] = {"note": "context only: the reference quotes these on NVIDIA cards "
                                          "(window_attn.py:10-13, delta_scan.py:22-24)", **published}
    if dec is not None and dec_cold_us is not None:
        step_bytes = decode_step_bytes(DEC_B, H, D, DEC_W)
        result["decode"]["cold_us_per_step"] = round(dec_cold_us, 3)
        result["decode"]["cold_hbm_frac"] = round(step_bytes / (dec_cold_us / 1e6) / 1e9 / HBM_PEAK_GBS, 4)
        result["decode"]["cold_tok_s"] = round(DEC_B / (dec_cold_us / 1e6), 1)
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(torch)
        result["cpu_legs"] = cpu_legs(torch)
    log(f"prefill step {pre['step_ms']:.4f} ms captured, {pre['eager_step_ms']:.4f} eager (scan {pre['scan_ms']:.4f}, "
        f"attn {pre['attn_ms']:.4f}), wall {pre['wall_s']:.2f} s")
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
