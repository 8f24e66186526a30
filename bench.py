"""Benchmark of the fused sequence-mixing kernels on one MI355X.

Headline (one JSON line, BASELINE.json metric): the config-2 Mamba selective scan,
forward + backward (B=8, T=2048, D=1536, N=16; u, dt, z bf16; A, B, C, D f32), as
whole-step algorithmic HBM GB/s.  A "step" is one forward (writing the backward's
state checkpoints) plus one backward over one batch of synthetic input already
resident in HBM.  The other configs are reported under "configs" (not the value).

Algorithmic bytes (per call, what roofline.achieved divides by):
  selective scan fwd = 4*B*T*D*2 (u, dt, z, y) + 2*B*T*N*4 (B, C) + D*N*4 + D*4
  selective scan bwd = 7*B*T*D*2 (u, dt, z, dy in; du, ddt, dz out) + 4*B*T*N*4 + 2*(D*N*4 + D*4)
  MinGRU fwd = 3*B*T*H*s, bwd = 6*B*T*H*s (s = element size)
  linear scan fwd = 3*B*T*H*s (a, b in; h out), bwd = 5*B*T*H*s (a, h, dy in; da, db out)

Timing: the headline value times exactly K fwd+bwd steps (after W warm-ups) with host
synchronisation on both sides; every per-kernel figure (and each config's roofline) is the
median of max(K, 50) HIP-event timed runs after max(W, 10) warm-ups, events recorded on the
stream the kernels are launched on; the scan rows evict the caches before each timed run by
reading a 512 MiB buffer (the 256 MB MALL could otherwise hold a whole scan's inputs; a read
leaves no dirty lines to be written back during the timed run, see --flush).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--only mingru,block,linear,c3,delta,c4,flash,hybrid]
       [--flush read|write|none] [--copy-probe]
(the config-2 headline always runs; --only selects the other rows)
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import tempfile
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0
# VALU issue slots per second: 256 CUs x 4 SIMDs x 16 lanes at the 2.4 GHz shader clock
# measured under load (a wave64 FMA occupies a SIMD for 4 cycles = 64 lane slots)
VALU_PEAK_TSLOTS = 256 * 4 * 16 * 2.4e9 / 1e12
# Selective scan, VALU issue slots per (b, t, d, n) element that the recurrence itself needs,
# v_exp_f32 counted as 2.5 (10 cycles per wave instruction, measured, against 4 for an FMA):
#   forward  dt * A, exp, B * dt_b x, state update, C * h and its sum over the states   -> 7.5
#   backward the forward's first four again (5.5); dh += dy C, dy h, dh dt_b x, dh B,
#            dh *= a, dh h_prev, dA += ... (7); the sums over states (dx, ddt) and over
#            channels (dB, dC), one add each (4)                                     -> 16.5
SS_VALU_SLOTS = (7.5, 16.5)


def ss_bytes(B, T, D, N):
    fwd = 4 * B * T * D * 2 + 2 * B * T * N * 4 + D * N * 4 + D * 4
    bwd = 7 * B * T * D * 2 + 4 * B * T * N * 4 + 2 * (D * N * 4 + D * 4)
    return fwd, bwd


MIN_RUNS, MIN_WARMUP = 50, 10


class Flush:
    """Cache eviction between timed runs.  The default ("read") sums a 512 MiB buffer: twice
    the 256 MB MALL, so the next run's inputs come from HBM, and the evicting lines are clean.
    "write" fills 256 MiB instead; the dirty lines it leaves in L2 / MALL are written back
    during the next timed run and bill that run for up to 256 MiB of extra HBM writes.
    "none" times back-to-back runs."""

    mode = "read"

    def __init__(self, torch):
        self.torch = torch
        n = (128 if self.mode == "read" else 64) * 2 ** 20
        self.buf = torch.ones(n, dtype=torch.float32, device="cuda") if self.mode != "none" else None

    def __call__(self):
        if self.mode == "read":
            self.torch.sum(self.buf)
        elif self.mode == "write":
            self.buf.fill_(1.0)


def median_ms(torch, fn, runs, warmup, flush=None):
    """Median duration (ms) of one call of ``fn`` over ``runs`` timed runs after ``warmup``
    untimed ones, from HIP events on torch's current stream (the stream every entry point here
    launches on); ``flush`` runs before each timed call, outside the events."""
    for _ in range(warmup):
        fn()
    pairs = []
    for _ in range(runs):
        if flush is not None:
            flush()
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        fn()
        e.record()
        pairs.append((s, e))
    torch.cuda.synchronize()
    return float(np.median([s.elapsed_time(e) for s, e in pairs]))


def roofline(bound, work, ms, kernels=None, profile=None):
    """Roofline dict for ``work`` algorithmic bytes ("hbm") or flops ("mfma") done in ``ms``;
    ``traffic`` is the HBM bytes of the named kernels per call from the committed rocprofv3
    FETCH_SIZE / WRITE_SIZE summary ``profiles/<profile>`` (None when not profiled)."""
    if bound == "hbm":
        achieved, peak, unit = work / ms / 1e6, HBM_PEAK_GBS, "GB/s"
    else:
        achieved, peak, unit = work / ms / 1e9, MFMA_BF16_PEAK_TFLOPS, "TFLOP/s"
    traffic = profiled_traffic(kernels, os.path.join(ROOT, "profiles", profile)) if kernels and profile else None
    return {"bound": bound, "achieved": round(achieved, 1), "peak": peak, "unit": unit,
            "frac": round(achieved / peak, 4), "traffic": traffic}


def bench_selective_scan(torch, steps, warmup, B=8, T=2048, D=1536, N=16):
    from edifice_amd import _native as nat
    from edifice_amd import fused_scan as fs

    g = torch.Generator(device="cuda").manual_seed(2000)
    dev = "cuda"
    bf, f32 = torch.bfloat16, torch.float32
    x = torch.randn(B, T, D, device=dev, generator=g).to(bf)
    dt = torch.nn.functional.softplus(torch.randn(B, T, D, device=dev, generator=g) - 4).to(bf)
    A = -torch.exp(torch.rand(D, N, device=dev, generator=g) * np.log(16.0))
    Bm = torch.randn(B, T, N, device=dev, generator=g)
    Cm = torch.randn(B, T, N, device=dev, generator=g)
    Dv = torch.randn(D, device=dev, generator=g)
    z = torch.randn(B, T, D, device=dev, generator=g).to(bf)
    dy = torch.randn(B, T, D, device=dev, generator=g).to(bf)
    out = torch.empty_like(x)
    states = torch.empty(nat.query("edf_selective_scan_states_bytes", B, T, D, N) // 4, dtype=f32, device=dev)
    dx, ddt, dz = torch.empty_like(x), torch.empty_like(x), torch.empty_like(x)
    dA = torch.empty(D, N, dtype=f32, device=dev)
    dB = torch.empty(B, T, N, dtype=f32, device=dev)
    dC = torch.empty(B, T, N, dtype=f32, device=dev)
    dD = torch.empty(D, dtype=f32, device=dev)
    wsb = nat.query("edf_selective_scan_backward_workspace_bytes", B, T, D, N, 0, 1)
    ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
    P = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)

    def fwd():
        nat.call("edf_fused_selective_scan", stream, P(x), P(dt), P(A), P(Bm), P(Cm), P(Dv), P(z), P(out),
                 P(states), None, 0, B, T, D, N, 1, 0, 0)

    def bwd():
        nat.call("edf_fused_selective_scan_backward", stream, P(x), P(dt), P(A), P(Bm), P(Cm), P(Dv), P(z), P(dy),
                 P(states), P(dx), P(ddt), P(dA), P(dB), P(dC), P(dD), P(dz), P(ws), wsb, B, T, D, N, 1, 0, 0)

    # the headline step: exactly `steps` fwd+bwd steps after `warmup`, host-synchronised
    for _ in range(warmup):
        fwd()
        bwd()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        fwd()
        bwd()
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) / steps
    # per-kernel medians (caches evicted before each run)
    runs, wu, fl = max(steps, MIN_RUNS), max(warmup, MIN_WARMUP), Flush(torch)
    fwd_ms = median_ms(torch, fwd, runs, wu, fl)
    bwd_ms = median_ms(torch, bwd, runs, wu, fl)
    fb, bb = ss_bytes(B, T, D, N)
    _ = fs  # imported for its side effect of validating the package import
    return dict(fwd_ms=fwd_ms, bwd_ms=bwd_ms, step_ms=wall * 1e3, fwd_bytes=fb, bwd_bytes=bb, runs=runs,
                fwd_gbs=fb / fwd_ms / 1e6, bwd_gbs=bb / bwd_ms / 1e6, step_gbs=(fb + bb) / (wall * 1e3) / 1e6,
                roofline=roofline("hbm", fb + bb, fwd_ms + bwd_ms,
                                  ["ss_fwd_kernel", "ss_bwd_kernel", "ss_reduce_bc_kernel", "ss_reduce_ad_kernel"],
                                  "selective_scan_c2.md"))


def bench_mingru(torch, steps, warmup, B, T, H, dtype):
    from edifice_amd import _native as nat

    dev = "cuda"
    g = torch.Generator(device="cuda").manual_seed(1000)
    gates = torch.randn(B, T, H, device=dev, generator=g).to(dtype)
    cand = torch.randn(B, T, H, device=dev, generator=g).to(dtype)
    dy = torch.randn(B, T, H, device=dev, generator=g).to(dtype)
    out, dg, dc = torch.empty_like(gates), torch.empty_like(gates), torch.empty_like(gates)
    flag = 1 if dtype == torch.bfloat16 else 0
    P = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)

    def fwd():
        nat.call("edf_mingru", stream, P(gates), P(cand), P(out), B, T, H, flag)

    def bwd():
        nat.call("edf_mingru_backward", stream, P(gates), P(cand), P(out), P(dy), P(dg), P(dc), B, T, H, flag)

    runs, wu, fl = max(steps, MIN_RUNS), max(warmup, MIN_WARMUP), Flush(torch)
    fwd_ms, bwd_ms = median_ms(torch, fwd, runs, wu, fl), median_ms(torch, bwd, runs, wu, fl)
    s = gates.element_size()
    fb, bb = 3 * B * T * H * s, 6 * B * T * H * s
    prof = "linear_scans_8x2048x1536.md" if (B, T, H) == (8, 2048, 1536) else None
    return dict(shape=[B, T, H], dtype=str(dtype).replace("torch.", ""), fwd_us=fwd_ms * 1e3, bwd_us=bwd_ms * 1e3,
                fwd_gbs=fb / fwd_ms / 1e6, bwd_gbs=bb / bwd_ms / 1e6, runs=runs,
                roofline=roofline("hbm", fb + bb, fwd_ms + bwd_ms, None, prof))


def bench_hbm_ceiling(torch, steps, warmup, nbytes=8 * 2048 * 1536 * 2):
    """The HBM rate a plain streaming kernel of this library reaches (edf_probe_stream, a
    layout-free 16-byte-per-lane stream declared in tests/edifice_hip_probes.h): out = in0 + in1
    over `nbytes` per stream (2 reads + 1 write, the MinGRU forward's traffic at the bandwidth
    row's bf16 size) and out = in0 (1 read + 1 write), caches evicted before each run, over a
    sweep of grid sizes; the best of the sweep is the ceiling the scan rows are read against."""
    from edifice_amd import _native as nat

    fn = nat.lib().edf_probe_stream
    fn.restype = ctypes.c_int
    fn.argtypes = [ctypes.c_void_p] * 4 + [ctypes.c_long, ctypes.c_int, ctypes.c_int]
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    a = torch.ones(nbytes // 4, dtype=torch.int32, device="cuda")
    b, o = torch.ones_like(a), torch.empty_like(a)
    runs, wu, fl = max(steps, MIN_RUNS), max(warmup, MIN_WARMUP), Flush(torch)
    out = {}
    for nin in (2, 1):
        best = None
        for blocks in (512, 1024, 2048, 4096, 8192):
            def run():
                rc = fn(stream, a.data_ptr(), b.data_ptr(), o.data_ptr(), nbytes, nin, blocks)
                if rc != 0:
                    raise RuntimeError(nat.lib().edf_last_error().decode())
            ms = median_ms(torch, run, runs, wu, fl)
            gbs = (nin + 1) * nbytes / ms / 1e6
            if best is None or gbs > best[1]:
                best = (blocks, gbs, ms)
        key = "read2_write1" if nin == 2 else "read1_write1"
        out[key] = dict(bytes=(nin + 1) * nbytes, us=round(best[2] * 1e3, 2), gbs=round(best[1], 1),
                        frac_of_peak=round(best[1] / HBM_PEAK_GBS, 4), blocks=best[0])
    return out


def bench_linear_scan(torch, steps, warmup, B, T, H, dtype):
    """Generic linear scan h_t = a_t h_{t-1} + b_t (fwd reads a, b, writes h; bwd reads a,
    h, dy, writes da, db)."""
    from edifice_amd import _native as nat

    dev = "cuda"
    g = torch.Generator(device="cuda").manual_seed(1001)
    a = torch.rand(B, T, H, device=dev, generator=g).to(dtype)
    b = torch.randn(B, T, H, device=dev, generator=g).to(dtype)
    dy = torch.randn(B, T, H, device=dev, generator=g).to(dtype)
    out, da, db = torch.empty_like(a), torch.empty_like(a), torch.empty_like(a)
    flag = 1 if dtype == torch.bfloat16 else 0
    P = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)

    def fwd():
        nat.call("edf_fused_linear_scan", stream, P(a), P(b), None, P(out), B, T, H, flag)

    def bwd():
        nat.call("edf_fused_linear_scan_backward", stream, P(a), None, P(out), P(dy), P(da), P(db), None, B, T, H,
                 flag)

    runs, wu, fl = max(steps, MIN_RUNS), max(warmup, MIN_WARMUP), Flush(torch)
    fwd_ms, bwd_ms = median_ms(torch, fwd, runs, wu, fl), median_ms(torch, bwd, runs, wu, fl)
    s = a.element_size()
    fb, bb = 3 * B * T * H * s, 5 * B * T * H * s
    return dict(shape=[B, T, H], dtype=str(dtype).replace("torch.", ""), fwd_us=fwd_ms * 1e3, bwd_us=bwd_ms * 1e3,
                fwd_gbs=fb / fwd_ms / 1e6, bwd_gbs=bb / bwd_ms / 1e6, runs=runs,
                roofline=roofline("hbm", fb + bb, fwd_ms + bwd_ms))


def bench_block(torch, steps, warmup, B, T, H, L, dtype, kind="mingru"):
    """Multi-layer block inference (FusedScan.{mingru,minlstm,linear}_block/4): per layer
    LayerNorm, P projections (2 P B T H^2 flops; P = 3 for MinLSTM, else 2), scan, residual."""
    from edifice_amd import _native as nat

    dev = "cuda"
    g = torch.Generator(device="cuda").manual_seed(1002)
    x = torch.randn(B, T, H, device=dev, generator=g).to(dtype)
    nproj = 3 if kind == "minlstm" else 2
    w = (torch.randn(L * (nproj * (H * H + H) + 2 * H), device=dev, generator=g) * H ** -0.5).to(dtype)
    out = torch.empty_like(x)
    flag = 1 if dtype == torch.bfloat16 else 0
    wsb = nat.query(f"edf_{kind}_block_workspace_bytes", B, T, H, L, flag)
    ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
    P = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)

    def fwd():
        nat.call(f"edf_fused_{kind}_block_scan", stream, P(x), P(w), None, P(out), P(ws), wsb, B, T, H, L, flag)

    ms = median_ms(torch, fwd, max(steps, MIN_RUNS), max(warmup, MIN_WARMUP))
    return dict(shape=[B, T, H], layers=L, dtype=str(dtype).replace("torch.", ""), ms=ms,
                tokens_per_s=B * T / ms * 1e3, projection_tflops=2 * nproj * B * T * H * H * L / ms / 1e9)


def profiled_traffic(kernels, path=os.path.join(ROOT, "profiles", "selective_scan_c2.md")):
    """HBM bytes per launch of the named kernels, from the committed rocprofv3
    FETCH_SIZE / WRITE_SIZE summary (scaled by the copy-kernel reference there); None if absent."""
    import re

    try:
        text = open(path).read()
    except OSError:
        return None
    found = dict((k, int(v)) for k, v in re.findall(r"traffic_bytes\[(\w+)\] = (\d+)", text))
    if kernels == ["*"]:
        return sum(found.values()) if found else None
    if not all(k in found for k in kernels):
        return None
    return sum(found[k] for k in kernels)


def _time_pair(torch, steps, warmup, fwd, bwd, runs=None):
    """Medians of the forward and the backward entry point (no cache eviction: these rows are
    compute-bound)."""
    runs = runs or max(steps, MIN_RUNS)
    wu = max(warmup, MIN_WARMUP)
    return median_ms(torch, fwd, runs, wu), median_ms(torch, bwd, runs, wu)


def bench_delta_rule(torch, steps, warmup, B=4, H=16, T=4096, d=128, C=64):
    """Config 3: gated delta rule, bf16 I/O, per-head beta, f32 state.  The backward is the
    one the autograd path runs: from the per-chunk context the forward left in its workspace.
    Algorithmic flops (chunked-form convention): fwd 2 (5 C d + 3 d^2) per token-head, bwd 2x fwd."""
    from edifice_amd import _native as nat

    g = torch.Generator(device="cuda").manual_seed(3000)
    dev, bf = "cuda", torch.bfloat16

    def l2n(x):
        return x / torch.sqrt((x * x).sum(-1, keepdim=True) + 1e-6)

    q = l2n(torch.randn(B, T, H, d, device=dev, generator=g)).to(bf)
    k = l2n(torch.randn(B, T, H, d, device=dev, generator=g)).to(bf)
    v = torch.randn(B, T, H, d, device=dev, generator=g).to(bf)
    beta = torch.sigmoid(torch.randn(B, T, H, device=dev, generator=g)).to(bf)
    alpha = torch.exp(-torch.nn.functional.softplus(torch.randn(B, T, H, device=dev, generator=g))).to(bf)
    do = torch.randn(B, T, H, d, device=dev, generator=g).to(bf)
    out = torch.empty_like(v)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    db, da = torch.empty_like(beta), torch.empty_like(alpha)
    wsf = nat.query("edf_delta_rule_workspace_bytes", B, T, H, d, 1, 1)
    wsb = nat.query("edf_delta_rule_saved_backward_workspace_bytes", B, T, H, d, 1, 1)
    ws1 = torch.empty(max(wsf, 1), dtype=torch.uint8, device=dev)
    ws2 = torch.empty(max(wsb, 1), dtype=torch.uint8, device=dev)
    P = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)

    def fwd():
        nat.call("edf_fused_gated_delta_net_scan", stream, P(q), P(k), P(v), P(beta), P(alpha), P(out), P(ws1), wsf,
                 B, T, H, d, 1, 1)

    def bwd():  # from the context the forward left in its workspace (as fused_scan's autograd does)
        nat.call("edf_fused_delta_rule_scan_backward_saved", stream, P(q), P(k), P(v), P(beta), P(alpha), P(do),
                 P(dq), P(dk), P(dv), P(db), P(da), P(ws1), wsf, P(ws2), wsb, B, T, H, d, 1, 1)

    fwd_ms, bwd_ms = _time_pair(torch, steps, warmup, fwd, bwd)
    fflops = 2 * (5 * C * d + 3 * d * d) * B * H * T
    bflops = 2 * fflops
    return dict(fwd_ms=fwd_ms, bwd_ms=bwd_ms, fwd_tflops=fflops / fwd_ms / 1e9, bwd_tflops=bflops / bwd_ms / 1e9,
                fwd_bwd_tflops=(fflops + bflops) / (fwd_ms + bwd_ms) / 1e9,
                fwd_bwd_mfma_frac=(fflops + bflops) / (fwd_ms + bwd_ms) / 1e9 / MFMA_BF16_PEAK_TFLOPS,
                runs=max(steps, MIN_RUNS), shape=dict(B=B, H=H, T=T, d=d, chunk=C),
                roofline=roofline("mfma", fflops + bflops, fwd_ms + bwd_ms, ["*"], "delta_rule_c3.md"))


def bench_flash(torch, steps, warmup, B=4, H=32, T=4096, d=128, causal=True):
    """Config 4: causal flash attention, bf16.  Flops: fwd 4 B H T^2 d (/ 2 when causal), bwd 2.5x fwd."""
    from edifice_amd import _native as nat

    g = torch.Generator(device="cuda").manual_seed(4000)
    dev, bf = "cuda", torch.bfloat16
    std = d ** -0.25
    q, k, v, do = (torch.randn(B, H, T, d, device=dev, generator=g).mul_(std).to(bf) for _ in range(4))
    out = torch.empty_like(q)
    lse = torch.empty(B, H, T, dtype=torch.float32, device=dev)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    wsb = nat.query("edf_flash_attention_backward_workspace_bytes", B, H, T, d)
    ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
    P = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)

    def fwd():
        nat.call("edf_fused_flash_attention", stream, P(q), P(k), P(v), P(out), P(lse), B, H, T, d, int(causal), 1)

    def bwd():
        nat.call("edf_fused_flash_attention_backward", stream, P(q), P(k), P(v), P(out), P(do), P(lse), P(dq),
                 P(dk), P(dv), P(ws), wsb, B, H, T, d, int(causal), 1)

    fwd_ms, bwd_ms = _time_pair(torch, steps, warmup, fwd, bwd)
    fflops = 4 * B * H * T * T * d / (2 if causal else 1)
    bflops = 2.5 * fflops
    prof = "flash_c4.md" if (causal and (B, H, T, d) == (4, 32, 4096, 128)) else None
    return dict(fwd_ms=fwd_ms, bwd_ms=bwd_ms, fwd_tflops=fflops / fwd_ms / 1e9, bwd_tflops=bflops / bwd_ms / 1e9,
                fwd_bwd_tflops=(fflops + bflops) / (fwd_ms + bwd_ms) / 1e9,
                fwd_bwd_mfma_frac=(fflops + bflops) / (fwd_ms + bwd_ms) / 1e9 / MFMA_BF16_PEAK_TFLOPS,
                runs=max(steps, MIN_RUNS), shape=dict(B=B, H=H, T=T, d=d, causal=causal),
                roofline=roofline("mfma", fflops + bflops, fwd_ms + bwd_ms, ["*"], prof))


def bench_fox(torch, steps, warmup, B=4, H=32, T=4096, d=128):
    """FoX (forgetting) attention at the config-4 shape, bf16, causal: flops as config 4."""
    from edifice_amd import _native as nat

    g = torch.Generator(device="cuda").manual_seed(4001)
    dev, bf = "cuda", torch.bfloat16
    std = d ** -0.25
    q, k, v, do = (torch.randn(B, H, T, d, device=dev, generator=g).mul_(std).to(bf) for _ in range(4))
    cs = torch.cumsum(torch.nn.functional.logsigmoid(torch.randn(B, H, T, device=dev, generator=g) + 2.0), -1).to(bf)
    out = torch.empty_like(q)
    lse = torch.empty(B, H, T, dtype=torch.float32, device=dev)
    dq, dk, dv, dcs = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v), torch.empty_like(cs)
    wsb = nat.query("edf_fox_attention_backward_workspace_bytes", B, H, T, d)
    ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
    P = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)

    def fwd():
        nat.call("edf_fused_fox_attention", stream, P(q), P(k), P(v), P(cs), P(out), P(lse), B, H, T, d, 1)

    def bwd():
        nat.call("edf_fused_fox_attention_backward", stream, P(q), P(k), P(v), P(cs), P(out), P(do), P(lse), P(dq),
                 P(dk), P(dv), P(dcs), P(ws), wsb, B, H, T, d, 1)

    fwd_ms, bwd_ms = _time_pair(torch, steps, warmup, fwd, bwd)
    fflops = 4 * B * H * T * T * d / 2
    bflops = 2.5 * fflops
    return dict(fwd_ms=fwd_ms, bwd_ms=bwd_ms, fwd_tflops=fflops / fwd_ms / 1e9, bwd_tflops=bflops / bwd_ms / 1e9,
                fwd_bwd_tflops=(fflops + bflops) / (fwd_ms + bwd_ms) / 1e9,
                fwd_bwd_mfma_frac=(fflops + bflops) / (fwd_ms + bwd_ms) / 1e9 / MFMA_BF16_PEAK_TFLOPS,
                shape=dict(B=B, H=H, T=T, d=d, causal=True))


def bench_kda(torch, steps, warmup, B=8, T=2048, H=8, d=128):
    """KDA (per-row log decay, per-head beta), bf16, on the exact per-step kernels: fwd and bwd
    time per call and tokens/s (B T per call)."""
    from edifice_amd import _native as nat

    g = torch.Generator(device="cuda").manual_seed(3001)
    dev, bf = "cuda", torch.bfloat16
    l2n = lambda x: x / torch.sqrt((x * x).sum(-1, keepdim=True) + 1e-6)  # noqa: E731
    q = l2n(torch.randn(B, T, H, d, device=dev, generator=g)).to(bf)
    k = l2n(torch.randn(B, T, H, d, device=dev, generator=g)).to(bf)
    v = torch.randn(B, T, H, d, device=dev, generator=g).to(bf)
    alpha = (-0.3 * torch.rand(B, T, H, d, device=dev, generator=g)).to(bf)
    beta = torch.sigmoid(torch.randn(B, T, H, device=dev, generator=g)).to(bf)
    do = torch.randn(B, T, H, d, device=dev, generator=g).to(bf)
    out, dq, dk, dv, da = (torch.empty_like(v) for _ in range(5))
    db = torch.empty_like(beta)
    wsb = nat.query("edf_kda_scan_backward_workspace_bytes", B, T, H, d, 1)
    ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
    recb = nat.query("edf_kda_scan_context_bytes", B, T, H, d, 1)
    rec = torch.empty(recb, dtype=torch.uint8, device=dev)
    P = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)

    # the training pair the autograd path runs: a forward that keeps the 16-step states in the
    # same pass, and the backward from them
    def fwd():
        nat.call("edf_fused_kda_scan_with_context", stream, P(q), P(k), P(v), P(alpha), P(beta), P(out), P(rec),
                 recb, B, T, H, d, 1)

    def bwd():
        nat.call("edf_fused_kda_scan_backward_saved", stream, P(q), P(k), P(v), P(alpha), P(beta), P(do), P(dq),
                 P(dk), P(dv), P(da), P(db), P(rec), recb, P(ws), wsb, B, T, H, d, 1)

    fwd_ms, bwd_ms = _time_pair(torch, steps, warmup, fwd, bwd)
    return dict(fwd_ms=fwd_ms, bwd_ms=bwd_ms, tokens_per_s=B * T / (fwd_ms + bwd_ms) * 1e3,
                shape=dict(B=B, T=T, H=H, d=d))


def bench_delta_product(torch, steps, warmup, B=8, T=2048, NH=2, H=8, d=128):
    """DeltaProduct (n_h = 2 sub-steps per token, raw keys normalized in the kernel), bf16:
    fwd and bwd time per call and tokens/s (B T per call)."""
    from edifice_amd import _native as nat

    g = torch.Generator(device="cuda").manual_seed(3002)
    dev, bf = "cuda", torch.bfloat16
    q = torch.randn(B, T, H, d, device=dev, generator=g).to(bf)
    k = torch.randn(B, T, NH, H, d, device=dev, generator=g).to(bf)
    v = torch.randn(B, T, NH, H, d, device=dev, generator=g).to(bf)
    beta = torch.sigmoid(torch.randn(B, T, NH, H, device=dev, generator=g)).to(bf)
    do = torch.randn(B, T, H, d, device=dev, generator=g).to(bf)
    out, dq = torch.empty_like(q), torch.empty_like(q)
    dk, dv, db = torch.empty_like(k), torch.empty_like(v), torch.empty_like(beta)
    recb = nat.query("edf_delta_product_context_bytes", B, T, NH, H, d, 1)
    wsb = nat.query("edf_delta_product_backward_workspace_bytes", B, T, NH, H, d, 1)
    rec = torch.empty(recb, dtype=torch.uint8, device=dev)
    ws2 = torch.empty(wsb, dtype=torch.uint8, device=dev)
    P = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)

    # the training pair the autograd path runs: a forward that keeps the backward's context
    # (row-block partials, 16-sub-step states) in the same pass, and the backward from it
    def fwd():
        nat.call("edf_fused_delta_product_scan_with_context", stream, P(q), P(k), P(v), P(beta), P(out), P(rec),
                 recb, B, T, NH, H, d, 1)

    def bwd():
        nat.call("edf_fused_delta_product_scan_backward_saved", stream, P(q), P(k), P(v), P(beta), P(do), P(dq),
                 P(dk), P(dv), P(db), P(rec), recb, P(ws2), wsb, B, T, NH, H, d, 1)

    fwd_ms, bwd_ms = _time_pair(torch, steps, warmup, fwd, bwd)
    return dict(fwd_ms=fwd_ms, bwd_ms=bwd_ms, tokens_per_s=B * T / (fwd_ms + bwd_ms) * 1e3,
                shape=dict(B=B, T=T, n_h=NH, H=H, d=d))


def bench_rla(torch, steps, warmup, variant, B=8, T=2048, H=8, d=128):
    """RLA (variant 0) / RDN (variant 1), bf16, clip 1.0: fwd and bwd time per call and
    tokens/s (B T per call)."""
    from edifice_amd import _native as nat

    g = torch.Generator(device="cuda").manual_seed(3003)
    dev, bf = "cuda", torch.bfloat16
    l2n = lambda x: x / torch.sqrt((x * x).sum(-1, keepdim=True) + 1e-6)  # noqa: E731
    q = torch.randn(B, T, H, d, device=dev, generator=g).to(bf)
    k = l2n(torch.randn(B, T, H, d, device=dev, generator=g)).to(bf)
    v = torch.randn(B, T, H, d, device=dev, generator=g).to(bf)
    alpha, beta, gamma = ((0.3 + 0.65 * torch.rand(B, T, H, device=dev, generator=g)).to(bf) for _ in range(3))
    do = torch.randn(B, T, H, d, device=dev, generator=g).to(bf)
    out, dq, dk, dv = (torch.empty_like(q) for _ in range(4))
    da, db, dg = (torch.empty_like(alpha) for _ in range(3))
    wsb = nat.query("edf_rla_scan_backward_workspace_bytes", B, T, H, d, 1)
    ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
    recb = nat.query("edf_rla_scan_context_bytes", B, T, H, d, 1)
    rec = torch.empty(recb, dtype=torch.uint8, device=dev)
    P = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)

    # the training pair the autograd path runs: a forward that keeps both states every 8 steps
    # in the same pass, and the backward from them
    def fwd():
        nat.call("edf_fused_rla_scan_with_context", stream, P(q), P(k), P(v), P(alpha), P(beta), P(gamma), P(out),
                 P(rec), recb, B, T, H, d, variant, 1.0, 1)

    def bwd():
        nat.call("edf_fused_rla_scan_backward_saved", stream, P(q), P(k), P(v), P(alpha), P(beta), P(gamma), P(do),
                 P(dq), P(dk), P(dv), P(da), P(db), P(dg), P(rec), recb, P(ws), wsb, B, T, H, d, variant, 1.0, 1)

    fwd_ms, bwd_ms = _time_pair(torch, steps, warmup, fwd, bwd)
    return dict(fwd_ms=fwd_ms, bwd_ms=bwd_ms, tokens_per_s=B * T / (fwd_ms + bwd_ms) * 1e3,
                shape=dict(B=B, T=T, H=H, d=d))


def bench_ttt(torch, steps, warmup, B=8, T=2048, D=64):
    """TTT-Linear (inner model D x D per batch element), bf16: fwd and bwd time per call and
    tokens/s (B T per call).  One workgroup per batch element: the LayerNorm couples all rows
    of W at every step."""
    from edifice_amd import _native as nat

    g = torch.Generator(device="cuda").manual_seed(3004)
    dev, bf = "cuda", torch.bfloat16
    q = torch.randn(B, T, D, device=dev, generator=g).to(bf)
    k = (torch.randn(B, T, D, device=dev, generator=g) / D ** 0.5).to(bf)
    v = torch.randn(B, T, D, device=dev, generator=g).to(bf)
    eta = (torch.sigmoid(torch.randn(B, T, D, device=dev, generator=g)) / D).to(bf)
    w0 = (torch.randn(B, D, D, device=dev, generator=g) / D ** 0.5).to(bf)
    lg, lb = torch.ones(D, device=dev, dtype=bf), torch.zeros(D, device=dev, dtype=bf)
    do = torch.randn(B, T, D, device=dev, generator=g).to(bf)
    out = torch.empty_like(q)
    grads = [torch.empty_like(t) for t in (q, k, v, eta, w0, lg, lb)]
    wsb = nat.query("edf_ttt_scan_backward_workspace_bytes", B, T, D, 1)
    ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
    recb = nat.query("edf_ttt_scan_context_bytes", B, T, D, 1)
    rec = torch.empty(recb, dtype=torch.uint8, device=dev)
    P = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)

    # the training pair the autograd path runs: a forward that records the backward's context
    # in the same pass, and the backward from that context
    def fwd():
        nat.call("edf_fused_ttt_scan_with_context", stream, P(q), P(k), P(v), P(eta), P(w0), P(lg), P(lb), P(out),
                 P(rec), recb, B, T, D, 1)

    def bwd():
        nat.call("edf_fused_ttt_scan_backward_saved", stream, P(q), P(k), P(v), P(eta), P(w0), P(lg), P(lb), P(do),
                 *(P(t) for t in grads), P(rec), recb, P(ws), wsb, B, T, D, 1)

    fwd_ms, bwd_ms = _time_pair(torch, steps, warmup, fwd, bwd)
    return dict(fwd_ms=fwd_ms, bwd_ms=bwd_ms, tokens_per_s=B * T / (fwd_ms + bwd_ms) * 1e3,
                shape=dict(B=B, T=T, D=D))


def bench_rnn_block(torch, steps, warmup, kind, dtype, B=8, T=2048, H=256, L=4):
    """Multi-layer LSTM / GRU block (inference), random weights: ms per call and tokens/s."""
    from edifice_amd import _native as nat

    g = torch.Generator(device="cuda").manual_seed(3005)
    G = 4 if kind == "lstm" else 3
    sc = H ** -0.5
    per = []
    for _ in range(L):
        per += [sc * torch.randn(H * G * H, device="cuda", generator=g), 0.1 * torch.randn(G * H, device="cuda", generator=g),
                sc * torch.randn(H * G * H, device="cuda", generator=g), torch.ones(H, device="cuda"),
                torch.zeros(H, device="cuda")]
    w = torch.cat(per).to(dtype)
    x = torch.randn(B, T, H, device="cuda", generator=g).to(dtype)
    h0 = torch.zeros(B, L, H, device="cuda", dtype=dtype)
    out = torch.empty_like(x)
    flag = 1 if dtype == torch.bfloat16 else 0
    wsb = nat.query(f"edf_{kind}_block_workspace_bytes", B, T, H, L, flag)
    ws = torch.empty(wsb, dtype=torch.uint8, device="cuda")
    P = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)

    def run():
        if kind == "lstm":
            nat.call("edf_fused_lstm_block_scan", stream, P(x), P(w), P(h0), P(h0), P(out), P(ws), wsb, B, T, H, L, flag)
        else:
            nat.call("edf_fused_gru_block_scan", stream, P(x), P(w), P(h0), P(out), P(ws), wsb, B, T, H, L, flag)

    ms = median_ms(torch, run, steps, warmup)
    return dict(layers=L, dtype=str(dtype).replace("torch.", ""), ms=ms, tokens_per_s=B * T / ms * 1e3,
                shape=dict(B=B, T=T, H=H))


GEMM_SOLUTIONS = os.path.join(os.path.dirname(os.path.abspath(__file__)), "edifice_amd", "gemm_solutions_mi355x.csv")


def use_tuned_gemms(torch):
    """The config-5 model's torch GEMMs take the hipBLASLt / rocBLAS solutions that torch's
    TunableOp measured fastest per shape on an MI355X (``edifice_amd/gemm_solutions_mi355x.csv``,
    read before the model is built; no tuning runs here).  TunableOp checks the file's torch,
    HIP, hipBLASLt, rocBLAS and architecture lines and ignores a file that does not match, and
    shapes not in the file keep the library's default choice.  Returns what the GEMMs use."""
    tun = getattr(torch.cuda, "tunable", None)
    if tun is None or not os.path.exists(GEMM_SOLUTIONS):
        return "library default"
    tun.enable(True)
    tun.tuning_enable(False)
    tun.record_untuned_enable(False)
    tun.set_filename(os.path.join(tempfile.gettempdir(), "edifice_tunableop_unused%d.csv"), True)
    if not tun.read_file(GEMM_SOLUTIONS):
        tun.enable(False)
        return "library default (solution file not accepted)"
    return "TunableOp file edifice_amd/gemm_solutions_mi355x.csv"


def bench_hybrid(torch, steps, warmup, B=8, T=2048, vocab=32000, embed=1024):
    """Config 5: 4 Mamba + 2 DeltaNet + 2 causal-attention blocks, embed 1024, bf16 weights and
    activations, random init, synthetic token ids uniform over the vocabulary; one step = the
    forward and backward of the next-token loss (no optimizer step, as the metric states)."""
    from edifice_amd import blocks

    gemm = use_tuned_gemms(torch)
    torch.manual_seed(5000)
    model = blocks.HybridDecoder(vocab, embed).to("cuda", torch.bfloat16)
    g = torch.Generator(device="cuda").manual_seed(5001)
    tokens = torch.randint(0, vocab, (B, T + 1), device="cuda", generator=g)

    def step():
        for p in model.parameters():
            p.grad = None
        model.loss(tokens).backward()

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
    ev[0].record()
    for i in range(steps):
        step()
        ev[i + 1].record()
    torch.cuda.synchronize()
    per_step = [ev[i].elapsed_time(ev[i + 1]) for i in range(steps)]
    ms = float(np.median(per_step))
    torch.cuda.tunable.enable(False)
    return dict(step_ms=ms, tokens_per_s=B * T / ms * 1e3, steps=steps, warmup=warmup, gemm_solutions=gemm,
                step_ms_min=float(min(per_step)), step_ms_max=float(max(per_step)),
                shape=dict(batch=B, seq=T, vocab=vocab, embed=embed, layers="4 mamba + 2 delta_net + 2 attention"))


def cpu_model():
    """The host CPU's model name (the line lscpu prints as "Model name")."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _cpu_median(fn, warmup=2, reps=5):
    """Median wall time (s) of ``fn`` over ``reps`` runs after ``warmup`` untimed ones."""
    for _ in range(warmup):
        fn()
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return float(np.median(times))


def _cpu_lib():
    from oracle import cbuild

    lib = cbuild.lib()
    lib.cref_threads.restype = ctypes.c_int
    return lib


def _cpu_entry(value, unit, lib, sample, **extra):
    return dict(value=value, unit=unit, cores=int(lib.cref_threads()), kind="port", cpu_model=cpu_model(),
                host_cpus=os.cpu_count(), sample=sample, **extra)


CP = lambda a: a.ctypes.data_as(ctypes.c_void_p)  # noqa: E731


def _ss_cpu_inputs(rng, B, T, D, N):
    f32 = np.float32
    x = rng.normal(size=(B, T, D)).astype(f32)
    dt = np.log1p(np.exp(rng.normal(size=(B, T, D)) - 4)).astype(f32)
    A = (-np.exp(rng.uniform(0, np.log(16), size=(D, N)))).astype(f32)
    Bm, Cm = (rng.normal(size=(B, T, N)).astype(f32) for _ in range(2))
    Dv = rng.normal(size=D).astype(f32)
    z, dy = (rng.normal(size=(B, T, D)).astype(f32) for _ in range(2))
    return x, dt, A, Bm, Cm, Dv, z, dy


def _ss_cpu_step(lib, ins, B, T, D, N):
    x, dt, A, Bm, Cm, Dv, z, dy = ins
    out, dx, ddt, dz = (np.empty_like(x) for _ in range(4))
    dA, dB, dC, dD = np.zeros_like(A), np.zeros_like(Bm), np.zeros_like(Cm), np.zeros_like(Dv)

    def step():
        lib.cref_selective_scan_fwd(CP(x), CP(dt), CP(A), CP(Bm), CP(Cm), CP(Dv), CP(z), CP(out), B, T, D, N)
        lib.cref_selective_scan_bwd(CP(x), CP(dt), CP(A), CP(Bm), CP(Cm), CP(Dv), CP(z), CP(dy), CP(dx), CP(ddt),
                                    CP(dA), CP(dB), CP(dC), CP(dD), CP(dz), B, T, D, N)
    return step


def cpu_baseline_selective_scan(B=8, T=2048, D=1536, N=16):
    """Time the C restatement (oracle/cref.c, OpenMP f32) on the config-2 selective-scan
    workload (the full configuration, a fraction of a second per fwd+bwd step on the host's
    cores); returns GB/s under the same byte accounting as the GPU figure."""
    lib = _cpu_lib()
    t = _cpu_median(_ss_cpu_step(lib, _ss_cpu_inputs(np.random.default_rng(7), B, T, D, N), B, T, D, N))
    fb, bb = ss_bytes(B, T, D, N)
    return _cpu_entry((fb + bb) / t / 1e9, "GB/s", lib,
                      f"C restatement (Nx unavailable), selective scan fwd+bwd f32, B={B} T={T} D={D} N={N} "
                      f"(the full config-2 workload), median of 5 after 2 warm-ups, {t:.3f} s per step",
                      s_per_step=t)


def cpu_baseline_mingru(B=4, T=60, H=256):
    """Config 1 (MinGRU f32 4x60x256, fwd+bwd) on the C restatement, GB/s under the GPU row's
    byte accounting; the step is microseconds long, so each timed run is 200 steps."""
    lib = _cpu_lib()
    rng = np.random.default_rng(8)
    f32 = np.float32
    z = (1 / (1 + np.exp(-rng.normal(size=(B, T, H))))).astype(f32)
    c, dy = (rng.normal(size=(B, T, H)).astype(f32) for _ in range(2))
    out, dz, dc = (np.empty_like(z) for _ in range(3))
    nul = ctypes.c_void_p(None)

    def run():
        for _ in range(200):
            lib.cref_mingru_fwd(CP(z), CP(c), nul, CP(out), B, T, H)
            lib.cref_mingru_bwd(CP(z), CP(c), nul, CP(out), CP(dy), CP(dz), CP(dc), nul, B, T, H)
    t = _cpu_median(run) / 200
    return _cpu_entry(9 * B * T * H * 4 / t / 1e9, "GB/s", lib,
                      f"C restatement, MinGRU fwd+bwd f32 B={B} T={T} H={H} (the full config-1 workload), median of "
                      f"5 runs of 200 steps after 2 warm-ups, {t * 1e6:.1f} us per step", s_per_step=t)


def _delta_cpu(lib, B, T, H, d, per_head_beta, gated, seed):
    rng = np.random.default_rng(seed)
    f32 = np.float32
    l2 = lambda a: (a / np.sqrt((a * a).sum(-1, keepdims=True) + 1e-6)).astype(f32)  # noqa: E731
    q, k = l2(rng.normal(size=(B, T, H, d))), l2(rng.normal(size=(B, T, H, d)))
    v, do = (rng.normal(size=(B, T, H, d)).astype(f32) for _ in range(2))
    beta = (1 / (1 + np.exp(-rng.normal(size=(B, T, H) if per_head_beta else (B, T, H, d))))).astype(f32)
    alpha = np.exp(-np.log1p(np.exp(rng.normal(size=(B, T, H))))).astype(f32) if gated else None
    out, dq, dk, dv = (np.empty_like(q) for _ in range(4))
    db = np.empty_like(beta)
    da = np.empty((B, T, H), f32)
    nul = ctypes.c_void_p(None)
    ap, dap = (CP(alpha), CP(da)) if gated else (nul, nul)

    def step():
        lib.cref_delta_rule_fwd(CP(q), CP(k), CP(v), CP(beta), ap, CP(out), B, T, H, d, int(per_head_beta))
        lib.cref_delta_rule_bwd(CP(q), CP(k), CP(v), CP(beta), ap, CP(do), CP(dq), CP(dk), CP(dv), CP(db), dap,
                                B, T, H, d, int(per_head_beta))
    return step


def cpu_baseline_delta_rule(B=4, H=16, T=4096, d=128, C=64):
    """Config 3 on the C restatement (recurrent form, f32, states checkpointed every 64 steps
    for the backward), the full workload; TFLOP/s under the GPU row's chunked-form flop count."""
    lib = _cpu_lib()
    t = _cpu_median(_delta_cpu(lib, B, T, H, d, True, True, 9), warmup=2, reps=5)
    flops = 3 * 2 * (5 * C * d + 3 * d * d) * B * H * T
    return _cpu_entry(flops / t / 1e12, "TFLOP/s", lib,
                      f"C restatement, gated delta rule fwd+bwd f32 (recurrent form), B={B} H={H} T={T} d={d} (the "
                      f"full config-3 workload), median of 5 after 2 warm-ups, {t:.3f} s per step", s_per_step=t)


def _attn_cpu(lib, BH, T, d, causal, seed):
    rng = np.random.default_rng(seed)
    f32 = np.float32
    q, k, v, do = (rng.normal(scale=d ** -0.25, size=(BH, T, d)).astype(f32) for _ in range(4))
    out, dq, dk, dv = (np.empty_like(q) for _ in range(4))
    lse = np.empty((BH, T), f32)

    def step():
        lib.cref_attention_fwd(CP(q), CP(k), CP(v), CP(out), CP(lse), BH, T, d, int(causal))
        lib.cref_attention_bwd(CP(q), CP(k), CP(v), CP(out), CP(do), CP(lse), CP(dq), CP(dk), CP(dv), BH, T, d,
                               int(causal))
    return step


def cpu_baseline_attention(B=4, H=32, T=4096, d=128, sample_heads=16):
    """Config 4 on the C restatement (causal softmax attention, f32) over a bounded sample of
    the (b, h) heads, which are independent and equal in cost; TFLOP/s under the GPU row's flop
    count, and the full-step time scaled from the sample."""
    lib = _cpu_lib()
    t = _cpu_median(_attn_cpu(lib, sample_heads, T, d, True, 10), warmup=2, reps=5)
    flops = 3.5 * 4 * sample_heads * T * T * d / 2
    full = t * B * H / sample_heads
    return _cpu_entry(flops / t / 1e12, "TFLOP/s", lib,
                      f"C restatement, causal attention fwd+bwd f32 on {sample_heads} of the {B * H} heads "
                      f"(T={T} d={d}), median of 5 after 2 warm-ups, {t:.3f} s; full step scaled: {full:.2f} s",
                      s_per_step=full)


def cpu_baseline_hybrid(B=8, T=2048, embed=1024, sample_rows=1):
    """Config 5's fused-op mix on the C restatement over a sample of its batch rows (rows are
    independent and equal in cost): per row 4 Mamba selective scans (d_inner 2048, N 16), 2
    DeltaNet rules (8 heads x 128, per-element beta) and 2 causal attentions (8 heads x 128),
    forward and backward.  The dense layers, norms and loss are not timed (no CPU path here
    runs them in the reference's form); tokens/s is the whole batch over the scaled op time."""
    lib = _cpu_lib()
    inner, N, H, d = 2 * embed, 16, 8, embed // 8
    ss = _ss_cpu_step(lib, _ss_cpu_inputs(np.random.default_rng(11), sample_rows, T, inner, N), sample_rows, T,
                      inner, N)
    dr = _delta_cpu(lib, sample_rows, T, H, d, False, False, 12)
    at = _attn_cpu(lib, sample_rows * H, T, d, True, 13)

    def step():
        for _ in range(4):
            ss()
        for _ in range(2):
            dr()
            at()
    t = _cpu_median(step, warmup=2, reps=5) * B / sample_rows
    return _cpu_entry(B * T / t, "tokens/s", lib,
                      f"C restatement of config 5's fused ops only (4 selective scans, 2 delta rules, 2 causal "
                      f"attentions, fwd+bwd, f32) on {sample_rows} of {B} batch rows (T={T}), median of 5 after 1 "
                      f"warm-up, scaled to the batch: {t:.2f} s per step; dense layers excluded", s_per_step=t)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--only", default="")
    ap.add_argument("--flush", choices=("read", "write", "none"), default="read",
                    help="cache eviction before each timed scan-row run (default: read 512 MiB)")
    ap.add_argument("--copy-probe", action="store_true",
                    help="also run a plain 256 MiB device copy (scale reference for rocprof FETCH/WRITE_SIZE)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (see DESIGN.md, 'How it would shard')",
              file=sys.stderr)
        sys.exit(2)
    import torch

    Flush.mode = args.flush
    only = set(filter(None, args.only.split(",")))
    want = (lambda k: not only or k in only)  # noqa: E731
    configs = {}
    if want("mingru"):
        configs["hbm_ceiling_stream_probe"] = bench_hbm_ceiling(torch, args.steps, args.warmup)
        configs["c1_mingru_f32_4x60x256"] = bench_mingru(torch, args.steps, args.warmup, 4, 60, 256, torch.float32)
        for dt in (torch.bfloat16, torch.float32):
            key = f"mingru_bw_{str(dt).replace('torch.', '')}_8x2048x1536"
            configs[key] = bench_mingru(torch, args.steps, args.warmup, 8, 2048, 1536, dt)
    if want("block"):
        for kind, dt in (("mingru", torch.float32), ("mingru", torch.bfloat16), ("minlstm", torch.float32),
                         ("linear", torch.float32)):
            key = f"{kind}_block_{str(dt).replace('torch.', '')}_8x2048x256_L4"
            configs[key] = bench_block(torch, args.steps, args.warmup, 8, 2048, 256, 4, dt, kind)
        for kind in ("lstm", "gru"):
            configs[f"{kind}_block_float32_8x2048x256_L4"] = bench_rnn_block(
                torch, min(args.steps, 5), min(args.warmup, 2), kind, torch.float32)
    if want("linear"):
        for dt in (torch.bfloat16, torch.float32):
            key = f"linear_scan_{str(dt).replace('torch.', '')}_8x2048x1536"
            configs[key] = bench_linear_scan(torch, args.steps, args.warmup, 8, 2048, 1536, dt)
    ss = bench_selective_scan(torch, args.steps, args.warmup)
    configs["c2_selective_scan"] = ss
    if want("delta") or want("c3"):
        configs["c3_gated_delta_rule"] = bench_delta_rule(torch, args.steps, args.warmup)
    if want("delta"):
        configs["kda_8x2048x8x128"] = bench_kda(torch, args.steps, args.warmup)
        configs["delta_product_8x2048x2x8x128"] = bench_delta_product(torch, args.steps, args.warmup)
        configs["rla_8x2048x8x128"] = bench_rla(torch, args.steps, args.warmup, 0)
        configs["rdn_8x2048x8x128"] = bench_rla(torch, args.steps, args.warmup, 1)
        configs["ttt_8x2048x64"] = bench_ttt(torch, args.steps, args.warmup)
    if want("flash") or want("c4"):
        configs["c4_flash_attention"] = bench_flash(torch, args.steps, args.warmup)
    if want("flash"):
        configs["flash_attention_noncausal_4x32x2048x128"] = bench_flash(torch, args.steps, args.warmup, T=2048,
                                                                         causal=False)
        configs["fox_attention_4x32x4096x128"] = bench_fox(torch, args.steps, args.warmup)
    if want("hybrid"):
        configs["c5_hybrid_decoder"] = bench_hybrid(torch, max(5, args.steps // 4), 2)
    bwd_dom = ss["bwd_ms"] >= ss["fwd_ms"]
    dominant = ("edf_fused_selective_scan_backward (ss_bwd_kernel + dB/dC, dA/dD reductions)" if bwd_dom
                else "edf_fused_selective_scan (ss_fwd_kernel)")
    dom_ms = max(ss["bwd_ms"], ss["fwd_ms"])
    dom_bytes = ss["bwd_bytes"] if bwd_dom else ss["fwd_bytes"]
    achieved = dom_bytes / dom_ms / 1e6
    traffic = profiled_traffic(["ss_bwd_kernel", "ss_reduce_bc_kernel", "ss_reduce_ad_kernel"] if bwd_dom
                               else ["ss_fwd_kernel"])
    line = {
        "metric": "scan HBM GB/s (% of peak); delta-rule & flash-attn fwd+bwd TFLOP/s (% MFMA)",
        "value": round(ss["step_gbs"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ss["step_ms"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16 io / f32 math",
        "data": "synthetic (config-2 distributions, seeded torch generator)",
        "config": {"workload": "config 2: Mamba selective scan fwd+bwd, B=8 T=2048 D=1536 N=16, u/dt/z bf16, "
                               "A/B/C/D f32, D skip + silu(z) gate", "batch": 8, "seq_len": 2048, "d_inner": 1536,
                   "d_state": 16},
        "roofline": {"bound": "hbm", "kernel": dominant, "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic},
        # the bound this kernel actually meets: its VALU issue slots per element (SS_VALU_SLOTS)
        # over 8 x 2048 x 1536 x 16 elements, per second, against the VALU peak
        "valu_roofline": {"kernel": dominant, "slots_per_element": SS_VALU_SLOTS[1 if bwd_dom else 0],
                          "achieved": round(SS_VALU_SLOTS[1 if bwd_dom else 0] * 8 * 2048 * 1536 * 16 / dom_ms / 1e9, 2),
                          "peak": round(VALU_PEAK_TSLOTS, 2), "unit": "T slots/s",
                          "frac": round(SS_VALU_SLOTS[1 if bwd_dom else 0] * 8 * 2048 * 1536 * 16 / dom_ms / 1e9
                                        / VALU_PEAK_TSLOTS, 4)},
        "configs": configs,
    }
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline_selective_scan()
        # the same C restatement on every other config (CPU time and speed-up per config)
        cpu_rows = {"c1_mingru_f32_4x60x256": (cpu_baseline_mingru, "fwd_us", "bwd_us", 1e-6),
                    "c3_gated_delta_rule": (cpu_baseline_delta_rule, "fwd_ms", "bwd_ms", 1e-3),
                    "c4_flash_attention": (cpu_baseline_attention, "fwd_ms", "bwd_ms", 1e-3),
                    "c5_hybrid_decoder": (cpu_baseline_hybrid, "step_ms", None, 1e-3)}
        for key, (fn, f_key, b_key, unit_s) in cpu_rows.items():
            if key in configs:
                cb = fn()
                row = configs[key]
                gpu_s = (row[f_key] + (row[b_key] if b_key else 0.0)) * unit_s
                cb["speedup_gpu_over_cpu"] = round(cb["s_per_step"] / gpu_s, 1)
                row["cpu_baseline"] = cb
    if args.copy_probe:
        src = torch.ones(64 * 2 ** 20, dtype=torch.float32, device="cuda")  # 256 MiB
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
    print(json.dumps(line))


if __name__ == "__main__":
    main()
