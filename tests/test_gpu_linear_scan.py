"""GPU parity: MinGRU / MinLSTM / generic linear scans (HIP, through the C ABI) vs the CPU oracle."""
import ctypes

import numpy as np
import pytest
import torch

from oracle import scans
from tests.conftest import assert_close
from tests.gpu_util import TOL, announce, host, rounded, to_dev

pytestmark = pytest.mark.gpu

# odd hidden sizes take the one-channel-per-lane bf16 kernels, even ones the channel-pair kernels
SHAPES = [(1, 1, 2), (4, 60, 256), (2, 37, 100), (3, 129, 64), (2, 700, 130), (1, 2048, 96), (2, 45, 77)]
DTYPES = [torch.float32, torch.bfloat16]


def _sig(x):
    return 1 / (1 + np.exp(-x))


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("dtype", DTYPES)
def test_mingru_logits_fwd_bwd(shape, dtype, rng):
    from edifice_amd import fused_scan as fs
    announce("mingru_logits", shape=shape, dtype=dtype)
    g = rng.normal(size=shape)
    c = rng.normal(size=shape)
    dy = rng.normal(size=shape)
    tg, tc = to_dev(g, dtype).requires_grad_(), to_dev(c, dtype).requires_grad_()
    out = fs.mingru(tg, tc)
    out.backward(to_dev(dy, dtype))
    gr, cr, dyr = rounded(g, dtype), rounded(c, dtype), rounded(dy, dtype)
    assert_close(host(out), scans.min_gru_scan(gr, cr), TOL[dtype], "h")
    dg, dc = scans.min_gru_scan_backward(gr, cr, dyr)
    assert_close(host(tg.grad), dg, TOL[dtype], "dgates")
    assert_close(host(tc.grad), dc, TOL[dtype], "dcand")


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("dtype", DTYPES)
def test_minlstm_logits_fwd_bwd(shape, dtype, rng):
    from edifice_amd import fused_scan as fs
    announce("minlstm_logits", shape=shape, dtype=dtype)
    fg, ig, c, dy = (rng.normal(size=shape) for _ in range(4))
    tf, ti, tc = (to_dev(a, dtype).requires_grad_() for a in (fg, ig, c))
    out = fs.minlstm(tf, ti, tc)
    out.backward(to_dev(dy, dtype))
    fr, ir, cr, dyr = (rounded(a, dtype) for a in (fg, ig, c, dy))
    f, i = _sig(fr), _sig(ir)
    fwd = scans.minlstm_scan(f, i, cr)
    assert_close(host(out), fwd, TOL[dtype], "c")
    df, di, dc, _ = scans.minlstm_scan_backward(f, i, cr, None, fwd, dyr)
    assert_close(host(tf.grad), df * f * (1 - f), TOL[dtype], "dforget")
    assert_close(host(ti.grad), di * i * (1 - i), TOL[dtype], "dinput")
    assert_close(host(tc.grad), dc, TOL[dtype], "dcand")


def _call(name, *args):
    from edifice_amd import _native as nat
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    ptrs = [ctypes.c_void_p(a.data_ptr()) if isinstance(a, torch.Tensor) else a for a in args]
    nat.call(name, stream, *ptrs)


@pytest.mark.parametrize("shape", [(4, 60, 256), (2, 33, 70), (2, 1100, 262)])
@pytest.mark.parametrize("dtype", DTYPES)
def test_reference_shaped_entry_points(shape, dtype, rng):
    """edf_fused_mingru_scan / _backward and the MinLSTM pair: post-sigmoid gates, explicit h0."""
    announce("nif_shaped", shape=shape, dtype=dtype)
    bsz, seq, hid = shape
    flag = 1 if dtype == torch.bfloat16 else 0
    z = rng.uniform(0.02, 0.98, size=shape)
    i = rng.uniform(0.02, 0.98, size=shape)
    c, dy = rng.normal(size=shape), rng.normal(size=shape)
    h0 = rng.normal(size=(bsz, hid))
    tz, ti, tc, tdy, th0 = (to_dev(a, dtype) for a in (z, i, c, dy, h0))
    zr, ir, cr, dyr, h0r = (rounded(a, dtype) for a in (z, i, c, dy, h0))
    tol = TOL[dtype]

    out = torch.empty_like(tz)
    _call("edf_fused_mingru_scan", tz, tc, th0, out, bsz, seq, hid, flag)
    fwd = scans.mingru_scan(zr, cr, h0r)
    assert_close(host(out), fwd, tol, "mingru h")
    gz, gc, gh = torch.empty_like(tz), torch.empty_like(tz), torch.empty_like(th0)
    _call("edf_fused_mingru_scan_backward", tz, tc, th0, out, tdy, gz, gc, gh, bsz, seq, hid, flag)
    ez, ec, eh = scans.mingru_scan_backward(zr, cr, h0r, host(out), dyr)
    assert_close(host(gz), ez, tol, "dz")
    assert_close(host(gc), ec, tol, "dcand")
    assert_close(host(gh), eh, tol, "dh0")

    out = torch.empty_like(tz)
    _call("edf_fused_minlstm_scan", tz, ti, tc, th0, out, bsz, seq, hid, flag)
    fwd = scans.minlstm_scan(zr, ir, cr, h0r)
    assert_close(host(out), fwd, tol, "minlstm c")
    gf, gi, gc, gh = (torch.empty_like(t) for t in (tz, tz, tz, th0))
    _call("edf_fused_minlstm_scan_backward", tz, ti, tc, th0, out, tdy, gf, gi, gc, gh, bsz, seq, hid, flag)
    ef, ei, ec, eh = scans.minlstm_scan_backward(zr, ir, cr, h0r, host(out), dyr)
    for a, e, n in ((gf, ef, "df"), (gi, ei, "di"), (gc, ec, "dcand"), (gh, eh, "dh0")):
        assert_close(host(a), e, tol, n)


def test_mingru_seq1_known_answer():
    """backward_kernels_test.exs:271-287 through the HIP entry points."""
    announce("mingru_known_answer")
    f32 = dict(dtype=torch.float32, device="cuda")
    z = torch.tensor([[[0.3, 0.7]]], **f32)
    c = torch.tensor([[[2.0, -1.0]]], **f32)
    h0 = torch.zeros(1, 2, **f32)
    out = torch.empty_like(z)
    _call("edf_fused_mingru_scan", z, c, h0, out, 1, 1, 2, 0)
    assert torch.allclose(out, torch.tensor([[[0.6, -0.7]]], **f32), atol=1e-6)
    gz, gc, gh = torch.empty_like(z), torch.empty_like(z), torch.empty_like(h0)
    _call("edf_fused_mingru_scan_backward", z, c, h0, out, torch.ones_like(z), gz, gc, gh, 1, 1, 2, 0)
    assert torch.allclose(gz.cpu(), torch.tensor([[[2.0, -1.0]]]), atol=1e-6)
    assert torch.allclose(gc.cpu(), torch.tensor([[[0.3, 0.7]]]), atol=1e-6)
    assert torch.allclose(gh.cpu(), torch.tensor([[0.7, 0.3]]), atol=1e-6)


@pytest.mark.parametrize("spin", [None, "0"])
@pytest.mark.parametrize("dtype", DTYPES)
def test_lookback_paths(dtype, spin, rng, monkeypatch):
    """Sequences of at least 512 steps run the look-back scans (parts of 128 steps forward, 64
    backward, each part's carry from the maps of the parts before / after it); with a poll
    limit of 0 a part whose neighbours' maps are not published at the first look folds them
    from their rows instead.  Every path against the oracle, and against the
    one-workgroup-per-tile kernels (EDF_LIN_LOOKBACK=0)."""
    from edifice_amd import fused_scan as fs
    if spin is not None:
        monkeypatch.setenv("EDF_LIN_LOOKBACK_SPIN", spin)
    shape = (3, 1100, 262)  # a partial last part and a partial last channel tile
    announce("lookback_paths", dtype=dtype, spin=spin)
    g, c, dy = (rng.normal(size=shape) for _ in range(3))
    a = rng.uniform(0.0, 1.0, size=shape)
    gr, cr, dyr, ar = (rounded(x, dtype) for x in (g, c, dy, a))

    def run():
        tg, tc, ta, tb = (to_dev(x, dtype).requires_grad_() for x in (g, c, a, c))
        h = fs.mingru(tg, tc)
        h.backward(to_dev(dy, dtype))
        lin = fs.linear_scan(ta, tb)
        lin.backward(to_dev(dy, dtype))
        return [host(x) for x in (h, tg.grad, tc.grad, lin, ta.grad, tb.grad)]

    got = run()
    tol = TOL[dtype]
    assert_close(got[0], scans.min_gru_scan(gr, cr), tol, "mingru h")
    eg, ec = scans.min_gru_scan_backward(gr, cr, dyr)
    assert_close(got[1], eg, tol, "mingru d gate")
    assert_close(got[2], ec, tol, "mingru d cand")
    lin = scans.linear_scan(ar, cr)
    assert_close(got[3], lin, tol, "linear h")
    da, db, _ = scans.linear_scan_backward(ar, None, rounded(got[3], dtype), dyr)
    assert_close(got[4], da, tol, "linear da")
    assert_close(got[5], db, tol, "linear db")
    monkeypatch.setenv("EDF_LIN_LOOKBACK", "0")
    for x, y, name in zip(got, run(), ("h", "d gate", "d cand", "linear h", "da", "db")):
        assert_close(x, y, tol, f"paths {name}")


@pytest.mark.parametrize("dtype", DTYPES)
def test_mingru_bandwidth_shape_full_size(dtype, rng):
    """The MinGRU bandwidth row (B=8, T=2048, H=1536) against the oracle at full size."""
    from edifice_amd import fused_scan as fs
    shape = (8, 2048, 1536)
    announce("mingru_full", shape=shape, dtype=dtype)
    g = rng.normal(size=shape).astype(np.float32)
    c = rng.normal(size=shape).astype(np.float32)
    tg, tc = to_dev(g, dtype).requires_grad_(), to_dev(c, dtype).requires_grad_()
    out = fs.mingru(tg, tc)
    gr, cr = rounded(g, dtype), rounded(c, dtype)
    assert_close(host(out), scans.min_gru_scan(gr, cr), TOL[dtype], "h full")
    # z -> 1 (large logits): h == cand exactly up to storage rounding
    big = torch.full_like(tg, 30.0)
    assert torch.allclose(fs.mingru(big, tc).float(), tc.float(), rtol=0, atol=1e-6)


# ---------------------------------------------------------------------------
# generic linear scan  h_t = a_t h_{t-1} + b_t
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("dtype", DTYPES)
def test_linear_scan_fwd_bwd(shape, dtype, rng):
    """FusedScan.linear_scan/2 with its custom_grad backward (h0 = 0)."""
    from edifice_amd import fused_scan as fs
    announce("linear_scan", shape=shape, dtype=dtype)
    a = rng.uniform(-0.99, 0.99, size=shape)
    b, dy = rng.normal(size=shape), rng.normal(size=shape)
    ta, tb = to_dev(a, dtype).requires_grad_(), to_dev(b, dtype).requires_grad_()
    out = fs.linear_scan(ta, tb)
    out.backward(to_dev(dy, dtype))
    ar, br, dyr = rounded(a, dtype), rounded(b, dtype), rounded(dy, dtype)
    fwd = scans.linear_scan(ar, br)
    assert_close(host(out), fwd, TOL[dtype], "h")
    da, db, _ = scans.linear_scan_backward(ar, None, rounded(host(out), dtype), dyr)
    assert_close(host(ta.grad), da, TOL[dtype], "da")
    assert_close(host(tb.grad), db, TOL[dtype], "db")


@pytest.mark.parametrize("shape", [(4, 60, 256), (2, 33, 70), (3, 50, 31)])
@pytest.mark.parametrize("dtype", DTYPES)
def test_linear_scan_reference_shaped_entry_points(shape, dtype, rng):
    """edf_fused_linear_scan / _backward with an explicit h0 (and with h0 = NULL)."""
    announce("linear_nif_shaped", shape=shape, dtype=dtype)
    bsz, seq, hid = shape
    flag = 1 if dtype == torch.bfloat16 else 0
    a = rng.uniform(-1.0, 1.0, size=shape)
    b, dy = rng.normal(size=shape), rng.normal(size=shape)
    h0 = rng.normal(size=(bsz, hid))
    ta, tb, tdy, th0 = (to_dev(x, dtype) for x in (a, b, dy, h0))
    ar, br, dyr, h0r = (rounded(x, dtype) for x in (a, b, dy, h0))
    tol = TOL[dtype]
    for with_h0 in (True, False):
        out = torch.empty_like(ta)
        _call("edf_fused_linear_scan", ta, tb, th0 if with_h0 else None, out, bsz, seq, hid, flag)
        assert_close(host(out), scans.linear_scan(ar, br, h0r if with_h0 else None), tol, "h")
        ga, gb, gh = torch.empty_like(ta), torch.empty_like(ta), torch.empty_like(th0)
        _call("edf_fused_linear_scan_backward", ta, th0 if with_h0 else None, out, tdy, ga, gb, gh, bsz, seq, hid,
              flag)
        ea, eb, eh = scans.linear_scan_backward(ar, h0r if with_h0 else None, rounded(host(out), dtype), dyr)
        for x, e, n in ((ga, ea, "da"), (gb, eb, "db"), (gh, eh, "dh0")):
            assert_close(host(x), e, tol, n)


def test_linear_scan_seq1_known_answer():
    """backward_kernels_test.exs:76-95 through the HIP entry points: a = 0.5, b = 1."""
    announce("linear_known_answer")
    f32 = dict(dtype=torch.float32, device="cuda")
    a, b, h0 = torch.full((1, 1, 1), 0.5, **f32), torch.ones(1, 1, 1, **f32), torch.zeros(1, 1, **f32)
    out = torch.empty_like(a)
    _call("edf_fused_linear_scan", a, b, h0, out, 1, 1, 1, 0)
    assert out.item() == 1.0
    ga, gb, gh = torch.empty_like(a), torch.empty_like(a), torch.empty_like(h0)
    _call("edf_fused_linear_scan_backward", a, h0, out, torch.ones_like(a), ga, gb, gh, 1, 1, 1, 0)
    assert (ga.item(), gb.item(), gh.item()) == (0.0, 1.0, 0.5)


@pytest.mark.parametrize("dtype", DTYPES)
def test_linear_scan_full_size(dtype, rng):
    """B=8, T=2048, H=1536 against the oracle, plus the a = 1 (cumulative sum) and a = 0 cases."""
    from edifice_amd import fused_scan as fs
    shape = (8, 2048, 1536)
    announce("linear_full", shape=shape, dtype=dtype)
    a = rng.uniform(0.0, 1.0, size=shape).astype(np.float32)
    b = rng.normal(size=shape).astype(np.float32)
    ta, tb = to_dev(a, dtype), to_dev(b, dtype)
    out = fs.linear_scan(ta, tb)
    assert_close(host(out), scans.linear_scan(rounded(a, dtype), rounded(b, dtype)), TOL[dtype], "h full")
    assert torch.equal(fs.linear_scan(torch.zeros_like(ta), tb), tb)
    cs = fs.linear_scan(torch.ones_like(ta), tb).float()
    ref = torch.cumsum(tb.float(), dim=1)
    assert ((cs - ref).abs().max() / ref.abs().max()).item() < (1e-5 if dtype == torch.float32 else 2e-2)


# ---------------------------------------------------------------------------
# multi-layer MinGRU block (inference)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("bsz,seq,hid,layers", [(1, 5, 8, 1), (2, 37, 64, 2), (3, 130, 100, 3), (2, 64, 256, 2),
                                                 (1, 33, 77, 4)])
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("kind", ["mingru", "minlstm", "linear"])
def test_block(kind, bsz, seq, hid, layers, dtype, rng):
    """FusedScan.{mingru,minlstm,linear}_block/4 against the layer-parallel oracle (itself
    pinned to the per-timestep walk of the reference kernels)."""
    from edifice_amd import fused_scan as fs
    announce(f"{kind}_block", shape=(bsz, seq, hid), layers=layers, dtype=dtype)
    nproj = scans.BLOCK_PROJECTIONS[kind]
    x = rng.normal(size=(bsz, seq, hid))
    w = rng.normal(scale=hid ** -0.5, size=layers * (nproj * (hid * hid + hid) + 2 * hid))
    if kind == "linear":  # keep |a| < 1 so the recurrence stays bounded: a = n W_a + b_a, b_a = 0.5
        wl = w.reshape(layers, -1)
        wl[:, :hid * hid] *= 0.1
        wl[:, hid * hid:hid * hid + hid] = 0.5
        w = wl.reshape(-1)
    h0 = rng.normal(scale=0.5, size=(bsz, layers, hid))
    op = getattr(fs, f"{kind}_block")
    out = op(to_dev(x, dtype), to_dev(w, dtype), to_dev(h0, dtype), layers)
    expect = scans.block(kind, rounded(x, dtype), rounded(w, dtype), rounded(h0, dtype), layers)
    assert_close(host(out), expect, TOL[dtype], "block out")
    out0 = op(to_dev(x, dtype), to_dev(w, dtype), None, layers)
    expect0 = scans.block(kind, rounded(x, dtype), rounded(w, dtype), None, layers)
    assert_close(host(out0), expect0, TOL[dtype], "block out, h0 = 0")


def test_mingru_block_full_size(rng):
    """B=8, T=2048, H=256, 4 layers (the bench shape), float32, against the oracle."""
    from edifice_amd import fused_scan as fs
    bsz, seq, hid, layers = 8, 2048, 256, 4
    announce("mingru_block_full", shape=(bsz, seq, hid), layers=layers)
    x = rng.normal(size=(bsz, seq, hid)).astype(np.float32)
    w = rng.normal(scale=hid ** -0.5, size=layers * (2 * hid * hid + 4 * hid)).astype(np.float32)
    out = fs.mingru_block(to_dev(x, torch.float32), to_dev(w, torch.float32), None, layers)
    assert_close(host(out), scans.mingru_block(x, w, None, layers), TOL[torch.float32], "block full")


RNN_BLOCK_CASES = [
    # (kind, B, T, H, layers, dtype, initial states given)
    ("lstm", 2, 9, 8, 2, torch.float32, True),
    ("lstm", 1, 1, 16, 3, torch.float32, True),   # one step: every layer on one launch diagonal
    ("gru", 3, 1, 16, 1, torch.float32, False),
    ("gru", 2, 9, 8, 2, torch.float32, True),
    ("lstm", 3, 17, 50, 3, torch.float32, False),
    ("gru", 9, 6, 33, 1, torch.float32, True),     # B past one 8-row step tile
    ("lstm", 2, 12, 256, 2, torch.float32, True),   # reference maximum H
    ("gru", 2, 12, 256, 2, torch.float32, False),
    ("lstm", 1, 40, 128, 4, torch.bfloat16, True),
    ("gru", 2, 70, 64, 2, torch.bfloat16, True),
]


@pytest.mark.parametrize("case", RNN_BLOCK_CASES)
def test_rnn_block(case, rng):
    """FusedScan.lstm_block/5 and gru_block/4 against the layer-by-layer oracle (itself pinned
    to torch.nn.LSTM / torch.nn.GRU and to the step-by-step kernel order)."""
    from edifice_amd import fused_scan as fs
    kind, bsz, seq, hid, layers, dtype, init = case
    announce("rnn_block", case=case)
    gh = scans.RNN_BLOCK_GATES[kind] * hid
    sc = 1 / np.sqrt(hid)
    per = []
    for _ in range(layers):
        per += [sc * rng.normal(size=hid * gh), 0.3 * rng.normal(size=gh), sc * rng.normal(size=hid * gh),
                1 + 0.2 * rng.normal(size=hid), 0.2 * rng.normal(size=hid)]
    w = np.concatenate(per)
    x = rng.normal(size=(bsz, seq, hid))
    h0 = rng.normal(size=(bsz, layers, hid)) if init else None
    c0 = rng.normal(size=(bsz, layers, hid)) if init and kind == "lstm" else None
    tx, tw = to_dev(x, dtype), to_dev(w, dtype)
    th0 = to_dev(h0, dtype) if h0 is not None else None
    tc0 = to_dev(c0, dtype) if c0 is not None else None
    out = fs.lstm_block(tx, tw, th0, tc0, layers) if kind == "lstm" else fs.gru_block(tx, tw, th0, layers)
    r = lambda a: None if a is None else rounded(a, dtype)  # noqa: E731
    want = scans.rnn_block(kind, r(x), r(w), r(h0), r(c0), layers)
    assert_close(host(out), want, TOL[dtype], "out")


@pytest.mark.parametrize("case", [RNN_BLOCK_CASES[3], RNN_BLOCK_CASES[6], RNN_BLOCK_CASES[8]])
def test_rnn_block_paths_agree(case, rng, monkeypatch):
    """The whole recurrence in one persistent launch (grid barrier between diagonals) and
    one launch per diagonal run the same arithmetic: bit-identical outputs, both against
    the oracle."""
    from edifice_amd import fused_scan as fs
    kind, bsz, seq, hid, layers, dtype, init = case
    announce("rnn_block_paths", case=case)
    gh = scans.RNN_BLOCK_GATES[kind] * hid
    sc = 1 / np.sqrt(hid)
    per = []
    for _ in range(layers):
        per += [sc * rng.normal(size=hid * gh), 0.3 * rng.normal(size=gh), sc * rng.normal(size=hid * gh),
                1 + 0.2 * rng.normal(size=hid), 0.2 * rng.normal(size=hid)]
    w = np.concatenate(per)
    x = rng.normal(size=(bsz, seq, hid))
    h0 = rng.normal(size=(bsz, layers, hid)) if init else None
    c0 = rng.normal(size=(bsz, layers, hid)) if init and kind == "lstm" else None
    tx, tw = to_dev(x, dtype), to_dev(w, dtype)
    th0 = to_dev(h0, dtype) if h0 is not None else None
    tc0 = to_dev(c0, dtype) if c0 is not None else None

    def run():
        return host(fs.lstm_block(tx, tw, th0, tc0, layers) if kind == "lstm" else fs.gru_block(tx, tw, th0, layers))

    whole = run()
    monkeypatch.setenv("EDF_RNN_BLOCK_PER_STEP", "1")
    stepwise = run()
    assert np.array_equal(whole, stepwise)
    r = lambda a: None if a is None else rounded(a, dtype)  # noqa: E731
    assert_close(whole, scans.rnn_block(kind, r(x), r(w), r(h0), r(c0), layers), TOL[dtype], "out")


@pytest.mark.parametrize("kind", ["lstm", "gru"])
def test_rnn_block_barrier_timeout_surfaces(kind, rng, monkeypatch):
    """The persistent kernel's bounded grid-barrier wait, had it given up, must not hand the
    caller numbers with EDF_OK.  EDF_RNN_BLOCK_PRESET_ABORT=1 starts the call with the abort
    word set (no wait times out: every wait ends at once and the kernel finishes normally):
    the output is NaN, the status query returns EDF_ERR_LAUNCH and the Python op raises.  A
    following ordinary call on the same workspace is clean again."""
    from edifice_amd import _native as nat
    from edifice_amd import fused_scan as fs
    bsz, seq, hid, layers = 2, 12, 64, 2
    announce("rnn_block_abort", kind=kind)
    gh = scans.RNN_BLOCK_GATES[kind] * hid
    sc = 1 / np.sqrt(hid)
    per = []
    for _ in range(layers):
        per += [sc * rng.normal(size=hid * gh), 0.3 * rng.normal(size=gh), sc * rng.normal(size=hid * gh),
                1 + 0.2 * rng.normal(size=hid), 0.2 * rng.normal(size=hid)]
    tw = to_dev(np.concatenate(per), torch.float32)
    tx = to_dev(rng.normal(size=(bsz, seq, hid)), torch.float32)
    monkeypatch.delenv("EDF_RNN_BLOCK_PER_STEP", raising=False)
    wsb = nat.query(f"edf_{kind}_block_workspace_bytes", bsz, seq, hid, layers, 0)
    ws = torch.empty(wsb, dtype=torch.uint8, device=tx.device)
    out = torch.empty_like(tx)
    L = nat.lib()
    stream = torch.cuda.current_stream().cuda_stream

    def launch():
        if kind == "lstm":
            return L.edf_fused_lstm_block_scan(stream, tx.data_ptr(), tw.data_ptr(), None, None, out.data_ptr(),
                                               ws.data_ptr(), wsb, bsz, seq, hid, layers, 0)
        return L.edf_fused_gru_block_scan(stream, tx.data_ptr(), tw.data_ptr(), None, out.data_ptr(), ws.data_ptr(),
                                          wsb, bsz, seq, hid, layers, 0)

    status = getattr(L, f"edf_{kind}_block_status")
    monkeypatch.setenv("EDF_RNN_BLOCK_PRESET_ABORT", "1")
    assert launch() == 0
    assert status(stream, ws.data_ptr(), wsb, bsz, seq, hid, layers) == 3  # EDF_ERR_LAUNCH
    assert b"timed out" in L.edf_last_error()
    assert torch.isnan(out).all()
    with pytest.raises(nat.EdificeHipError, match="timed out"):
        fs.lstm_block(tx, tw, None, None, layers) if kind == "lstm" else fs.gru_block(tx, tw, None, layers)
    monkeypatch.delenv("EDF_RNN_BLOCK_PRESET_ABORT")
    assert launch() == 0
    assert status(stream, ws.data_ptr(), wsb, bsz, seq, hid, layers) == 0
    want = scans.rnn_block(kind, rounded(tx.cpu().numpy(), torch.float32), rounded(tw.cpu().numpy(), torch.float32),
                           None, None, layers)
    assert_close(host(out), want, TOL[torch.float32], "clean call after the aborted one")
