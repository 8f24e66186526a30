"""numpy float64 restatement of Edifice's fused sequence-mixing ops — TEST INFRASTRUCTURE ONLY.

Only tests, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline leg may use
this module, as the checker.  Every function cites the reference file:line whose
semantics it restates (paths relative to the Edifice repository root).

Layouts follow the reference exactly:
  scans / delta rule   [batch, seq, hidden]  and  [batch, seq, heads, head_dim]
  attention            [batch, heads, seq, head_dim]

Pinning (what independently checks each function; see tests/test_oracle_*.py):
  linear_scan / _backward       seq_len=1 known answer (backward_kernels_test.exs:76-95),
                                a≡1 ⇒ cumulative sum, a≡0 ⇒ b, a = 1 - z, b = z h~ ⇒
                                mingru_scan, torch autograd of a closed-form
                                (cumulative-product) forward, finite differences.
  block (mingru/minlstm/linear) the per-timestep restatement of the reference kernels
                                (block_stepwise), one MinGRU / MinLSTM / linear layer ==
                                LayerNorm + dense + mingru_scan / minlstm_scan /
                                linear_scan + residual written out, W = 0 with a closed
                                form, layers compose (L layers == 1 layer applied L times).
  rnn_block (lstm / gru)        one layer == LayerNorm + torch.nn.LSTM / torch.nn.GRU (z rows
                                negated for torch's h' = (1 - z) n + z h) + residual; layer by
                                layer == step by step (the fused kernels' order).
  mingru_scan / _backward       seq_len=1 known answer (backward_kernels_test.exs:271-287),
                                min_gru_random.safetensors block fixture, z≡1 / z≡0
                                closed forms, torch autograd + finite differences.
  minlstm_scan / _backward      f'+i'≈1 invariant, i≡0 ⇒ constant state, closed form
                                at T=1, torch autograd + finite differences.
  selective_scan (channel mode) B≡0 ⇒ y≡0; N=1, A=0 ⇒ cumulative sum; torch autograd
                                of an independent associative-scan formulation.
  selective_scan (mean mode)    mamba_random.safetensors block fixture.
  selective_scan_backward       torch autograd of the forward, finite differences,
                                clip mask ⇒ ddt=0 outside [1e-3, 0.1].
  delta_rule                    delta_net_random.safetensors (forward and input
                                gradient), β≡0 ⇒ o≡0, α≡1 ⇒ DeltaNet, T=1 closed form.
  kda_scan / _backward          alpha = 0 ==> DeltaNet, rows sharing one decay ==>
                                GatedDeltaNet, torch autograd of an independent forward.
  delta_rule_backward           delta_net_random.safetensors gradient.input, torch
                                autograd of the forward, finite differences.
  delta_product / _backward     the reference's literal [key][value] matrix form, one-step
                                closed form (output follows the key), n_h = 1 ==> the delta
                                rule's states, beta = 0 sub-step ==> identity, torch autograd.
  rla_scan / _backward          gamma = 0 RLA ==> decayed linear attention closed form, RDN
                                with alpha = 1, gamma = 0 ==> DeltaNet, clip 0 ==> empty
                                residual state, torch autograd (with clipped errors).
  ttt_scan / _backward          eta = 0 ==> o = w0 q, w0 = 0 one-step closed form, torch
                                autograd through torch.nn.functional.layer_norm.
  laser_attention / _backward   identical value rows ==> O = that row; torch autograd of an
                                independent torch forward (vmax held constant).
  fox_attention / _backward     cs = const ==> causal flash_attention; torch autograd of an
                                independent torch forward; d cs sums to zero; shift
                                invariance in cs.
  flash_attention / _backward   torch.nn.functional.scaled_dot_product_attention and
                                its autograd, gqa_random.safetensors block fixture,
                                causal row 0 == V[0], identical keys ⇒ mean of V.
"""
from __future__ import annotations

import numpy as np

DT_MIN = 1.0e-3  # fused_selective_scan.cu:30, fused_scan.ex:1469
DT_MAX = 0.1  # fused_selective_scan.cu:31
MINLSTM_EPS = 1.0e-6  # min_lstm.ex:83-84, fused_minlstm_scan.cu:27
KEY_NORM_EPS = 1.0e-6  # delta_net.ex:297-298, gated_delta_net.ex:383-386


def _f64(*xs):
    return [None if x is None else np.asarray(x, dtype=np.float64) for x in xs]


def sigmoid(x):
    x = np.asarray(x, dtype=np.float64)
    return 0.5 * (1.0 + np.tanh(0.5 * x))


def silu(x):
    return x * sigmoid(x)


def softplus(x):
    x = np.asarray(x, dtype=np.float64)
    return np.logaddexp(0.0, x)


# ---------------------------------------------------------------------------
# MinGRU   h_t = (1 - z_t) h_{t-1} + z_t h~_t
# ---------------------------------------------------------------------------

def mingru_scan(z, cand, h0=None):
    """Forward with post-sigmoid gates and explicit h0.

    Follows ``mingru_scan_fallback`` (lib/edifice/cuda/fused_scan.ex:516-528) and the
    kernel contract of native/cuda/fused_mingru_scan.cu:38-65.
    """
    z, cand, h0 = _f64(z, cand, h0)
    bsz, seq, hid = z.shape
    h = np.zeros((bsz, hid)) if h0 is None else h0.copy()
    out = np.empty_like(z)
    for t in range(seq):
        h = (1.0 - z[:, t]) * h + z[:, t] * cand[:, t]
        out[:, t] = h
    return out


def mingru_scan_backward(z, cand, h0, fwd, dy):
    """Reverse pass -> (dz, dcand, dh0).

    Follows ``mingru_backward_fallback`` (fused_scan.ex:548-581): dh accumulates the
    upstream gradient, dz = dh (h~_t - h_{t-1}), dcand = dh z_t, carry dh (1 - z_t).
    """
    z, cand, h0, fwd, dy = _f64(z, cand, h0, fwd, dy)
    bsz, seq, hid = z.shape
    if h0 is None:
        h0 = np.zeros((bsz, hid))
    dz = np.empty_like(z)
    dc = np.empty_like(z)
    carry = np.zeros((bsz, hid))
    for t in range(seq - 1, -1, -1):
        dh = dy[:, t] + carry
        h_prev = h0 if t == 0 else fwd[:, t - 1]
        dz[:, t] = dh * (cand[:, t] - h_prev)
        dc[:, t] = dh * z[:, t]
        carry = dh * (1.0 - z[:, t])
    return dz, dc, carry


def min_gru_scan(gates, cand):
    """Logit-level MinGRU: sigmoid applied first, h0 = 0 (min_gru.ex:305-326)."""
    return mingru_scan(sigmoid(gates), cand, None)


def min_gru_scan_backward(gates, cand, dy):
    """Gradients of ``min_gru_scan`` w.r.t. (gates, cand).

    The post-sigmoid gradient comes from ``mingru_scan_backward``; the chain rule
    dz * z (1 - z) follows fused_scan.ex:474-480.
    """
    z = sigmoid(gates)
    fwd = mingru_scan(z, cand, None)
    dz, dc, _ = mingru_scan_backward(z, cand, None, fwd, dy)
    return dz * z * (1.0 - z), dc


# ---------------------------------------------------------------------------
# Generic linear scan  h_t = a_t h_{t-1} + b_t
# ---------------------------------------------------------------------------

def linear_scan(a, b, h0=None):
    """Forward -> all hidden states.

    Follows ``linear_scan_cc_fallback`` / ``linear_scan_fallback``
    (lib/edifice/cuda/fused_scan.ex:869-881, 4429-4443) and the kernel contract of
    native/cuda/fused_linear_scan.cu:42-64; h0 = None means zeros.
    """
    a, b, h0 = _f64(a, b, h0)
    bsz, seq, hid = a.shape
    h = np.zeros((bsz, hid)) if h0 is None else h0.copy()
    out = np.empty_like(a)
    for t in range(seq):
        h = a[:, t] * h + b[:, t]
        out[:, t] = h
    return out


def linear_scan_backward(a, h0, fwd, dy):
    """Reverse pass -> (da, db, dh0).

    Follows ``linear_scan_backward_fallback`` (fused_scan.ex:884-915) and
    native/cuda/fused_linear_scan_backward.cu:42-80: dh = dy_t + carry,
    da_t = dh h_{t-1}, db_t = dh, carry = dh a_t; dh0 is the final carry.
    """
    a, h0, fwd, dy = _f64(a, h0, fwd, dy)
    bsz, seq, hid = a.shape
    if h0 is None:
        h0 = np.zeros((bsz, hid))
    da = np.empty_like(a)
    db = np.empty_like(a)
    carry = np.zeros((bsz, hid))
    for t in range(seq - 1, -1, -1):
        dh = dy[:, t] + carry
        h_prev = h0 if t == 0 else fwd[:, t - 1]
        da[:, t] = dh * h_prev
        db[:, t] = dh
        carry = dh * a[:, t]
    return da, db, carry


# ---------------------------------------------------------------------------
# Multi-layer MinGRU block (inference)
# ---------------------------------------------------------------------------

BLOCK_LN_EPS = 1.0e-5  # fused_mingru_block_scan.cu:110, fused_scan.ex:4544


BLOCK_PROJECTIONS = {"mingru": 2, "minlstm": 3, "linear": 2}


def _block_layer_weights(weights, layer, hid, nproj):
    """Slices of the per-layer packing W_1 [H][H], b_1, .., W_P, b_P, gamma, beta
    (min_gru.ex:217-241; fused_scan.ex:4525-4540, 4653-4672, 4789-4802)."""
    w = np.asarray(weights, dtype=np.float64).reshape(-1)
    off = layer * (nproj * (hid * hid + hid) + 2 * hid)
    proj = []
    for _ in range(nproj):
        proj.append((w[off:off + hid * hid].reshape(hid, hid), w[off + hid * hid:off + hid * hid + hid]))
        off += hid * hid + hid
    return proj, w[off:off + hid], w[off + hid:off + 2 * hid]


def _block_norm(x, gamma, beta):
    mean = x.mean(-1, keepdims=True)
    var = ((x - mean) ** 2).mean(-1, keepdims=True)
    return (x - mean) / np.sqrt(var + BLOCK_LN_EPS) * gamma + beta


def _block_step_coeffs(kind, p):
    """(a, b) of h = a h + b from the layer's projections (fused_mingru_block_scan.cu:127-131,
    fused_minlstm_block_scan.cu:128-137, fused_linear_block_scan.cu:112-123)."""
    if kind == "mingru":
        z = sigmoid(p[0])
        return 1.0 - z, z * p[1]
    if kind == "minlstm":
        sf, si = sigmoid(p[0]), sigmoid(p[1])
        s = sf + si + MINLSTM_EPS
        return sf / s, si / s * p[2]
    return p[0], p[1]


def block(kind, x, weights, h0, num_layers):
    """Layer by layer over the whole sequence, as the reference fallbacks
    ``mingru_block_fallback`` / ``minlstm_block_fallback`` / ``linear_block_fallback``
    (lib/edifice/cuda/fused_scan.ex:4521-4571, 4647-4705, 4785-4835): LayerNorm (biased
    variance, eps 1e-5, gamma, beta), the projections, the layer's scan from h0[:, l],
    residual x + h.  h0 = None means zeros."""
    x = np.asarray(x, dtype=np.float64)
    bsz, seq, hid = x.shape
    h0 = np.zeros((bsz, num_layers, hid)) if h0 is None else np.asarray(h0, dtype=np.float64)
    for layer in range(num_layers):
        proj, gamma, beta = _block_layer_weights(weights, layer, hid, BLOCK_PROJECTIONS[kind])
        n = _block_norm(x, gamma, beta)
        a, b = _block_step_coeffs(kind, [n @ w + bias for w, bias in proj])
        h = h0[:, layer].copy()
        hs = np.empty_like(x)
        for t in range(seq):
            h = a[:, t] * h + b[:, t]
            hs[:, t] = h
        x = x + hs
    return x


def block_stepwise(kind, x, weights, h0, num_layers):
    """Timestep by timestep, every layer per step, as the reference kernels walk it
    (fused_mingru_block_scan.cu:73-135, fused_minlstm_block_scan.cu:66-144,
    fused_linear_block_scan.cu:68-130); an independent formulation of ``block``."""
    x = np.asarray(x, dtype=np.float64)
    bsz, seq, hid = x.shape
    h = np.zeros((bsz, num_layers, hid)) if h0 is None else np.array(h0, dtype=np.float64)
    lw = [_block_layer_weights(weights, layer, hid, BLOCK_PROJECTIONS[kind]) for layer in range(num_layers)]
    out = np.empty_like(x)
    for t in range(seq):
        xv = x[:, t].copy()
        for layer, (proj, gamma, beta) in enumerate(lw):
            n = _block_norm(xv, gamma, beta)
            a, b = _block_step_coeffs(kind, [n @ w + bias for w, bias in proj])
            h[:, layer] = a * h[:, layer] + b
            xv = xv + h[:, layer]
        out[:, t] = xv
    return out


RNN_BLOCK_GATES = {"lstm": 4, "gru": 3}


def _rnn_layer_weights(weights, layer, hid, gates):
    """Per-layer packing W_x [H, G H], b_x [G H], R [H, G H], gamma [H], beta [H]
    (fused_lstm_block_scan.cu:14-16, fused_gru_block_scan.cu:14-16)."""
    w = np.asarray(weights, dtype=np.float64)
    gh = gates * hid
    o = layer * (2 * hid * gh + gh + 2 * hid)
    wx = w[o:o + hid * gh].reshape(hid, gh)
    o += hid * gh
    bx = w[o:o + gh]
    o += gh
    r = w[o:o + hid * gh].reshape(hid, gh)
    o += hid * gh
    return wx, bx, r, w[o:o + hid], w[o + hid:o + 2 * hid]


def _rnn_cell(kind, xp, rh, h, c, hid):
    """One LSTM (gates i, f, g, o) or GRU (r, z, n; reset on the recurrent part of n only,
    h = (1 - z) h + z n) step from the input and recurrent projections."""
    sl = [slice(k * hid, (k + 1) * hid) for k in range(RNN_BLOCK_GATES[kind])]
    if kind == "lstm":
        i, f, o = (sigmoid(xp[..., s] + rh[..., s]) for s in (sl[0], sl[1], sl[3]))
        g = np.tanh(xp[..., sl[2]] + rh[..., sl[2]])
        c = f * c + i * g
        return o * np.tanh(c), c
    r, z = (sigmoid(xp[..., s] + rh[..., s]) for s in (sl[0], sl[1]))
    n = np.tanh(xp[..., sl[2]] + r * rh[..., sl[2]])
    return (1.0 - z) * h + z * n, c


def rnn_block(kind, x, weights, h0, c0, num_layers):
    """Multi-layer LSTM / GRU block, layer by layer as ``lstm_block_fallback`` /
    ``gru_block_fallback`` (fused_scan.ex:4911-4990, 5055-5120): LayerNorm (biased variance,
    eps 1e-5), input projection n W_x + b_x for all steps, the recurrence with R h_{t-1} from
    h0[:, l] (and c0[:, l]), residual x + h.  None initial states mean zeros."""
    x = np.asarray(x, dtype=np.float64)
    bsz, seq, hid = x.shape
    h0 = np.zeros((bsz, num_layers, hid)) if h0 is None else np.asarray(h0, dtype=np.float64)
    c0 = np.zeros((bsz, num_layers, hid)) if c0 is None else np.asarray(c0, dtype=np.float64)
    for layer in range(num_layers):
        wx, bx, r, gamma, beta = _rnn_layer_weights(weights, layer, hid, RNN_BLOCK_GATES[kind])
        xp = _block_norm(x, gamma, beta) @ wx + bx
        h, c = h0[:, layer].copy(), c0[:, layer].copy()
        hs = np.empty_like(x)
        for t in range(seq):
            h, c = _rnn_cell(kind, xp[:, t], h @ r, h, c, hid)
            hs[:, t] = h
        x = x + hs
    return x


def rnn_block_stepwise(kind, x, weights, h0, c0, num_layers):
    """Timestep by timestep, every layer per step, as the fused reference kernels walk it
    (fused_lstm_block_scan.cu:80-170, fused_gru_block_scan.cu:75-165)."""
    x = np.asarray(x, dtype=np.float64)
    bsz, seq, hid = x.shape
    h = np.zeros((bsz, num_layers, hid)) if h0 is None else np.array(h0, dtype=np.float64)
    c = np.zeros((bsz, num_layers, hid)) if c0 is None else np.array(c0, dtype=np.float64)
    lw = [_rnn_layer_weights(weights, layer, hid, RNN_BLOCK_GATES[kind]) for layer in range(num_layers)]
    out = np.empty_like(x)
    for t in range(seq):
        xv = x[:, t].copy()
        for layer, (wx, bx, r, gamma, beta) in enumerate(lw):
            xp = _block_norm(xv, gamma, beta) @ wx + bx
            h[:, layer], c[:, layer] = _rnn_cell(kind, xp, h[:, layer] @ r, h[:, layer], c[:, layer], hid)
            xv = xv + h[:, layer]
        out[:, t] = xv
    return out


def mingru_block(x, weights, h0, num_layers):
    """``block("mingru", ...)``: the multi-layer MinGRU block (fused_scan.ex:4521-4571)."""
    return block("mingru", x, weights, h0, num_layers)


def mingru_block_stepwise(x, weights, h0, num_layers):
    return block_stepwise("mingru", x, weights, h0, num_layers)


# ---------------------------------------------------------------------------
# MinLSTM  c_t = f'_t c_{t-1} + i'_t h~_t,  f' = f/(f+i+eps), i' = i/(f+i+eps)
# ---------------------------------------------------------------------------

def minlstm_scan(f, i, cand, h0=None):
    """Forward with post-sigmoid gates (fused_scan.ex:583-602, fused_minlstm_scan.cu:37-68)."""
    f, i, cand, h0 = _f64(f, i, cand, h0)
    bsz, seq, hid = f.shape
    s = f + (i + MINLSTM_EPS)
    fn, inn = f / s, i / s
    c = np.zeros((bsz, hid)) if h0 is None else h0.copy()
    out = np.empty_like(f)
    for t in range(seq):
        c = fn[:, t] * c + inn[:, t] * cand[:, t]
        out[:, t] = c
    return out


def minlstm_scan_backward(f, i, cand, h0, fwd, dy):
    """Reverse pass -> (df, di, dcand, dh0), quotient rule through the normalisation.

    Follows ``minlstm_backward_fallback`` (fused_scan.ex:623-677).
    """
    f, i, cand, h0, fwd, dy = _f64(f, i, cand, h0, fwd, dy)
    bsz, seq, hid = f.shape
    if h0 is None:
        h0 = np.zeros((bsz, hid))
    df = np.empty_like(f)
    di = np.empty_like(f)
    dcand = np.empty_like(f)
    carry = np.zeros((bsz, hid))
    for t in range(seq - 1, -1, -1):
        dc = dy[:, t] + carry
        ft, it = f[:, t], i[:, t]
        s = ft + (it + MINLSTM_EPS)
        c_prev = h0 if t == 0 else fwd[:, t - 1]
        df_n = dc * c_prev
        di_n = dc * cand[:, t]
        dcand[:, t] = dc * (it / s)
        carry = dc * (ft / s)
        s2 = s * s
        df[:, t] = (df_n * (it + MINLSTM_EPS) - di_n * it) / s2
        di[:, t] = (-df_n * ft + di_n * (ft + MINLSTM_EPS)) / s2
    return df, di, dcand, carry


def min_lstm_scan(forget_gates, input_gates, cand):
    """Logit-level MinLSTM (min_lstm.ex:304-334)."""
    return minlstm_scan(sigmoid(forget_gates), sigmoid(input_gates), cand, None)


# ---------------------------------------------------------------------------
# Selective scan (Mamba)
# ---------------------------------------------------------------------------

def selective_scan(x, dt, A, B, C, D=None, z=None, mode="channel", return_states=False):
    """Mamba selective scan, forward.

    mode="channel" — kernel semantics: dt clipped to [1e-3, 0.1], A_bar = exp(dt A[d,n]),
      B_bar = dt B (native/cuda/fused_selective_scan.cu:41-91; restated in
      test/edifice/cuda/backward_kernels_test.exs:1563-1586).
    mode="mean" — block CPU semantics: B_bar = mean_d(clip(dt)) B
      (lib/edifice/ssm/common.ex:402-445 discretize_ssm, :492-513 sequential_scan,
      :462-471 compute_ssm_output, :661-668 selective_scan_fallback).
    Optional extensions with no reference kernel counterpart (the Mamba block applies
    the gate outside the scan, common.ex:270-278): y += D[d] x, then y *= silu(z).
    """
    x, dt, A, B, C, D, z = _f64(x, dt, A, B, C, D, z)
    bsz, seq, hid = x.shape
    n = A.shape[1]
    dtc = np.clip(dt, DT_MIN, DT_MAX)
    if mode == "mean":
        dtb = np.broadcast_to(dtc.mean(axis=2, keepdims=True), dtc.shape)
    elif mode == "channel":
        dtb = dtc
    else:
        raise ValueError(mode)
    h = np.zeros((bsz, hid, n))
    y = np.empty_like(x)
    states = []
    for t in range(seq):
        a_bar = np.exp(dtc[:, t, :, None] * A[None])
        h = a_bar * h + (dtb[:, t, :, None] * B[:, t, None, :]) * x[:, t, :, None]
        if return_states:
            states.append(h.copy())
        y[:, t] = np.einsum("bdn,bn->bd", h, C[:, t])
    if D is not None:
        y = y + D[None, None, :] * x
    out = y * silu(z) if z is not None else y
    if return_states:
        return out, np.stack(states, axis=1)
    return out


def selective_scan_backward(x, dt, A, B, C, dout, D=None, z=None, mode="channel"):
    """Reverse pass -> dict(dx, ddt, dA, dB, dC, dD, dz).

    The scan part follows ``selective_scan_backward_fallback`` (fused_scan.ex:1453-1533):
    dh += dy C; dC += sum_d dy h; dx += sum_n dh dt B; ddt += sum_n dh (h_prev A_bar A + B x),
    zeroed where dt was clipped; dB += sum_d dh x dt; carry dh A_bar.  Extensions with no
    reference counterpart: dA = sum_{b,t} dh h_prev A_bar dt (the reference kernel has
    no dA output, fused_selective_scan_backward.cu:198-238), dD, dz (silu gate), and the
    mean-mode dt coupling.
    """
    x, dt, A, B, C, dout, D, z = _f64(x, dt, A, B, C, dout, D, z)
    bsz, seq, hid = x.shape
    n = A.shape[1]
    dtc = np.clip(dt, DT_MIN, DT_MAX)
    in_range = (dt >= DT_MIN) & (dt <= DT_MAX)
    mean_mode = mode == "mean"
    dtb = np.broadcast_to(dtc.mean(axis=2, keepdims=True), dtc.shape) if mean_mode else dtc

    # recompute forward states (h_prev for each t)
    h = np.zeros((bsz, hid, n))
    hprev = np.empty((bsz, seq, hid, n))
    for t in range(seq):
        hprev[:, t] = h
        a_bar = np.exp(dtc[:, t, :, None] * A[None])
        h = a_bar * h + (dtb[:, t, :, None] * B[:, t, None, :]) * x[:, t, :, None]

    res = {}
    if z is not None:
        y_ssm = selective_scan(x, dt, A, B, C, D, None, mode)
        sz = sigmoid(z)
        dy = dout * z * sz
        res["dz"] = dout * y_ssm * sz * (1.0 + z * (1.0 - sz))
    else:
        dy = dout
        res["dz"] = None
    dx = np.zeros_like(x)
    if D is not None:
        res["dD"] = np.einsum("btd,btd->d", dy, x)
        dx += dy * D[None, None, :]
    else:
        res["dD"] = None
    ddt = np.zeros_like(x)
    dA = np.zeros_like(A)
    dB = np.zeros_like(B)
    dC = np.zeros_like(C)
    dh = np.zeros((bsz, hid, n))
    for t in range(seq - 1, -1, -1):
        a_bar = np.exp(dtc[:, t, :, None] * A[None])
        hp = hprev[:, t]
        h_cur = a_bar * hp + (dtb[:, t, :, None] * B[:, t, None, :]) * x[:, t, :, None]
        dh = dh + dy[:, t, :, None] * C[:, t, None, :]
        dC[:, t] = np.einsum("bd,bdn->bn", dy[:, t], h_cur)
        dx[:, t] += np.einsum("bdn,bd,bn->bd", dh, dtb[:, t], B[:, t])
        g_a = np.einsum("bdn,bdn->bd", dh * hp, a_bar * A[None])
        dA += np.einsum("bdn,bd->dn", dh * hp * a_bar, dtc[:, t])
        g_b = np.einsum("bdn,bn,bd->bd", dh, B[:, t], x[:, t])
        if mean_mode:
            ddt[:, t] = g_a + g_b.sum(axis=1, keepdims=True) / hid
            dB[:, t] = np.einsum("bdn,bd->bn", dh, x[:, t]) * dtb[:, t, 0][:, None]
        else:
            ddt[:, t] = g_a + g_b
            dB[:, t] = np.einsum("bdn,bd,bd->bn", dh, x[:, t], dtc[:, t])
        dh = dh * a_bar
    ddt = np.where(in_range, ddt, 0.0)
    res.update(dx=dx, ddt=ddt, dA=dA, dB=dB, dC=dC)
    return res


# ---------------------------------------------------------------------------
# Delta rule (DeltaNet / GatedDeltaNet)
# ---------------------------------------------------------------------------

def _beta4(beta, shape):
    beta = np.asarray(beta, dtype=np.float64)
    if beta.ndim == 3:  # per-head beta [B,T,H] broadcast along the value rows
        beta = np.broadcast_to(beta[..., None], shape)
    return beta


def _decay4(alpha, shape):
    """Per-row decay [B,T,H,d_v] from a per-head alpha [B,T,H] (broadcast along the rows) or
    a per-row one; None stays None."""
    if alpha is None:
        return None
    alpha = np.asarray(alpha, dtype=np.float64)
    return np.broadcast_to(alpha[..., None], shape) if alpha.ndim == 3 else alpha


def l2_normalize_keys(k):
    """k / sqrt(sum k^2 + 1e-6) over head_dim (delta_net.ex:297-298)."""
    k = np.asarray(k, dtype=np.float64)
    return k / np.sqrt((k * k).sum(axis=-1, keepdims=True) + KEY_NORM_EPS)


def delta_rule(q, k, v, beta, alpha=None, return_states=False):
    """o_t = S_t q_t with S_t = a_t S_{t-1} + diag(beta_t)(v_t - a_t S_{t-1} k_t) k_t^T.

    S is [heads, d_v, d_k] per batch, retrieval S k contracts the key axis.
    alpha=None is DeltaNet (delta_net.ex:231-273); otherwise GatedDeltaNet with a per
    (b, t, head) scalar decay (gated_delta_net.ex:300-353), or a decay per value row
    [B,T,H,d_v] (multiplicative; ``kda_scan`` passes exp of KDA's log decay).  beta is per element
    [B,T,H,d] as in the reference, or per head [B,T,H] (broadcast along d).
    No 1/sqrt(d) scaling of q (delta_net.ex:266-268).
    """
    q, k, v = _f64(q, k, v)
    alpha = _decay4(alpha, v.shape)
    beta = _beta4(beta, v.shape)
    bsz, seq, nh, d = q.shape
    dv = v.shape[3]
    S = np.zeros((bsz, nh, dv, d))
    out = np.empty((bsz, seq, nh, dv))
    states = []
    for t in range(seq):
        if alpha is not None:
            S = alpha[:, t, :, :, None] * S
        r = np.einsum("bhij,bhj->bhi", S, k[:, t])
        err = beta[:, t] * (v[:, t] - r)
        S = S + err[..., :, None] * k[:, t, :, None, :]
        if return_states:
            states.append(S.copy())
        out[:, t] = np.einsum("bhij,bhj->bhi", S, q[:, t])
    if return_states:
        return out, np.stack(states, axis=1)
    return out


def delta_rule_backward(q, k, v, beta, do, alpha=None):
    """Reverse pass -> dict(dq, dk, dv, dbeta, dalpha).

    Follows ``delta_rule_backward_fallback`` (fused_scan.ex:1257-1328) and
    ``gated_delta_net_backward_fallback`` (fused_scan.ex:1347-1431):
      dS_total = dS + do q^T; dq = S_t^T do; ds_k = dS_total k;
      dv = beta ds_k; dbeta = err ds_k;
      dk = dS_total^T (beta err) - S_g^T (beta ds_k);
      dalpha = sum(dS_to_decayed * S_prev); dS_prev = alpha dS_to_decayed.
    For per-head beta the per-element dbeta is summed over the value rows.
    """
    q, k, v, do = _f64(q, k, v, do)
    per_head_alpha = alpha is not None and np.asarray(alpha).ndim == 3
    alpha = _decay4(alpha, v.shape)
    per_head_beta = np.asarray(beta).ndim == 3
    beta = _beta4(beta, v.shape)
    bsz, seq, nh, d = q.shape
    dv_ = v.shape[3]
    # forward states
    S = np.zeros((bsz, nh, dv_, d))
    s_prev = np.empty((bsz, seq, nh, dv_, d))
    for t in range(seq):
        s_prev[:, t] = S
        sg = S if alpha is None else alpha[:, t, :, :, None] * S
        r = np.einsum("bhij,bhj->bhi", sg, k[:, t])
        S = sg + (beta[:, t] * (v[:, t] - r))[..., :, None] * k[:, t, :, None, :]
    dq = np.empty_like(q)
    dk = np.empty_like(k)
    dvv = np.empty_like(v)
    dbeta = np.empty_like(v)
    dalpha = np.empty((bsz, seq, nh, dv_)) if alpha is not None else None
    dS = np.zeros((bsz, nh, dv_, d))
    for t in range(seq - 1, -1, -1):
        sp = s_prev[:, t]
        a = None if alpha is None else alpha[:, t, :, :, None]
        sg = sp if a is None else a * sp
        kt, qt, bt = k[:, t], q[:, t], beta[:, t]
        err = v[:, t] - np.einsum("bhij,bhj->bhi", sg, kt)
        s_new = sg + (bt * err)[..., :, None] * kt[..., None, :]
        dtot = dS + do[:, t][..., :, None] * qt[..., None, :]
        dq[:, t] = np.einsum("bhij,bhi->bhj", s_new, do[:, t])
        ds_k = np.einsum("bhij,bhj->bhi", dtot, kt)
        d_dec = dtot - (bt * ds_k)[..., :, None] * kt[..., None, :]
        dvv[:, t] = bt * ds_k
        dbeta[:, t] = err * ds_k
        dk[:, t] = (np.einsum("bhij,bhi->bhj", dtot, bt * err)
                    - np.einsum("bhij,bhi->bhj", sg, bt * ds_k))
        if a is None:
            dS = d_dec
        else:
            dalpha[:, t] = (d_dec * sp).sum(axis=3)
            dS = a * d_dec
    if per_head_beta:
        dbeta = dbeta.sum(axis=3)
    if per_head_alpha:
        dalpha = dalpha.sum(axis=3)
    return dict(dq=dq, dk=dk, dv=dvv, dbeta=dbeta, dalpha=dalpha)


def kda_scan(q, k, v, alpha, beta):
    """KDA: the delta rule with decay exp(alpha_t) per value row and a per-head beta
    (``kda_scan_fallback``, fused_scan.ex:2632-2665; kernel fused_kda_scan.cu:1-24)."""
    return delta_rule(q, k, v, beta, np.exp(np.asarray(alpha, dtype=np.float64)))


def kda_scan_backward(q, k, v, alpha, beta, do):
    """-> dict(dq, dk, dv, dbeta [B,T,H], dalpha [B,T,H,d] in log space)
    (``kda_backward_fallback``, fused_scan.ex:1552-1640): the decay gradient of
    ``delta_rule_backward`` times exp(alpha)."""
    dec = np.exp(np.asarray(alpha, dtype=np.float64))
    g = delta_rule_backward(q, k, v, beta, do, dec)
    g["dalpha"] = g["dalpha"] * dec
    return g


TTT_LN_EPS = 1.0e-6  # fused_ttt_scan.cu:35


def _ttt_fwd(q, k, v, eta, w0, ln_g, ln_b):
    """-> (out, list of W before each step, x_hat, err, rstd)."""
    bsz, seq, dd = q.shape
    W = w0.copy()
    out = np.empty_like(q)
    ws, xh, er, rs = [], np.empty_like(q), np.empty_like(q), np.empty((bsz, seq))
    for t in range(seq):
        ws.append(W)
        pred = np.einsum("bij,bj->bi", W, k[:, t])
        mu = pred.mean(axis=-1, keepdims=True)
        var = ((pred - mu) ** 2).mean(axis=-1, keepdims=True)
        r = 1.0 / np.sqrt(var + TTT_LN_EPS)
        x = (pred - mu) * r
        err = ln_g * x + ln_b - v[:, t]
        W = W - (eta[:, t] * err)[..., :, None] * k[:, t][:, None, :]
        out[:, t] = np.einsum("bij,bj->bi", W, q[:, t])
        xh[:, t], er[:, t], rs[:, t] = x, err, r[..., 0]
    return out, ws, xh, er, rs


def ttt_scan(q, k, v, eta, w0, ln_g, ln_b):
    """TTT-Linear: an inner linear model W [B, D, D] (initial w0) trained at every step by one
    LayerNorm-ed reconstruction step (fused_ttt_scan.cu:1-30 and 85-150; fallback
    ``ttt_scan_fallback``, ttt.ex:369-404):
      pred = W k;  x_hat = (pred - mean) / sqrt(var + 1e-6) (population variance over D);
      err = ln_g x_hat + ln_b - v;  W = W - (eta err) k^T;  o = W q.
    q, k, v, eta (post-sigmoid, per element) [B, T, D]; ln_g, ln_b [D]."""
    q, k, v, eta, w0, ln_g, ln_b = _f64(q, k, v, eta, w0, ln_g, ln_b)
    return _ttt_fwd(q, k, v, eta, w0, ln_g, ln_b)[0]


def ttt_scan_backward(q, k, v, eta, w0, ln_g, ln_b, do):
    """Reverse pass -> dict(dq, dk, dv, deta [B,T,D], dw0 [B,D,D], dln_g, dln_b [D])
    (fused_ttt_scan_backward.cu:300-420 for the per-step math): with dW the adjoint after
    step t, dW_t = dW + do q^T, dq = W_t^T do, d se = -dW_t k, deta = d se * err,
    d err = d se * eta, dv = -d err, dln_g += d err x_hat, dln_b += d err,
    dx = ln_g d err, d pred = rstd (dx - mean(dx) - x_hat mean(dx x_hat)),
    dk = -dW_t^T se + W_p^T d pred, dW <- dW_t + d pred k^T; dw0 = the final dW."""
    q, k, v, eta, w0, ln_g, ln_b, do = _f64(q, k, v, eta, w0, ln_g, ln_b, do)
    bsz, seq, dd = q.shape
    _, ws, xh, er, rs = _ttt_fwd(q, k, v, eta, w0, ln_g, ln_b)
    dq, dk, dv, de = (np.empty_like(q) for _ in range(4))
    dg, db = np.zeros(dd), np.zeros(dd)
    dW = np.zeros_like(w0)
    for t in range(seq - 1, -1, -1):
        wp = ws[t]
        se = eta[:, t] * er[:, t]
        wt = wp - se[..., :, None] * k[:, t][:, None, :]
        dwt = dW + do[:, t][..., :, None] * q[:, t][:, None, :]
        dq[:, t] = np.einsum("bij,bi->bj", wt, do[:, t])
        dse = -np.einsum("bij,bj->bi", dwt, k[:, t])
        de[:, t] = dse * er[:, t]
        derr = dse * eta[:, t]
        dv[:, t] = -derr
        dg += (derr * xh[:, t]).sum(axis=0)
        db += derr.sum(axis=0)
        dx = ln_g * derr
        x = xh[:, t]
        dpred = rs[:, t][:, None] * (dx - dx.mean(-1, keepdims=True) - x * (dx * x).mean(-1, keepdims=True))
        dk[:, t] = -np.einsum("bij,bi->bj", dwt, se) + np.einsum("bij,bi->bj", wp, dpred)
        dW = dwt + dpred[..., :, None] * k[:, t][:, None, :]
    return dict(dq=dq, dk=dk, dv=dv, deta=de, dw0=dW, dln_g=dg, dln_b=db)


RLA_VARIANTS = {"rla": 0, "rdn": 1}  # fused_scan.ex:425-433


def _rla_step(S, R, kt, vt, a, b, g, variant, clip):
    """One RLA / RDN step from (S, R) -> (S_t, R_t, e, re, rr) (fused_rla_scan.cu:114-165,
    ``rla_scan_fallback`` fused_scan.ex:2692-2768).  a, b, g broadcast as [B, H, 1]."""
    rs = np.einsum("bhij,bhj->bhi", S, kt)
    e = vt - rs
    re = np.clip(e, -clip, clip)
    if variant == 0:   # RLA: S = a S + b v k^T, R = a R + g re k^T
        rr = None
        cs, cr = b * vt, g * re
    else:              # RDN: S = a S + b (v - S k) k^T, R = a R + g (re - R k) k^T
        rr = np.einsum("bhij,bhj->bhi", R, kt)
        cs, cr = b * e, g * (re - rr)
    S_t = a[..., None] * S + cs[..., :, None] * kt[..., None, :]
    R_t = a[..., None] * R + cr[..., :, None] * kt[..., None, :]
    return S_t, R_t, e, re, rr


def rla_scan(q, k, v, alpha, beta, gamma, variant=0, clip=1.0):
    """Residual linear attention: base state S and residual state R [H, d_v, d_k],
    retrieval S_{t-1} k_t, residual error re = clip(v - S_{t-1} k_t, -c, c),
    o_t = (S_t + R_t) q_t.  variant 0 (RLA) / 1 (RDN); alpha, beta, gamma per head [B,T,H]."""
    q, k, v, alpha, beta, gamma = _f64(q, k, v, alpha, beta, gamma)
    bsz, seq, nh, d = q.shape
    S = np.zeros((bsz, nh, d, d))
    R = np.zeros((bsz, nh, d, d))
    out = np.empty_like(q)
    for t in range(seq):
        S, R, *_ = _rla_step(S, R, k[:, t], v[:, t], alpha[:, t, :, None], beta[:, t, :, None],
                             gamma[:, t, :, None], variant, clip)
        out[:, t] = np.einsum("bhij,bhj->bhi", S + R, q[:, t])
    return out


def rla_scan_backward(q, k, v, alpha, beta, gamma, do, variant=0, clip=1.0):
    """Reverse pass -> dict(dq, dk, dv, dalpha, dbeta, dgamma) (the per-head gate gradients
    [B,T,H]); structure of ``rla_backward_fallback`` (fused_scan.ex:1675-1812) and
    fused_rla_scan_backward.cu:62-618, the clip passing gradient where |e| <= c
    (fused_rla_scan_backward.cu:163).  Per step (S_p, R_p before it):
      dS_tot = dS + do q^T, dR_tot = dR + do q^T, dq = (S_t + R_t)^T do,
      ds_k = dS_tot k, dr_k = dR_tot k, m = [|e| <= c]; with cS, cR the row coefficients of
      k^T in the two updates, dE_S = g dr_k m (RLA) or b ds_k + g dr_k m (RDN) and
      dE_R = 0 (RLA) or g dr_k (RDN):
      dv = b ds_k + g dr_k m,  dk = dS_tot^T cS + dR_tot^T cR - S_p^T dE_S - R_p^T dE_R,
      dalpha = <dS_tot, S_p> + <dR_tot, R_p>, dbeta = ds_k . (v or e), dgamma = dr_k . cR / g,
      dS <- a dS_tot - dE_S k^T, dR <- a dR_tot - dE_R k^T."""
    q, k, v, alpha, beta, gamma, do = _f64(q, k, v, alpha, beta, gamma, do)
    bsz, seq, nh, d = q.shape
    S = np.zeros((bsz, nh, d, d))
    R = np.zeros((bsz, nh, d, d))
    hist = []
    for t in range(seq):
        hist.append((S, R))
        S, R, *_ = _rla_step(S, R, k[:, t], v[:, t], alpha[:, t, :, None], beta[:, t, :, None],
                             gamma[:, t, :, None], variant, clip)
    g_ = {n: np.empty_like(x) for n, x in (("dq", q), ("dk", k), ("dv", v), ("dalpha", alpha),
                                            ("dbeta", beta), ("dgamma", gamma))}
    dS = np.zeros_like(S)
    dR = np.zeros_like(R)
    for t in range(seq - 1, -1, -1):
        sp, rp = hist[t]
        a, b, g = alpha[:, t, :, None], beta[:, t, :, None], gamma[:, t, :, None]
        kt, vt, qt, dot = k[:, t], v[:, t], q[:, t], do[:, t]
        s_t, r_t, e, re, rr = _rla_step(sp, rp, kt, vt, a, b, g, variant, clip)
        m = (np.abs(e) <= clip).astype(np.float64)
        outer = dot[..., :, None] * qt[..., None, :]
        dst, drt = dS + outer, dR + outer
        g_["dq"][:, t] = np.einsum("bhij,bhi->bhj", s_t + r_t, dot)
        ds_k = np.einsum("bhij,bhj->bhi", dst, kt)
        dr_k = np.einsum("bhij,bhj->bhi", drt, kt)
        if variant == 0:
            cs, cr, cb, cg = b * vt, g * re, vt, re
            des, der = g * dr_k * m, np.zeros_like(dr_k)
        else:
            cs, cr, cb, cg = b * e, g * (re - rr), e, re - rr
            des, der = b * ds_k + g * dr_k * m, g * dr_k
        g_["dv"][:, t] = b * ds_k + g * dr_k * m
        g_["dk"][:, t] = (np.einsum("bhij,bhi->bhj", dst, cs) + np.einsum("bhij,bhi->bhj", drt, cr)
                          - np.einsum("bhij,bhi->bhj", sp, des) - np.einsum("bhij,bhi->bhj", rp, der))
        g_["dalpha"][:, t] = (dst * sp).sum(axis=(2, 3)) + (drt * rp).sum(axis=(2, 3))
        g_["dbeta"][:, t] = (ds_k * cb).sum(axis=-1)
        g_["dgamma"][:, t] = (dr_k * cg).sum(axis=-1)
        dS = a[..., None] * dst - des[..., :, None] * kt[..., None, :]
        dR = a[..., None] * drt - der[..., :, None] * kt[..., None, :]
    return g_


DP_NORM_EPS = 1.0e-6  # fused_delta_product_scan.cu:38 (key L2 norm and output RMS norm)


def _dp_states(k, v, beta, t, S):
    """The n_h Householder sub-steps of token t from state S -> list of the n_h + 1 states
    (S before each sub-step, then after the last)."""
    kn = l2_normalize_keys(k[:, t])                     # [B, n_h, H, d]
    out = [S]
    for j in range(k.shape[2]):
        r = np.einsum("bhij,bhj->bhi", S, kn[:, j])
        err = beta[:, t, j][..., None] * (v[:, t, j] - r)
        S = S + err[..., :, None] * kn[:, j][..., None, :]
        out.append(S)
    return out


def delta_product(q, k, v, beta, return_raw=False):
    """DeltaProduct: n_h delta-rule (generalized Householder) sub-steps per token,
    then o_t = RMS_norm(contraction of S_t with q_t).

    q [B,T,H,d]; k, v [B,T,n_h,H,d]; beta [B,T,n_h,H] (post-sigmoid, one gate per head
    and sub-step).  Each sub-step normalizes its key, kn = k / sqrt(|k|^2 + 1e-6), and
    applies S = S + beta (v - S kn) kn^T with S [H, d_v, d_k] as in ``delta_rule``.  The
    reference keeps the transpose S_ref[key][value] and outputs S_ref q
    (fused_delta_product_scan.cu:94-271 and 274-299; ``delta_product_scan_fallback``,
    delta_product.ex:287-347), which here contracts the VALUE rows:
    o_raw[j] = sum_i S[i][j] q[i]; out = o_raw / sqrt(mean(o_raw^2) + 1e-6).
    """
    q, k, v, beta = _f64(q, k, v, beta)
    bsz, seq, nh, d = q.shape
    S = np.zeros((bsz, nh, v.shape[-1], k.shape[-1]))
    raw = np.empty((bsz, seq, nh, k.shape[-1]))
    for t in range(seq):
        S = _dp_states(k, v, beta, t, S)[-1]
        raw[:, t] = np.einsum("bhij,bhi->bhj", S, q[:, t])
    out = raw / np.sqrt((raw * raw).mean(axis=-1, keepdims=True) + DP_NORM_EPS)
    return (out, raw) if return_raw else out


def delta_product_backward(q, k, v, beta, do):
    """Reverse pass -> dict(dq [B,T,H,d], dk, dv [B,T,n_h,H,d], dbeta [B,T,n_h,H]).

    Per token t in reverse (structure of ``delta_product_backward_fallback``,
    fused_scan.ex:1947-2090, and fused_delta_product_scan_backward.cu:165-361):
      dO = do / r - o_raw (do . o_raw) / (d r^3)   (RMS norm; the fallback's o_raw / r^2
      factor drops the 1/r that the CUDA kernel keeps, fused_delta_product_scan_backward.cu:188-202)
      dq = S_t dO (contracts the key axis);  dS += q_t dO^T
      per sub-step j in reverse (S_p the state before it): err = v - S_p kn, ds_k = dS kn,
      dv = beta ds_k, dbeta = err . ds_k, dkn = dS^T (beta err) - S_p^T (beta ds_k),
      dk = (dkn - kn (dkn . kn)) / sqrt(|k|^2 + 1e-6),  dS <- dS - beta ds_k kn^T.
    """
    q, k, v, beta, do = _f64(q, k, v, beta, do)
    bsz, seq, nh, d = q.shape
    nhh = k.shape[2]
    S = np.zeros((bsz, nh, v.shape[-1], k.shape[-1]))
    per_tok = []
    for t in range(seq):
        sts = _dp_states(k, v, beta, t, S)
        per_tok.append(sts)
        S = sts[-1]
    dq = np.empty_like(q)
    dk = np.empty_like(k)
    dvv = np.empty_like(v)
    dbeta = np.empty_like(beta)
    dS = np.zeros_like(S)
    for t in range(seq - 1, -1, -1):
        sts = per_tok[t]
        st_ = sts[-1]
        raw = np.einsum("bhij,bhi->bhj", st_, q[:, t])
        r = np.sqrt((raw * raw).mean(axis=-1, keepdims=True) + DP_NORM_EPS)
        dO = do[:, t] / r - raw * (do[:, t] * raw).sum(axis=-1, keepdims=True) / (d * r ** 3)
        dq[:, t] = np.einsum("bhij,bhj->bhi", st_, dO)
        dS = dS + q[:, t][..., :, None] * dO[..., None, :]
        kraw = k[:, t]
        nrm = np.sqrt((kraw * kraw).sum(axis=-1, keepdims=True) + DP_NORM_EPS)
        kn = kraw / nrm
        for j in range(nhh - 1, -1, -1):
            sp, bt, knj = sts[j], beta[:, t, j][..., None], kn[:, j]
            err = v[:, t, j] - np.einsum("bhij,bhj->bhi", sp, knj)
            ds_k = np.einsum("bhij,bhj->bhi", dS, knj)
            dvv[:, t, j] = bt * ds_k
            dbeta[:, t, j] = (err * ds_k).sum(axis=-1)
            dkn = (np.einsum("bhij,bhi->bhj", dS, bt * err)
                   - np.einsum("bhij,bhi->bhj", sp, bt * ds_k))
            dk[:, t, j] = (dkn - knj * (dkn * knj).sum(axis=-1, keepdims=True)) / nrm[:, j]
            dS = dS - (bt * ds_k)[..., :, None] * knj[..., None, :]
    return dict(dq=dq, dk=dk, dv=dvv, dbeta=dbeta)


# ---------------------------------------------------------------------------
# Flash attention
# ---------------------------------------------------------------------------

def _scores(q, k, causal):
    d = q.shape[-1]
    s = np.einsum("bhid,bhjd->bhij", q, k) / np.sqrt(d)
    if causal:
        tq, tk = s.shape[-2:]
        mask = np.arange(tq)[:, None] >= np.arange(tk)[None, :]
        s = np.where(mask, s, -np.inf)
    return s


def flash_attention(q, k, v, causal=False, return_lse=False):
    """softmax(Q K^T / sqrt(d) + causal -inf) V (fused_scan.ex:3476-3508).

    Causal mask keeps key j <= query i (rows >= cols).  Optionally also returns the
    row log-sum-exp of the scaled scores (natural log).
    """
    q, k, v = _f64(q, k, v)
    s = _scores(q, k, causal)
    m = s.max(axis=-1, keepdims=True)
    w = np.exp(s - m)
    l = w.sum(axis=-1, keepdims=True)
    o = np.einsum("bhij,bhjd->bhid", w / l, v)
    if return_lse:
        return o, (m + np.log(l))[..., 0]
    return o


def flash_attention_backward(q, k, v, do, causal=False):
    """-> (dq, dk, dv) following ``flash_attention_backward_fallback`` (fused_scan.ex:3527-3570)."""
    q, k, v, do = _f64(q, k, v, do)
    d = q.shape[-1]
    s = _scores(q, k, causal)
    w = np.exp(s - s.max(axis=-1, keepdims=True))
    w = w / w.sum(axis=-1, keepdims=True)
    dv = np.einsum("bhij,bhid->bhjd", w, do)
    dw = np.einsum("bhid,bhjd->bhij", do, v)
    ds = w * (dw - (dw * w).sum(axis=-1, keepdims=True)) / np.sqrt(d)
    dq = np.einsum("bhij,bhjd->bhid", ds, k)
    dk = np.einsum("bhij,bhid->bhjd", ds, q)
    return dq, dk, dv


# ---------------------------------------------------------------------------
# FoX (forgetting) attention
# ---------------------------------------------------------------------------

def _fox_scores(q, k, cs):
    """Q K^T / sqrt(d) + (cs_i - cs_j), causal (fused_scan.ex:3860-3900; the diagonal
    bias the reference zeroes explicitly is cs_i - cs_i = 0)."""
    s = _scores(q, k, True)
    return s + (cs[..., :, None] - cs[..., None, :])


def fox_attention(q, k, v, cs, return_lse=False):
    """softmax(Q K^T / sqrt(d) + cs_i - cs_j, causal) V (``fox_attention_fallback``,
    fused_scan.ex:3860-3907; kernel native/cuda/fused_fox_attention.cu:1-14)."""
    q, k, v, cs = _f64(q, k, v, cs)
    s = _fox_scores(q, k, cs)
    m = s.max(axis=-1, keepdims=True)
    w = np.exp(s - m)
    l = w.sum(axis=-1, keepdims=True)
    o = np.einsum("bhij,bhjd->bhid", w / l, v)
    if return_lse:
        return o, (m + np.log(l))[..., 0]
    return o


def fox_attention_backward(q, k, v, cs, do):
    """-> (dq, dk, dv, dcs) following ``fox_attention_backward_fallback``
    (fused_scan.ex:3926-3984): the attention backward with the bias, and
    dcs_i = sum_j dS_ij - sum_j dS_ji (dS the gradient of the biased scores)."""
    q, k, v, cs, do = _f64(q, k, v, cs, do)
    d = q.shape[-1]
    s = _fox_scores(q, k, cs)
    w = np.exp(s - s.max(axis=-1, keepdims=True))
    w = w / w.sum(axis=-1, keepdims=True)
    dv = np.einsum("bhij,bhid->bhjd", w, do)
    dw = np.einsum("bhid,bhjd->bhij", do, v)
    g = w * (dw - (dw * w).sum(axis=-1, keepdims=True))
    dq = np.einsum("bhij,bhjd->bhid", g, k) / np.sqrt(d)
    dk = np.einsum("bhij,bhid->bhjd", g, q) / np.sqrt(d)
    dcs = g.sum(axis=-1) - g.sum(axis=-2)
    return dq, dk, dv, dcs


# ---------------------------------------------------------------------------
# LASER attention
# ---------------------------------------------------------------------------

LASER_CLAMP = 1.0e-7  # fused_scan.ex:3703


def laser_attention(q, k, v, causal=True):
    """log(max(softmax(Q K^T / sqrt(d)) exp(V - vmax), 1e-7)) + vmax, vmax the per-column
    max of V over the sequence (``laser_attention`` / ``laser_attention_fallback``,
    fused_scan.ex:3593-3600, 3667-3704)."""
    q, k, v = _f64(q, k, v)
    vmax = v.max(axis=2, keepdims=True)
    s = _scores(q, k, causal)
    w = np.exp(s - s.max(axis=-1, keepdims=True))
    w = w / w.sum(axis=-1, keepdims=True)
    return np.log(np.maximum(w @ np.exp(v - vmax), LASER_CLAMP)) + vmax


def laser_attention_backward(q, k, v, do, causal=True):
    """-> (dq, dk, dv) following ``laser_attention_backward_fallback`` (fused_scan.ex:3720-3771):
    dR = dO exp(vmax - O), dV = (P^T dR) exp(V - vmax), dS from dR exp(V - vmax)^T; vmax is
    held constant."""
    q, k, v, do = _f64(q, k, v, do)
    d = q.shape[-1]
    vmax = v.max(axis=2, keepdims=True)
    ev = np.exp(v - vmax)
    s = _scores(q, k, causal)
    w = np.exp(s - s.max(axis=-1, keepdims=True))
    w = w / w.sum(axis=-1, keepdims=True)
    o = np.log(np.maximum(w @ ev, LASER_CLAMP)) + vmax
    dr = do * np.exp(vmax - o)
    dv = np.einsum("bhij,bhid->bhjd", w, dr) * ev
    dw = np.einsum("bhid,bhjd->bhij", dr, ev)
    ds = w * (dw - (dw * w).sum(axis=-1, keepdims=True)) / np.sqrt(d)
    dq = np.einsum("bhij,bhjd->bhid", ds, k)
    dk = np.einsum("bhij,bhid->bhjd", ds, q)
    return dq, dk, dv

