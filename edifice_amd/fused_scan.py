"""Host-side mirror of ``Edifice.CUDA.FusedScan`` (lib/edifice/cuda/fused_scan.ex).

Same op names, argument order and meaning as the Elixir module; tensors are torch
tensors resident on the GPU (the role Nx/EXLA device buffers play in the
reference).  Each op launches the HIP kernel through the C ABI on torch's current
stream and is differentiable: the backward is the fused HIP backward kernel,
which the reference only wires through ``Nx.Defn.Kernel.custom_grad``
(e.g. fused_scan.ex:474-480, 2205-2209, 2606-2611, 3438-3442).

There is no CPU or eager fallback: CPU tensors, unsupported dtypes or a missing
library raise ``EdificeHipError`` (the reference's fallback tier is the parity
oracle in ``oracle/``, which the product never calls).
"""
from __future__ import annotations

import ctypes

import torch
import torch.nn.functional as F

from . import _native as nat
from ._native import EdificeHipError

F32, BF16 = 0, 1
_DT = {torch.float32: F32, torch.bfloat16: BF16}
SS_DT_PER_CHANNEL, SS_DT_MEAN = 0, 1
SS_DT_SOFTPLUS = 2  # mode flag: dt is the pre-activation, the kernels take softplus(dt)


def dtype_flag(t: torch.Tensor) -> int:
    """0 = f32, 1 = bf16, as ``dtype_flag/1`` (fused_scan.ex:39-44); other dtypes raise."""
    try:
        return _DT[t.dtype]
    except KeyError:
        raise EdificeHipError(f"unsupported dtype {t.dtype} (float32 or bfloat16)") from None


def _dev(*ts):
    for t in ts:
        if t is None:
            continue
        if not t.is_cuda:
            raise EdificeHipError("edifice_amd ops need GPU tensors (no CPU fallback)")
        if not t.is_contiguous():
            raise EdificeHipError("edifice_amd ops need contiguous tensors")


def _p(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _same(dtype_of, *ts):
    for t in ts:
        if t is not None and t.dtype != dtype_of.dtype:
            raise EdificeHipError(f"dtype mismatch: {t.dtype} vs {dtype_of.dtype}")


def _c(t):
    return None if t is None else t.contiguous()


def _shape(name, t, want):
    """Raise before any launch when ``t`` is not of shape ``want``: the kernels index every
    operand by the leading tensor's sizes, so a mismatch would read or write out of bounds."""
    if t is not None and tuple(t.shape) != tuple(want):
        raise EdificeHipError(f"{name} must have shape {tuple(want)}, got {tuple(t.shape)}")


def _rank(name, t, ndim):
    if t.dim() != ndim:
        raise EdificeHipError(f"{name} must be {ndim}-d, got shape {tuple(t.shape)}")


# ---------------------------------------------------------------------------
# MinGRU / MinLSTM
# ---------------------------------------------------------------------------

class _MinGRU(torch.autograd.Function):
    @staticmethod
    def forward(ctx, gates, cand):
        gates, cand = gates.contiguous(), cand.contiguous()
        _rank("gates", gates, 3)
        _shape("candidates", cand, gates.shape)
        _dev(gates, cand)
        _same(gates, cand)
        bsz, seq, hid = gates.shape
        out = torch.empty_like(gates)
        nat.call("edf_mingru", _stream(), _p(gates), _p(cand), _p(out), bsz, seq, hid, dtype_flag(gates))
        ctx.save_for_backward(gates, cand, out)
        return out

    @staticmethod
    def backward(ctx, dy):
        gates, cand, out = ctx.saved_tensors
        dy = dy.contiguous().to(gates.dtype)
        bsz, seq, hid = gates.shape
        dg = torch.empty_like(gates)
        dc = torch.empty_like(cand)
        nat.call("edf_mingru_backward", _stream(), _p(gates), _p(cand), _p(out), _p(dy), _p(dg), _p(dc),
                 bsz, seq, hid, dtype_flag(gates))
        return dg, dc


def mingru(gates: torch.Tensor, candidates: torch.Tensor) -> torch.Tensor:
    """``FusedScan.mingru/2`` (fused_scan.ex:60-74): gate logits [B,T,H], candidates [B,T,H].

    z = sigmoid(gates) is fused into the kernel; h0 = 0; returns all hidden states.
    """
    return _MinGRU.apply(gates, candidates)


class _MinLSTM(torch.autograd.Function):
    @staticmethod
    def forward(ctx, fg, ig, cand):
        fg, ig, cand = fg.contiguous(), ig.contiguous(), cand.contiguous()
        _rank("forget_gates", fg, 3)
        _shape("input_gates", ig, fg.shape)
        _shape("candidates", cand, fg.shape)
        _dev(fg, ig, cand)
        _same(fg, ig, cand)
        bsz, seq, hid = fg.shape
        out = torch.empty_like(fg)
        nat.call("edf_minlstm", _stream(), _p(fg), _p(ig), _p(cand), _p(out), bsz, seq, hid, dtype_flag(fg))
        ctx.save_for_backward(fg, ig, cand, out)
        return out

    @staticmethod
    def backward(ctx, dy):
        fg, ig, cand, out = ctx.saved_tensors
        dy = dy.contiguous().to(fg.dtype)
        bsz, seq, hid = fg.shape
        df, di, dc = torch.empty_like(fg), torch.empty_like(ig), torch.empty_like(cand)
        nat.call("edf_minlstm_backward", _stream(), _p(fg), _p(ig), _p(cand), _p(out), _p(dy), _p(df), _p(di),
                 _p(dc), bsz, seq, hid, dtype_flag(fg))
        return df, di, dc


def minlstm(forget_gates: torch.Tensor, input_gates: torch.Tensor, candidates: torch.Tensor) -> torch.Tensor:
    """``FusedScan.minlstm/3`` (fused_scan.ex:77-91): gate logits, sigmoids fused, h0 = 0."""
    return _MinLSTM.apply(forget_gates, input_gates, candidates)


# ---------------------------------------------------------------------------
# Generic linear scan
# ---------------------------------------------------------------------------

class _LinearScan(torch.autograd.Function):
    @staticmethod
    def forward(ctx, a, b):
        a, b = a.contiguous(), b.contiguous()
        _dev(a, b)
        _same(a, b)
        bsz, seq, hid = a.shape
        if b.shape != a.shape:
            raise EdificeHipError(f"shape mismatch: a {tuple(a.shape)} vs b {tuple(b.shape)}")
        out = torch.empty_like(a)
        nat.call("edf_fused_linear_scan", _stream(), _p(a), _p(b), None, _p(out), bsz, seq, hid, dtype_flag(a))
        ctx.save_for_backward(a, out)
        return out

    @staticmethod
    def backward(ctx, dy):
        a, out = ctx.saved_tensors
        da, db, _ = linear_scan_backward(a, None, out, dy.contiguous().to(a.dtype))
        return da, db


def linear_scan(a_vals: torch.Tensor, b_vals: torch.Tensor) -> torch.Tensor:
    """``FusedScan.linear_scan/2`` (fused_scan.ex:171-185): h_t = a_t h_{t-1} + b_t, h0 = 0.

    a_vals, b_vals: [B, T, H] precomputed coefficients (no activation inside);
    returns all hidden states.  The backward is the fused reverse scan
    (``linear_scan_backward``), as the reference's custom_grad (fused_scan.ex:834-849).
    """
    return _LinearScan.apply(a_vals, b_vals)


def linear_scan_backward(a_vals, h0, forward_out, grad_output):
    """``linear_scan_backward_fallback/4`` (fused_scan.ex:884-915) on the GPU -> (da, db, dh0).

    h0 may be None (zeros).  da = dh h_{t-1}, db = dh, dh0 = a_0 dh_0.
    """
    a_vals, forward_out, grad_output = a_vals.contiguous(), forward_out.contiguous(), grad_output.contiguous()
    h0 = _c(h0)
    _dev(a_vals, h0, forward_out, grad_output)
    _same(a_vals, h0, forward_out, grad_output)
    bsz, seq, hid = a_vals.shape
    da, db = torch.empty_like(a_vals), torch.empty_like(a_vals)
    dh0 = torch.empty((bsz, hid), dtype=a_vals.dtype, device=a_vals.device)
    nat.call("edf_fused_linear_scan_backward", _stream(), _p(a_vals), _p(h0), _p(forward_out), _p(grad_output),
             _p(da), _p(db), _p(dh0), bsz, seq, hid, dtype_flag(a_vals))
    return da, db, dh0


_BLOCK_PROJ = {"mingru": 2, "minlstm": 3, "linear": 2}


def _block(kind, input, weights, h0, num_layers):
    input, weights = input.contiguous(), weights.contiguous()
    h0 = _c(h0)
    _dev(input, weights, h0)
    _same(input, weights, h0)
    bsz, seq, hid = input.shape
    per_layer = _BLOCK_PROJ[kind] * (hid * hid + hid) + 2 * hid
    if weights.numel() != num_layers * per_layer:
        raise EdificeHipError(f"weights hold {weights.numel()} values, expected {num_layers} x {per_layer}")
    if h0 is not None and tuple(h0.shape) != (bsz, num_layers, hid):
        raise EdificeHipError(f"h0 must be [B, num_layers, H] = {(bsz, num_layers, hid)}")
    out = torch.empty_like(input)
    flag = dtype_flag(input)
    wsb = nat.query(f"edf_{kind}_block_workspace_bytes", bsz, seq, hid, num_layers, flag)
    ws = _u8(wsb, input)
    nat.call(f"edf_fused_{kind}_block_scan", _stream(), _p(input), _p(weights), _p(h0), _p(out), _p(ws), wsb,
             bsz, seq, hid, num_layers, flag)
    return out


def mingru_block(input, weights, h0, num_layers: int):
    """``FusedScan.mingru_block/4`` (fused_scan.ex:4465-4479): multi-layer MinGRU inference.

    input [B, T, H]; weights the flat per-layer packing of min_gru.ex:217-241
    (W_z [H][H] input-major, b_z, W_h, b_h, gamma, beta) in input's dtype; h0
    [B, num_layers, H] or None (zeros); H <= 256.  Returns the last layer's output
    [B, T, H].  Inference only (the reference has no backward for it).
    """
    return _block("mingru", input, weights, h0, num_layers)


def minlstm_block(input, weights, h0, num_layers: int):
    """``FusedScan.minlstm_block/4`` (fused_scan.ex:4591-4605): as ``mingru_block`` with
    three projections per layer (W_f, b_f, W_i, b_i, W_h, b_h, gamma, beta)."""
    return _block("minlstm", input, weights, h0, num_layers)


def linear_block(input, weights, h0, num_layers: int):
    """``FusedScan.linear_block/4`` (fused_scan.ex:4729-4743): projections a, b per layer
    (W_a, b_a, W_b, b_b, gamma, beta), h = a h + b, residual."""
    return _block("linear", input, weights, h0, num_layers)


_RNN_GATES = {"lstm": 4, "gru": 3}


def _rnn_block(kind, input, weights, h0, c0, num_layers):
    input, weights = input.contiguous(), weights.contiguous()
    h0, c0 = _c(h0), _c(c0)
    _dev(input, weights, h0, c0)
    _same(input, weights, h0, c0)
    bsz, seq, hid = input.shape
    gh = _RNN_GATES[kind] * hid
    per_layer = 2 * hid * gh + gh + 2 * hid
    if weights.numel() != num_layers * per_layer:
        raise EdificeHipError(f"weights hold {weights.numel()} values, expected {num_layers} x {per_layer}")
    for name, t in (("h0", h0), ("c0", c0)):
        if t is not None and tuple(t.shape) != (bsz, num_layers, hid):
            raise EdificeHipError(f"{name} must be [B, num_layers, H] = {(bsz, num_layers, hid)}")
    out = torch.empty_like(input)
    flag = dtype_flag(input)
    wsb = nat.query(f"edf_{kind}_block_workspace_bytes", bsz, seq, hid, num_layers, flag)
    ws = _u8(wsb, input)
    if kind == "lstm":
        nat.call("edf_fused_lstm_block_scan", _stream(), _p(input), _p(weights), _p(h0), _p(c0), _p(out), _p(ws),
                 wsb, bsz, seq, hid, num_layers, flag)
    else:
        nat.call("edf_fused_gru_block_scan", _stream(), _p(input), _p(weights), _p(h0), _p(out), _p(ws), wsb,
                 bsz, seq, hid, num_layers, flag)
    # a grid barrier that gave up raises here (the output then holds NaN); waits for the stream
    nat.call(f"edf_{kind}_block_status", _stream(), _p(ws), wsb, bsz, seq, hid, num_layers)
    return out


def lstm_block(input, weights, h0, c0, num_layers: int):
    """``FusedScan.lstm_block/5`` (fused_scan.ex:4854-4868): multi-layer LSTM inference.

    input [B, T, H]; weights the flat per-layer packing W_x [H, 4H] (gates i, f, g, o), b_x
    [4H], R [H, 4H], gamma [H], beta [H] in input's dtype; h0, c0 [B, num_layers, H] or None
    (zeros); H <= 256.  Returns the last layer's output [B, T, H].
    """
    return _rnn_block("lstm", input, weights, h0, c0, num_layers)


def gru_block(input, weights, h0, num_layers: int):
    """``FusedScan.gru_block/4`` (fused_scan.ex:4999-5013): multi-layer GRU inference, gates
    r, z, n (W_x [H, 3H], b_x [3H], R [H, 3H], gamma, beta per layer), h = (1 - z) h + z n."""
    return _rnn_block("gru", input, weights, h0, None, num_layers)


# ---------------------------------------------------------------------------
# Causal depthwise conv1d + SiLU (block callers)
# ---------------------------------------------------------------------------

def _conv_operands(x, weight, bias):
    if x.dim() != 3 or x.stride(2) != 1:
        raise EdificeHipError(f"x must be [B, T, C] with contiguous channels, got shape {tuple(x.shape)}")
    bsz, seq, ch = x.shape
    # The kernels address row (b, t) at (b * seq + t) * row_stride: every row equally spaced,
    # across batch elements too.  With one step the batch stride is the row stride; a size-1
    # dimension's stride carries no meaning and is not used.
    row_stride = x.stride(1) if seq > 1 else (x.stride(0) if bsz > 1 else ch)
    if row_stride < ch or (seq > 1 and bsz > 1 and x.stride(0) != seq * row_stride):
        x = x.contiguous()
        row_stride = ch
    w = weight.reshape(weight.shape[0], -1).contiguous()
    _shape("weight", w, (ch, w.shape[1]))
    b = _c(bias)
    _shape("bias", b, (ch,))
    _dev(w, b)
    if not x.is_cuda:
        raise EdificeHipError("edifice_amd ops need GPU tensors (no CPU fallback)")
    _same(x, w, b)
    return x, w, b, bsz, seq, ch, w.shape[1], row_stride


class _CausalConvSilu(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, weight, bias):
        x, w, b, bsz, seq, ch, k, xs = _conv_operands(x, weight, bias)
        out = torch.empty((bsz, seq, ch), dtype=x.dtype, device=x.device)
        nat.call("edf_causal_conv1d_silu", _stream(), _p(x), xs, _p(w), _p(b), _p(out), bsz, seq, ch, k,
                 dtype_flag(x))
        ctx.save_for_backward(x, w, b)
        ctx.wshape, ctx.has_bias, ctx.row_stride = weight.shape, bias is not None, xs
        return out

    @staticmethod
    def backward(ctx, dy):
        x, w, b = ctx.saved_tensors
        bsz, seq, ch = x.shape
        k = w.shape[1]
        xs = ctx.row_stride
        dy = dy.contiguous().to(x.dtype)
        dx = torch.empty((bsz, seq, ch), dtype=x.dtype, device=x.device)
        dw = torch.empty_like(w)
        db = torch.empty_like(b) if ctx.has_bias else None
        wsb = nat.query("edf_causal_conv1d_silu_backward_workspace_bytes", bsz, seq, ch, k)
        ws = torch.empty(wsb, dtype=torch.uint8, device=x.device)
        nat.call("edf_causal_conv1d_silu_backward", _stream(), _p(x), xs, _p(w), _p(b), _p(dy), _p(dx), _p(dw),
                 _p(db), _p(ws), wsb, bsz, seq, ch, k, dtype_flag(x))
        return dx, dw.reshape(ctx.wshape), db


def causal_conv1d_silu(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor = None) -> torch.Tensor:
    """silu(causal depthwise conv1d(x)) over time: the Mamba block's x branch
    (common.ex:251-252, ``build_depthwise_conv1d`` common.ex:298-309) and the GatedDeltaNet
    short convolution (gated_delta_net.ex:239-245).

    x: [B, T, C] with contiguous channels (a column slice of a wider projection is read in
    place); weight: nn.Conv1d's [C, 1, K] (or [C, K]); bias: [C] or None; one dtype.
    y[t] = silu(bias + sum_j w[j] x[t - (K - 1) + j]), x = 0 before t = 0, f32 inside.
    """
    return _CausalConvSilu.apply(x, weight, bias)


# ---------------------------------------------------------------------------
# Softmax cross entropy (block callers' loss)
# ---------------------------------------------------------------------------

class _CrossEntropy(torch.autograd.Function):
    @staticmethod
    def forward(ctx, logits, targets):
        logits, targets = logits.contiguous(), targets.contiguous()
        _dev(logits, targets)
        _rank("logits", logits, 2)
        rows, vocab = logits.shape
        _shape("targets", targets, (rows,))
        if targets.dtype != torch.int64:
            raise EdificeHipError(f"targets must be int64, got {targets.dtype}")
        loss_rows = torch.empty(rows, dtype=torch.float32, device=logits.device)
        lse = torch.empty(rows, dtype=torch.float32, device=logits.device)
        nat.call("edf_cross_entropy", _stream(), _p(logits), _p(targets), _p(loss_rows), _p(lse), rows, vocab,
                 dtype_flag(logits))
        ctx.save_for_backward(logits, targets, lse)
        return loss_rows.mean()

    @staticmethod
    def backward(ctx, grad):
        logits, targets, lse = ctx.saved_tensors
        rows, vocab = logits.shape
        grad = grad.reshape(1).to(torch.float32).contiguous()
        dlogits = torch.empty_like(logits)
        nat.call("edf_cross_entropy_backward", _stream(), _p(logits), _p(targets), _p(lse), _p(grad), 1.0 / rows,
                 _p(dlogits), rows, vocab, dtype_flag(logits))
        return dlogits, None


def cross_entropy(logits: torch.Tensor, targets: torch.Tensor) -> torch.Tensor:
    """Mean softmax cross entropy of ``logits`` [N, V] (float32 or bfloat16, reduced in float32)
    against int64 ``targets`` [N]: the decoder models' next-token loss, as
    ``F.cross_entropy(logits.float(), targets)`` computes it, without a float32 copy of the
    logits or of their gradient.  Targets outside [0, V) contribute 0 (the mean still divides
    by N)."""
    return _CrossEntropy.apply(logits, targets)


# ---------------------------------------------------------------------------
# Layer normalisation (block callers' pre-norms and final norms)
# ---------------------------------------------------------------------------

class _LayerNorm(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, weight, bias, eps):
        x, weight, bias = _c(x), _c(weight), _c(bias)
        _dev(x, weight, bias)
        cols = x.shape[-1]
        rows = x.numel() // max(cols, 1)
        for name, t in (("weight", weight), ("bias", bias)):
            if t is not None:
                _shape(name, t, (cols,))
        if weight is not None and bias is not None:
            _same(weight, bias)
        pt = weight if weight is not None else bias
        y = torch.empty_like(x)
        mean = torch.empty(rows, dtype=torch.float32, device=x.device)
        rstd = torch.empty(rows, dtype=torch.float32, device=x.device)
        nat.call("edf_layer_norm", _stream(), _p(x), _p(weight), _p(bias), _p(y), _p(mean), _p(rstd), rows, cols,
                 float(eps), dtype_flag(x), dtype_flag(pt) if pt is not None else dtype_flag(x))
        ctx.save_for_backward(x, weight, mean, rstd)
        ctx.has_bias = bias is not None
        ctx.pdtype = pt.dtype if pt is not None else x.dtype
        return y

    @staticmethod
    def backward(ctx, dy):
        x, weight, mean, rstd = ctx.saved_tensors
        cols = x.shape[-1]
        rows = x.numel() // max(cols, 1)
        dy = dy.contiguous().to(x.dtype)
        dx = torch.empty_like(x)
        dw = torch.empty(cols, dtype=ctx.pdtype, device=x.device) if weight is not None else None
        db = torch.empty(cols, dtype=ctx.pdtype, device=x.device) if ctx.has_bias else None
        wsb = nat.query("edf_layer_norm_backward_workspace_bytes", rows, cols)
        ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device=x.device)
        pflag = F32 if ctx.pdtype == torch.float32 else BF16
        nat.call("edf_layer_norm_backward", _stream(), _p(x), _p(weight), _p(mean), _p(rstd), _p(dy), _p(dx),
                 _p(dw), _p(db), _p(ws), wsb, rows, cols, dtype_flag(x), pflag)
        return dx, dw, db, None


def layer_norm(x: torch.Tensor, weight: torch.Tensor = None, bias: torch.Tensor = None,
               eps: float = 1e-5) -> torch.Tensor:
    """Layer normalisation over the last dimension, ``F.layer_norm(x, (C,), weight, bias, eps)``
    (biased variance, eps inside the square root): the block models' pre-norms and final norms
    (Axon.layer_norm, e.g. common.ex:224, delta_net.ex:159,199, model_builder.ex:111,165).
    x float32 or bfloat16 with C <= 8192 columns; weight / bias [C] (float32 or bfloat16, one
    dtype) or None; statistics and arithmetic in float32."""
    return _LayerNorm.apply(x, weight, bias, eps)


class _AddLayerNorm(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, res, weight, bias, eps):
        x, res, weight, bias = _c(x), _c(res), _c(weight), _c(bias)
        _dev(x, res, weight, bias)
        _same(x, res)
        if x.shape != res.shape:
            raise EdificeHipError(f"add_layer_norm: x {tuple(x.shape)} and res {tuple(res.shape)} differ")
        cols = x.shape[-1]
        rows = x.numel() // max(cols, 1)
        for name, t in (("weight", weight), ("bias", bias)):
            if t is not None:
                _shape(name, t, (cols,))
        if weight is not None and bias is not None:
            _same(weight, bias)
        pt = weight if weight is not None else bias
        total, y = torch.empty_like(x), torch.empty_like(x)
        mean = torch.empty(rows, dtype=torch.float32, device=x.device)
        rstd = torch.empty(rows, dtype=torch.float32, device=x.device)
        nat.call("edf_add_layer_norm", _stream(), _p(x), _p(res), _p(total), _p(weight), _p(bias), _p(y), _p(mean),
                 _p(rstd), rows, cols, float(eps), dtype_flag(x), dtype_flag(pt) if pt is not None else dtype_flag(x))
        ctx.save_for_backward(total, weight, mean, rstd)
        ctx.has_bias = bias is not None
        ctx.pdtype = pt.dtype if pt is not None else x.dtype
        ctx.set_materialize_grads(False)
        return total, y

    @staticmethod
    def backward(ctx, dtotal, dy):
        total, weight, mean, rstd = ctx.saved_tensors
        cols = total.shape[-1]
        rows = total.numel() // max(cols, 1)
        if dy is None:  # the normalised output unused: the sum's gradient passes through
            dx = torch.zeros_like(total) if dtotal is None else dtotal
            zp = (lambda on: torch.zeros(cols, dtype=ctx.pdtype, device=total.device) if on else None)
            return dx, dx, zp(weight is not None), zp(ctx.has_bias), None
        dy = dy.contiguous().to(total.dtype)
        ga = None if dtotal is None else dtotal.contiguous().to(total.dtype)
        dx = torch.empty_like(total)
        dw = torch.empty(cols, dtype=ctx.pdtype, device=total.device) if weight is not None else None
        db = torch.empty(cols, dtype=ctx.pdtype, device=total.device) if ctx.has_bias else None
        wsb = nat.query("edf_layer_norm_backward_workspace_bytes", rows, cols)
        ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device=total.device)
        pflag = F32 if ctx.pdtype == torch.float32 else BF16
        nat.call("edf_layer_norm_backward_add", _stream(), _p(total), _p(weight), _p(mean), _p(rstd), _p(dy), _p(ga),
                 _p(dx), _p(dw), _p(db), _p(ws), wsb, rows, cols, dtype_flag(total), pflag)
        return dx, dx, dw, db, None


def add_layer_norm(x: torch.Tensor, res: torch.Tensor, weight: torch.Tensor = None, bias: torch.Tensor = None,
                   eps: float = 1e-5):
    """(s, layer_norm(s)) with s = x + res: a pre-norm block stack's residual add and the next
    block's norm in one pass (the residual adds of transformer_block.ex:118,144 and
    common.ex:119 followed by Axon.layer_norm).  s is rounded to x's dtype as a separate add
    stores it; the backward adds the gradient reaching s through the residual path into the
    normalisation's input gradient in the same pass.  Shapes and dtypes as ``layer_norm``."""
    return _AddLayerNorm.apply(x, res, weight, bias, eps)


def softplus_forward(x: torch.Tensor) -> torch.Tensor:
    """softplus(x) by the HIP kernel, no autograd (``x`` made contiguous)."""
    x = x.contiguous()
    _dev(x)
    y = torch.empty_like(x)
    if x.numel():
        nat.call("edf_softplus", _stream(), _p(x), _p(y), x.numel(), dtype_flag(x))
    return y


def softplus_backward(x: torch.Tensor, dy: torch.Tensor) -> torch.Tensor:
    """dy sigmoid(x), the gradient of softplus at x (x contiguous, dy cast to x's dtype)."""
    dy = dy.contiguous().to(x.dtype)
    dx = torch.empty_like(x)
    if x.numel():
        nat.call("edf_softplus_backward", _stream(), _p(x), _p(dy), _p(dx), x.numel(), dtype_flag(x))
    return dx


class _Softplus(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x):
        x = x.contiguous()
        ctx.save_for_backward(x)
        return softplus_forward(x)

    @staticmethod
    def backward(ctx, dy):
        (x,) = ctx.saved_tensors
        return softplus_backward(x, dy)


def softplus(x: torch.Tensor) -> torch.Tensor:
    """log(1 + e^x) elementwise (float32 or bfloat16, f32 inside), ``F.softplus(x)``: the Mamba
    block's dt activation (Axon.activation(:softplus), common.ex:366)."""
    return _Softplus.apply(x)


class _L2Normalize(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, eps):
        x = x.contiguous()
        _dev(x)
        d = x.shape[-1]
        rows = x.numel() // max(d, 1)
        y = torch.empty_like(x)
        if x.numel():
            nat.call("edf_l2_normalize", _stream(), _p(x), _p(y), rows, d, float(eps), dtype_flag(x))
        ctx.save_for_backward(x)
        ctx.eps = eps
        return y

    @staticmethod
    def backward(ctx, dy):
        (x,) = ctx.saved_tensors
        d = x.shape[-1]
        rows = x.numel() // max(d, 1)
        dy = dy.contiguous().to(x.dtype)
        dx = torch.empty_like(x)
        if x.numel():
            nat.call("edf_l2_normalize_backward", _stream(), _p(x), _p(dy), _p(dx), rows, d, float(ctx.eps),
                     dtype_flag(x))
        return dx, None


def l2_normalize(x: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """x / sqrt(sum x^2 + eps) over the last dimension (<= 1024 elements; float32 or bfloat16,
    f32 inside): the DeltaNet / GatedDeltaNet key norm (delta_net.ex:291,
    gated_delta_net.ex:387)."""
    return _L2Normalize.apply(x, eps)


class _DeltaNetSplit(torch.autograd.Function):
    @staticmethod
    def forward(ctx, proj, num_heads, eps):
        proj = proj.contiguous()
        _dev(proj)
        *lead, width = proj.shape
        if width % (4 * num_heads):
            raise EdificeHipError(f"delta_net_split: last dimension {width} is not 4 x num_heads x head_dim")
        d = width // (4 * num_heads)
        rows = proj.numel() // max(width, 1)
        outs = [proj.new_empty(*lead, num_heads, d) for _ in range(4)]
        if rows:
            nat.call("edf_delta_net_split", _stream(), _p(proj), *(_p(t) for t in outs), rows, num_heads, d,
                     float(eps), dtype_flag(proj))
        ctx.save_for_backward(proj)
        ctx.num_heads, ctx.d, ctx.eps = num_heads, d, eps
        return tuple(outs)

    @staticmethod
    def backward(ctx, dq, dk, dv, db):
        (proj,) = ctx.saved_tensors
        rows = proj.numel() // max(proj.shape[-1], 1)
        g = [t.contiguous().to(proj.dtype) for t in (dq, dk, dv, db)]
        dproj = torch.empty_like(proj)
        if rows:
            nat.call("edf_delta_net_split_backward", _stream(), _p(proj), *(_p(t) for t in g), _p(dproj), rows,
                     ctx.num_heads, ctx.d, float(ctx.eps), dtype_flag(proj))
        return dproj, None, None


def delta_net_split(proj: torch.Tensor, num_heads: int, eps: float = 1e-6):
    """The DeltaNet layer's input split (delta_net.ex:274-300): proj [..., 4 H d] (the qkvb
    projection, q | k | v | beta_pre) -> q, k / sqrt(sum_d k^2 + eps), v, sigmoid(beta_pre),
    each [..., H, d], in one pass each way (float32 or bfloat16, f32 inside)."""
    return _DeltaNetSplit.apply(proj, num_heads, eps)


def _ptr_array(ts):
    arr = (ctypes.c_void_p * len(ts))(*[t.data_ptr() for t in ts])
    return ctypes.cast(arr, ctypes.c_void_p), arr


def _heads_split(x, parts, num_heads):
    bsz, seq, width = x.shape
    d = width // (parts * num_heads)
    outs = [x.new_empty(bsz, num_heads, seq, d) for _ in range(parts)]
    if x.numel():
        ptr, _keep = _ptr_array(outs)  # the host array lives until the call returns
        nat.call("edf_heads_split", _stream(), _p(x), ptr, bsz, seq, parts, num_heads, d, dtype_flag(x))
    return outs


def _heads_merge(ts):
    bsz, nh, seq, d = ts[0].shape
    y = ts[0].new_empty(bsz, seq, len(ts) * nh * d)
    if y.numel():
        ptr, _keep = _ptr_array(ts)
        nat.call("edf_heads_merge", _stream(), ptr, _p(y), bsz, seq, len(ts), nh, d, dtype_flag(y))
    return y


class _SplitHeads(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, parts, num_heads):
        x = x.contiguous()
        _dev(x)
        _rank("x", x, 3)
        if x.shape[-1] % (parts * num_heads):
            raise EdificeHipError(f"split_heads: last dimension {x.shape[-1]} is not parts x num_heads x head_dim")
        return tuple(_heads_split(x, parts, num_heads))

    @staticmethod
    def backward(ctx, *grads):
        g = [t.contiguous() for t in grads]
        _dev(*g)
        return _heads_merge(g), None, None


class _MergeHeads(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x):
        x = x.contiguous()
        _dev(x)
        _rank("x", x, 4)
        ctx.num_heads = x.shape[1]
        return _heads_merge([x])

    @staticmethod
    def backward(ctx, dy):
        return _heads_split(dy.contiguous(), 1, ctx.num_heads)[0]


def split_heads(x: torch.Tensor, parts: int, num_heads: int):
    """[B, T, P H d] (P stacked projections, e.g. q | k | v) -> P tensors [B, H, T, d], the
    attention kernels' layout, in one pass (and its backward in one pass): the attention
    blocks' head split (Nx reshape + transpose in the reference, e.g. transformer_block.ex:118)."""
    return _SplitHeads.apply(x, parts, num_heads)


def merge_heads(x: torch.Tensor) -> torch.Tensor:
    """[B, H, T, d] -> [B, T, H d], one pass each way: the attention output's head merge."""
    return _MergeHeads.apply(x)


class _Embedding(torch.autograd.Function):
    @staticmethod
    def forward(ctx, ids, weight, padding_idx):
        out = torch.nn.functional.embedding(ids, weight, padding_idx)
        ctx.save_for_backward(ids)
        ctx.vocab, ctx.padding_idx = weight.shape[0], padding_idx
        return out

    @staticmethod
    def backward(ctx, dy):
        (ids,) = ctx.saved_tensors
        dim = dy.shape[-1]
        g = dy.contiguous().reshape(-1, dim)
        flat = ids.contiguous().reshape(-1).to(torch.int64)
        _dev(g, flat)
        n = flat.numel()
        dw = g.new_empty(ctx.vocab, dim)
        wsb = nat.query("edf_embedding_backward_workspace_bytes", n, ctx.vocab)
        ws = _u8(wsb, g)
        pad = -1 if ctx.padding_idx is None else int(ctx.padding_idx) % ctx.vocab
        nat.call("edf_embedding_backward", _stream(), _p(flat), _p(g), _p(dw), _p(ws), wsb, n, ctx.vocab, dim, pad,
                 dtype_flag(g))
        return None, dw, None


def embedding(ids: torch.Tensor, weight: torch.Tensor, padding_idx: int = None) -> torch.Tensor:
    """``F.embedding(ids, weight, padding_idx)`` whose weight gradient is the HIP kernel
    (deterministic, every row written): the language models' token embedding (Axon.embedding,
    e.g. show_o.ex:123).  weight float32 or bfloat16; no max_norm / scale_grad_by_freq."""
    return _Embedding.apply(ids, weight, padding_idx)


def column_sum(x: torch.Tensor, out_dtype: torch.dtype = None, out: torch.Tensor = None) -> torch.Tensor:
    """Sum over the rows of a 2-D ``x`` (float32 or bfloat16, f32 inside, fixed order): the
    dense layers' bias gradients.  ``out``: a contiguous [cols] tensor to write (its dtype
    then decides the output type).  Not differentiable (a backward helper)."""
    x = x.contiguous()
    _dev(x)
    _rank("x", x, 2)
    rows, cols = x.shape
    if out is None:
        out = torch.empty(cols, dtype=out_dtype or x.dtype, device=x.device)
    elif out.shape != (cols,) or not out.is_contiguous() or out.dtype not in (torch.float32, torch.bfloat16):
        raise EdificeHipError(f"column_sum: out must be a contiguous [{cols}] float32 or bfloat16 tensor")
    else:
        _dev(x, out)
    wsb = nat.query("edf_column_sum_workspace_bytes", rows, cols)
    ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device=x.device)
    nat.call("edf_column_sum", _stream(), _p(x), _p(out), _p(ws), wsb, rows, cols, dtype_flag(x), dtype_flag(out))
    return out


# ---------------------------------------------------------------------------
# Selective scan
# ---------------------------------------------------------------------------

def _u8(nbytes, like):
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=like.device)


def selective_scan_forward(x, dt, A, B, C, D, z, mode, keep_states):
    """Run the fused selective scan (checked operands); returns (out, states), states the
    per-chunk float32 carries the backward reads (None unless ``keep_states``)."""
    x, dt, A, B, C, D, z = (_c(t) for t in (x, dt, A, B, C, D, z))
    _rank("x", x, 3)
    _rank("A", A, 2)
    bsz, seq, dim = x.shape
    n = A.shape[1]
    _shape("dt", dt, x.shape)
    _shape("z", z, x.shape)
    _shape("A", A, (dim, n))
    _shape("B", B, (bsz, seq, n))
    _shape("C", C, (bsz, seq, n))
    _shape("D", D, (dim,))
    _dev(x, dt, A, B, C, D, z)
    _same(x, dt, z)
    _same(A, B, C, D)
    io, par = dtype_flag(x), dtype_flag(A)
    out = torch.empty_like(x)
    states = None
    if keep_states:
        sb = nat.query("edf_selective_scan_states_bytes", bsz, seq, dim, n)
        states = torch.empty(sb // 4, dtype=torch.float32, device=x.device)
    wsb = nat.query("edf_selective_scan_workspace_bytes", bsz, seq, dim, n, mode)
    ws = _u8(wsb, x) if wsb else None
    nat.call("edf_fused_selective_scan", _stream(), _p(x), _p(dt), _p(A), _p(B), _p(C), _p(D), _p(z), _p(out),
             _p(states), _p(ws), wsb, bsz, seq, dim, n, io, par, mode)
    return out, states


def selective_scan_backward(x, dt, A, B, C, D, z, states, dout, mode):
    """Gradients of the fused selective scan for the operands of ``selective_scan_forward``:
    (dx, ddt, dA, dB, dC, dD, dz), dA / dB / dC / dD in float32, dD and dz None without D, z."""
    dout = dout.contiguous().to(x.dtype)
    bsz, seq, dim = x.shape
    n = A.shape[1]
    io, par = dtype_flag(x), dtype_flag(A)
    f32 = dict(dtype=torch.float32, device=x.device)
    dx, ddt = torch.empty_like(x), torch.empty_like(dt)
    dA = torch.empty((dim, n), **f32)
    dB = torch.empty((bsz, seq, n), **f32)
    dC = torch.empty((bsz, seq, n), **f32)
    dD = torch.empty((dim,), **f32) if D is not None else None
    dz = torch.empty_like(z) if z is not None else None
    wsb = nat.query("edf_selective_scan_backward_workspace_bytes", bsz, seq, dim, n, mode,
                    int(states is not None))
    ws = _u8(wsb, x)
    nat.call("edf_fused_selective_scan_backward", _stream(), _p(x), _p(dt), _p(A), _p(B), _p(C), _p(D), _p(z),
             _p(dout), _p(states), _p(dx), _p(ddt), _p(dA), _p(dB), _p(dC), _p(dD), _p(dz), _p(ws), wsb,
             bsz, seq, dim, n, io, par, mode)
    return dx, ddt, dA, dB, dC, dD, dz


class _SelectiveScan(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, dt, A, B, C, D, z, mode):
        x, dt, A, B, C, D, z = (_c(t) for t in (x, dt, A, B, C, D, z))
        out, states = selective_scan_forward(x, dt, A, B, C, D, z, mode, any(ctx.needs_input_grad[:7]))
        ctx.mode = mode
        ctx.save_for_backward(x, dt, A, B, C, D, z, states)
        return out

    @staticmethod
    def backward(ctx, dout):
        x, dt, A, B, C, D, z, states = ctx.saved_tensors
        dx, ddt, dA, dB, dC, dD, dz = selective_scan_backward(x, dt, A, B, C, D, z, states, dout, ctx.mode)
        cast = (lambda t, like: None if t is None else t.to(like.dtype))
        return dx, ddt, cast(dA, A), cast(dB, B), cast(dC, C), cast(dD, D), dz, None


def weight_grad(dy: torch.Tensor, x: torch.Tensor, out: torch.Tensor = None) -> torch.Tensor:
    """dW = dy^T x over k rows (into ``out``, a contiguous [m, n] tensor, when given).  For bf16
    with many rows and a small [m, n] output the product splits k into s slices, one batched
    product with float32 partials, summed and rounded once: a single [m, n] product over
    k = 16 384 has too few output tiles for the GPU (the config-5 model's 1024 x 1024 weight
    gradients: 97-110 µs as one product, 57 µs in 8 slices)."""
    k, m = dy.shape
    n = x.shape[1]
    s = 8 if m * n <= 1 << 20 else (4 if m * n <= 1 << 22 else 1)
    if s == 1 or dy.dtype != torch.bfloat16 or k % s or k // s < 1024:
        return dy.t().mm(x) if out is None else torch.mm(dy.t(), x, out=out)
    kc = k // s
    a = dy.reshape(s, kc, m).transpose(1, 2)
    b = x.reshape(s, kc, n).contiguous()  # the right operand stays a contiguous (non-transposed) tensor
    part = torch.bmm(a, b, out_dtype=torch.float32)
    # the s partials added in order and rounded to bf16 in one pass
    return column_sum(part.view(s, m * n), dy.dtype, out=None if out is None else out.view(m * n)).view(m, n)


def bias_grad(dy: torch.Tensor, out: torch.Tensor = None) -> torch.Tensor:
    """Sum of dy's rows (the bias gradient), into ``out`` when given: wide layers take the HIP
    column sum (torch's reduction reads [16384, 1024] bf16 at about 1.5 TB/s), narrow ones
    keep torch's."""
    if dy.is_cuda and dy.shape[1] >= 256:
        return column_sum(dy, out=out)
    r = dy.sum(0)
    return r if out is None else out.copy_(r)


class _MambaSSM(torch.autograd.Function):
    """The Mamba block between its conv and out_proj (common.ex:333-471): one product of xa
    over the stacked B / C and low-rank dt weights, B and C in float32, dt = softplus(dt_proj
    (low-rank dt)), then the fused selective scan in dt-mean mode with the SiLU(z) gate.
    One autograd node: the backward adds the projection's input gradient into the scan's
    (addmm) and assembles the projection's output gradient in one buffer, where separate
    torch ops would zero-fill and add a full-size gradient per slice."""

    @staticmethod
    def forward(ctx, xa, wcat, bcat, w_dt, b_dt, A, z, n_state):
        bsz, seq, inner = xa.shape
        x2 = xa.reshape(-1, inner)
        proj = F.linear(x2, wcat, bcat)  # [rows, 2 N + dt_rank]
        n2 = 2 * n_state
        b = proj[:, :n_state].float().contiguous().view(bsz, seq, n_state)
        c = proj[:, n_state:n2].float().contiguous().view(bsz, seq, n_state)
        # dt = softplus(dt_proj(.)) is applied inside the scan (mode flag): no dt tensor
        dt_pre = F.linear(proj[:, n2:], w_dt, b_dt).view(bsz, seq, inner)
        out, states = selective_scan_forward(xa, dt_pre, A, b, c, None, z, SS_DT_MEAN | SS_DT_SOFTPLUS, True)
        ctx.save_for_backward(xa, wcat, proj, w_dt, dt_pre, A, b, c, z, states)
        ctx.n_state, ctx.has_bcat, ctx.has_bdt = n_state, bcat is not None, b_dt is not None
        return out

    @staticmethod
    def backward(ctx, dout):
        xa, wcat, proj, w_dt, dt_pre, A, b, c, z, states = ctx.saved_tensors
        ns, n2 = ctx.n_state, 2 * ctx.n_state
        bsz, seq, inner = dt_pre.shape
        rows = bsz * seq
        dxa, ddt, dA, dB, dC, _, dz = selective_scan_backward(xa, dt_pre, A, b, c, None, z, states, dout,
                                                              SS_DT_MEAN | SS_DT_SOFTPLUS)
        ddt_pre = ddt.view(rows, inner)
        dproj = torch.empty_like(proj)
        dproj[:, :ns].copy_(dB.view(rows, ns))
        dproj[:, ns:n2].copy_(dC.view(rows, ns))
        dproj[:, n2:].copy_(ddt_pre.mm(w_dt))
        dxa.view(rows, inner).addmm_(dproj, wcat)
        need = ctx.needs_input_grad
        dwcat = weight_grad(dproj, xa.reshape(rows, inner)) if need[1] else None
        dbcat = bias_grad(dproj) if ctx.has_bcat and need[2] else None
        dw_dt = weight_grad(ddt_pre, proj[:, n2:]) if need[3] else None
        db_dt = bias_grad(ddt_pre) if ctx.has_bdt and need[4] else None
        dA = dA.to(A.dtype) if need[5] else None
        return dxa, dwcat, dbcat, dw_dt, db_dt, dA, dz, None


def mamba_ssm(xa, w_proj, b_proj, w_dt, b_dt, A, z, state_size: int):
    """The Mamba block's selective SSM after its conv (common.ex:333-471, the B / C and dt
    projections of :340-368 and the scan): xa [B, T, D] (model dtype); w_proj [2 N + R, D] the
    stacked B, C and low-rank dt weights (b_proj [2 N + R] or None); w_dt [D, R] (b_dt [D] or
    None) the dt up-projection; A [D, N] float32; z [B, T, D] the gate branch; N = state_size.
    B and C are taken in float32, dt = softplus(dt_proj(.)), and the scan runs in dt-mean mode
    with the SiLU(z) gate; returns y [B, T, D]."""
    return _MambaSSM.apply(xa, w_proj, b_proj, w_dt, b_dt, A, z, state_size)


class _FlashAttention(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, causal):
        q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
        _dev(q, k, v)
        _same(q, k, v)
        bsz, nh, seq, hd = q.shape
        if k.shape != q.shape or v.shape != q.shape:
            raise EdificeHipError("flash_attention needs q, k, v of one shape [B, H, T, d] (self-attention)")
        out = torch.empty_like(q)
        lse = torch.empty((bsz, nh, seq), dtype=torch.float32, device=q.device)
        nat.call("edf_fused_flash_attention", _stream(), _p(q), _p(k), _p(v), _p(out), _p(lse), bsz, nh, seq, hd,
                 int(causal), dtype_flag(q))
        ctx.causal = int(causal)
        ctx.save_for_backward(q, k, v, out, lse)
        return out

    @staticmethod
    def backward(ctx, dout):
        q, k, v, out, lse = ctx.saved_tensors
        dout = dout.contiguous().to(q.dtype)
        bsz, nh, seq, hd = q.shape
        dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
        wsb = nat.query("edf_flash_attention_backward_workspace_bytes", bsz, nh, seq, hd)
        ws = _u8(wsb, q)
        nat.call("edf_fused_flash_attention_backward", _stream(), _p(q), _p(k), _p(v), _p(out), _p(dout), _p(lse),
                 _p(dq), _p(dk), _p(dv), _p(ws), wsb, bsz, nh, seq, hd, ctx.causal, dtype_flag(q))
        return dq, dk, dv, None


class _FoxAttention(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, cs):
        q, k, v, cs = q.contiguous(), k.contiguous(), v.contiguous(), cs.contiguous()
        _dev(q, k, v, cs)
        _same(q, k, v, cs)
        bsz, nh, seq, hd = q.shape
        if k.shape != q.shape or v.shape != q.shape or tuple(cs.shape) != (bsz, nh, seq):
            raise EdificeHipError("fox_attention needs q, k, v [B, H, T, d] and cs [B, H, T]")
        out = torch.empty_like(q)
        lse = torch.empty((bsz, nh, seq), dtype=torch.float32, device=q.device)
        nat.call("edf_fused_fox_attention", _stream(), _p(q), _p(k), _p(v), _p(cs), _p(out), _p(lse), bsz, nh, seq,
                 hd, dtype_flag(q))
        ctx.save_for_backward(q, k, v, cs, out, lse)
        return out

    @staticmethod
    def backward(ctx, dout):
        q, k, v, cs, out, lse = ctx.saved_tensors
        dout = dout.contiguous().to(q.dtype)
        bsz, nh, seq, hd = q.shape
        dq, dk, dv, dcs = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v), torch.empty_like(cs)
        wsb = nat.query("edf_fox_attention_backward_workspace_bytes", bsz, nh, seq, hd)
        ws = _u8(wsb, q)
        nat.call("edf_fused_fox_attention_backward", _stream(), _p(q), _p(k), _p(v), _p(cs), _p(out), _p(dout),
                 _p(lse), _p(dq), _p(dk), _p(dv), _p(dcs), _p(ws), wsb, bsz, nh, seq, hd, dtype_flag(q))
        return dq, dk, dv, dcs


def fox_attention(q, k, v, cs):
    """``FusedScan.fox_attention/4`` (fused_scan.ex:3796-3810): causal attention with the
    forget bias cs_i - cs_j added to the scaled scores (fused_scan.ex:3860-3905); q, k, v
    [B, H, T, d], cs [B, H, T] (cumulative log forget gates).  Differentiable in all four."""
    return _FoxAttention.apply(q, k, v, cs)


class _LaserAttention(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, vmax, causal):
        q, k, v, vmax = q.contiguous(), k.contiguous(), v.contiguous(), vmax.contiguous()
        _dev(q, k, v, vmax)
        _same(q, k, v, vmax)
        bsz, nh, seq, hd = q.shape
        if k.shape != q.shape or v.shape != q.shape or tuple(vmax.shape) != (bsz, nh, 1, hd):
            raise EdificeHipError("laser_attention needs q, k, v [B, H, T, d] and vmax [B, H, 1, d]")
        out = torch.empty_like(q)
        lse = torch.empty((bsz, nh, seq), dtype=torch.float32, device=q.device)
        flag = dtype_flag(q)
        wsb = nat.query("edf_laser_attention_workspace_bytes", bsz, nh, seq, hd, flag)
        ws = _u8(wsb, q)
        nat.call("edf_fused_laser_attention", _stream(), _p(q), _p(k), _p(v), _p(vmax), _p(out), _p(lse), _p(ws), wsb,
                 bsz, nh, seq, hd, int(causal), flag)
        ctx.causal = int(causal)
        ctx.save_for_backward(q, k, v, vmax, out, lse)
        return out

    @staticmethod
    def backward(ctx, dout):
        q, k, v, vmax, out, lse = ctx.saved_tensors
        dout = dout.contiguous().to(q.dtype)
        bsz, nh, seq, hd = q.shape
        dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
        flag = dtype_flag(q)
        wsb = nat.query("edf_laser_attention_backward_workspace_bytes", bsz, nh, seq, hd, flag)
        ws = _u8(wsb, q)
        nat.call("edf_fused_laser_attention_backward", _stream(), _p(q), _p(k), _p(v), _p(vmax), _p(out), _p(dout),
                 _p(lse), _p(dq), _p(dk), _p(dv), _p(ws), wsb, bsz, nh, seq, hd, ctx.causal, flag)
        return dq, dk, dv, None, None


def laser_attention(q, k, v, causal: bool = True):
    """``FusedScan.laser_attention/4`` (fused_scan.ex:3593-3613): log(softmax(Q K^T / sqrt(d))
    exp(V - vmax)) + vmax with vmax = max over the sequence of V (computed here, as the
    reference wrapper does, and held constant in the backward)."""
    vmax = v.detach().amax(dim=2, keepdim=True)
    return _LaserAttention.apply(q, k, v, vmax, causal)


def flash_attention(q, k, v, causal: bool = False):
    """``FusedScan.flash_attention/4`` (fused_scan.ex:3398-3414): q, k, v [B, H, T, d].

    Scale 1/sqrt(d); causal keeps keys j <= i.  Differentiable (fused HIP backward).
    """
    return _FlashAttention.apply(q, k, v, bool(causal))


BETA_PER_ELEMENT, BETA_PER_HEAD = 0, 1


class _DeltaRule(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, beta, alpha):
        q, k, v, beta, alpha = (_c(t) for t in (q, k, v, beta, alpha))
        _dev(q, k, v, beta, alpha)
        _same(q, k, v, beta, alpha)
        bsz, seq, nh, hd = q.shape
        if k.shape != q.shape or v.shape != q.shape:
            raise EdificeHipError("delta rule needs q, k, v of one shape [B, T, H, d]")
        if beta.shape == q.shape:
            mode = BETA_PER_ELEMENT
        elif beta.shape == q.shape[:3]:
            mode = BETA_PER_HEAD
        else:
            raise EdificeHipError(f"beta must be [B,T,H,d] or [B,T,H], got {tuple(beta.shape)}")
        if alpha is not None and alpha.shape != q.shape[:3]:
            raise EdificeHipError(f"alpha must be [B,T,H], got {tuple(alpha.shape)}")
        dt = dtype_flag(q)
        out = torch.empty_like(v)
        # with gradients to come, a workspace that also keeps the states the backward reads
        # (the chunked path's per-chunk context, or the per-step path's 16-step states)
        query = ("edf_delta_rule_forward_context_bytes" if any(ctx.needs_input_grad)
                 else "edf_delta_rule_workspace_bytes")
        wsb = nat.query(query, bsz, seq, nh, hd, dt, mode)
        ws = _u8(wsb, q) if wsb else None
        if alpha is None:
            nat.call("edf_fused_delta_net_scan", _stream(), _p(q), _p(k), _p(v), _p(beta), _p(out), _p(ws), wsb,
                     bsz, seq, nh, hd, dt, mode)
        else:
            nat.call("edf_fused_gated_delta_net_scan", _stream(), _p(q), _p(k), _p(v), _p(beta), _p(alpha),
                     _p(out), _p(ws), wsb, bsz, seq, nh, hd, dt, mode)
        ctx.mode = mode
        ctx.fwd_ws, ctx.fwd_wsb = ws, wsb
        ctx.save_for_backward(q, k, v, beta, alpha)
        return out

    @staticmethod
    def backward(ctx, do):
        q, k, v, beta, alpha = ctx.saved_tensors
        do = do.contiguous().to(q.dtype)
        bsz, seq, nh, hd = q.shape
        dt = dtype_flag(q)
        dq, dk, dv, db = (torch.empty_like(t) for t in (q, k, v, beta))
        da = torch.empty_like(alpha) if alpha is not None else None
        wsb = nat.query("edf_delta_rule_saved_backward_workspace_bytes", bsz, seq, nh, hd, dt, ctx.mode)
        ws = _u8(wsb, q)
        nat.call("edf_fused_delta_rule_scan_backward_saved", _stream(), _p(q), _p(k), _p(v), _p(beta), _p(alpha),
                 _p(do), _p(dq), _p(dk), _p(dv), _p(db), _p(da), _p(ctx.fwd_ws), ctx.fwd_wsb, _p(ws), wsb,
                 bsz, seq, nh, hd, dt, ctx.mode)
        ctx.fwd_ws = None
        return dq, dk, dv, db, da


class _KDA(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, alpha, beta):
        q, k, v, alpha, beta = (t.contiguous() for t in (q, k, v, alpha, beta))
        _dev(q, k, v, alpha, beta)
        _same(q, k, v, alpha, beta)
        bsz, seq, nh, hd = q.shape
        if alpha.shape != q.shape or tuple(beta.shape) != (bsz, seq, nh):
            raise EdificeHipError("kda_scan needs alpha [B, T, H, d] and beta [B, T, H]")
        out = torch.empty_like(v)
        ctx.rec, ctx.recb = None, 0
        if any(ctx.needs_input_grad):  # keep the 16-step states the backward reads
            ctx.recb = nat.query("edf_kda_scan_context_bytes", bsz, seq, nh, hd, dtype_flag(q))
            ctx.rec = _u8(ctx.recb, q)
            nat.call("edf_fused_kda_scan_with_context", _stream(), _p(q), _p(k), _p(v), _p(alpha), _p(beta), _p(out),
                     _p(ctx.rec), ctx.recb, bsz, seq, nh, hd, dtype_flag(q))
        else:
            nat.call("edf_fused_kda_scan", _stream(), _p(q), _p(k), _p(v), _p(alpha), _p(beta), _p(out), bsz, seq,
                     nh, hd, dtype_flag(q))
        ctx.save_for_backward(q, k, v, alpha, beta, out)
        return out

    @staticmethod
    def backward(ctx, do):
        q, k, v, alpha, beta, out = ctx.saved_tensors
        do = do.contiguous().to(q.dtype)
        bsz, seq, nh, hd = q.shape
        dq, dk, dv, da, db = (torch.empty_like(t) for t in (q, k, v, alpha, beta))
        wsb = nat.query("edf_kda_scan_backward_workspace_bytes", bsz, seq, nh, hd, dtype_flag(q))
        ws = _u8(wsb, q)
        nat.call("edf_fused_kda_scan_backward_saved", _stream(), _p(q), _p(k), _p(v), _p(alpha), _p(beta), _p(do),
                 _p(dq), _p(dk), _p(dv), _p(da), _p(db), _p(ctx.rec), ctx.recb, _p(ws), wsb, bsz, seq, nh, hd,
                 dtype_flag(q))
        ctx.rec = None
        return dq, dk, dv, da, db


def kda_scan(q, k, v, alpha, beta):
    """``FusedScan.kda_scan/5`` (fused_scan.ex:398-412): the delta rule with a log-space decay
    per value row, S_g = diag(exp(alpha_t)) S; q, k, v, alpha [B, T, H, d], beta [B, T, H]."""
    return _KDA.apply(q, k, v, alpha, beta)


class _DeltaProduct(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, beta):
        q, k, v, beta = (t.contiguous() for t in (q, k, v, beta))
        _dev(q, k, v, beta)
        _same(q, k, v, beta)
        bsz, seq, nh, hd = q.shape
        if k.dim() != 5 or tuple(k.shape) != (bsz, seq, k.shape[2], nh, hd) or v.shape != k.shape \
                or tuple(beta.shape) != (bsz, seq, k.shape[2], nh):
            raise EdificeHipError("delta_product_scan needs q [B, T, H, d], k and v [B, T, n_h, H, d], "
                                  "beta [B, T, n_h, H]")
        nhh = k.shape[2]
        out = torch.empty_like(q)
        ctx.rec, ctx.recb = None, 0
        if any(ctx.needs_input_grad):  # keep the partials and states the backward reads
            ctx.recb = nat.query("edf_delta_product_context_bytes", bsz, seq, nhh, nh, hd, dtype_flag(q))
            ctx.rec = _u8(ctx.recb, q)
            nat.call("edf_fused_delta_product_scan_with_context", _stream(), _p(q), _p(k), _p(v), _p(beta), _p(out),
                     _p(ctx.rec), ctx.recb, bsz, seq, nhh, nh, hd, dtype_flag(q))
        else:
            wsb = nat.query("edf_delta_product_workspace_bytes", bsz, seq, nhh, nh, hd, dtype_flag(q))
            ws = _u8(wsb, q)
            nat.call("edf_fused_delta_product_scan", _stream(), _p(q), _p(k), _p(v), _p(beta), _p(out), _p(ws),
                     wsb, bsz, seq, nhh, nh, hd, dtype_flag(q))
        ctx.save_for_backward(q, k, v, beta, out)
        return out

    @staticmethod
    def backward(ctx, do):
        q, k, v, beta, out = ctx.saved_tensors
        do = do.contiguous().to(q.dtype)
        bsz, seq, nh, hd = q.shape
        nhh = k.shape[2]
        dq, dk, dv, db = (torch.empty_like(t) for t in (q, k, v, beta))
        wsb = nat.query("edf_delta_product_backward_workspace_bytes", bsz, seq, nhh, nh, hd, dtype_flag(q))
        ws = _u8(wsb, q)
        nat.call("edf_fused_delta_product_scan_backward_saved", _stream(), _p(q), _p(k), _p(v), _p(beta), _p(do),
                 _p(dq), _p(dk), _p(dv), _p(db), _p(ctx.rec), ctx.recb, _p(ws), wsb, bsz, seq, nhh, nh, hd,
                 dtype_flag(q))
        ctx.rec = None
        return dq, dk, dv, db


def delta_product_scan(q, k, v, beta):
    """``FusedScan.delta_product_scan/4`` (fused_scan.ex:246-260): n_h delta-rule sub-steps per
    token on L2-normalised keys, output RMS_norm of the state contracted with q over its
    value rows; q [B, T, H, d], k and v [B, T, n_h, H, d], beta [B, T, n_h, H] (post-sigmoid)."""
    return _DeltaProduct.apply(q, k, v, beta)


class _RLA(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, alpha, beta, gamma, variant, clip):
        q, k, v, alpha, beta, gamma = (t.contiguous() for t in (q, k, v, alpha, beta, gamma))
        _dev(q, k, v, alpha, beta, gamma)
        _same(q, k, v, alpha, beta, gamma)
        bsz, seq, nh, hd = q.shape
        if k.shape != q.shape or v.shape != q.shape or any(tuple(g.shape) != (bsz, seq, nh) for g in (alpha, beta, gamma)):
            raise EdificeHipError("rla_scan needs q, k, v [B, T, H, d] and alpha, beta, gamma [B, T, H]")
        out = torch.empty_like(q)
        ctx.rec, ctx.recb = None, 0
        if any(ctx.needs_input_grad):  # keep the states the backward reads
            ctx.recb = nat.query("edf_rla_scan_context_bytes", bsz, seq, nh, hd, dtype_flag(q))
            ctx.rec = _u8(ctx.recb, q)
            nat.call("edf_fused_rla_scan_with_context", _stream(), _p(q), _p(k), _p(v), _p(alpha), _p(beta),
                     _p(gamma), _p(out), _p(ctx.rec), ctx.recb, bsz, seq, nh, hd, variant, float(clip),
                     dtype_flag(q))
        else:
            nat.call("edf_fused_rla_scan", _stream(), _p(q), _p(k), _p(v), _p(alpha), _p(beta), _p(gamma), _p(out),
                     bsz, seq, nh, hd, variant, float(clip), dtype_flag(q))
        ctx.save_for_backward(q, k, v, alpha, beta, gamma, out)
        ctx.variant, ctx.clip = variant, float(clip)
        return out

    @staticmethod
    def backward(ctx, do):
        q, k, v, alpha, beta, gamma, out = ctx.saved_tensors
        do = do.contiguous().to(q.dtype)
        bsz, seq, nh, hd = q.shape
        dq, dk, dv, da, db, dg = (torch.empty_like(t) for t in (q, k, v, alpha, beta, gamma))
        wsb = nat.query("edf_rla_scan_backward_workspace_bytes", bsz, seq, nh, hd, dtype_flag(q))
        ws = _u8(wsb, q)
        nat.call("edf_fused_rla_scan_backward_saved", _stream(), _p(q), _p(k), _p(v), _p(alpha), _p(beta),
                 _p(gamma), _p(do), _p(dq), _p(dk), _p(dv), _p(da), _p(db), _p(dg), _p(ctx.rec), ctx.recb, _p(ws),
                 wsb, bsz, seq, nh, hd, ctx.variant, ctx.clip, dtype_flag(q))
        ctx.rec = None
        return dq, dk, dv, da, db, dg, None, None


def rla_scan(q, k, v, alpha, beta, gamma, variant="rla", clip_threshold=1.0):
    """``FusedScan.rla_scan/7`` (fused_scan.ex:431-448): residual linear attention with base
    state S and residual state R; q, k, v [B, T, H, d], alpha, beta, gamma [B, T, H];
    variant "rla" (S += b v k^T) or "rdn" (delta-rule updates of both states); the residual
    error is clipped to [-clip_threshold, clip_threshold]."""
    var = {"rla": 0, "rdn": 1}[variant]
    return _RLA.apply(q, k, v, alpha, beta, gamma, var, clip_threshold)


class _TTT(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, eta, w0, ln_g, ln_b):
        q, k, v, eta, w0, ln_g, ln_b = (t.contiguous() for t in (q, k, v, eta, w0, ln_g, ln_b))
        _dev(q, k, v, eta, w0, ln_g, ln_b)
        _same(q, k, v, eta, w0, ln_g, ln_b)
        bsz, seq, dd = q.shape
        if any(t.shape != q.shape for t in (k, v, eta)) or tuple(w0.shape) != (bsz, dd, dd) \
                or tuple(ln_g.shape) != (dd,) or tuple(ln_b.shape) != (dd,):
            raise EdificeHipError("ttt_scan needs q, k, v, eta [B, T, D], w0 [B, D, D], ln_gamma, ln_beta [D]")
        out = torch.empty_like(q)
        ctx.rec, ctx.recb = None, 0
        if any(ctx.needs_input_grad):  # record what the backward reads in the same pass
            ctx.recb = nat.query("edf_ttt_scan_context_bytes", bsz, seq, dd, dtype_flag(q))
            ctx.rec = _u8(ctx.recb, q)
            nat.call("edf_fused_ttt_scan_with_context", _stream(), _p(q), _p(k), _p(v), _p(eta), _p(w0), _p(ln_g),
                     _p(ln_b), _p(out), _p(ctx.rec), ctx.recb, bsz, seq, dd, dtype_flag(q))
        else:
            nat.call("edf_fused_ttt_scan", _stream(), _p(q), _p(k), _p(v), _p(eta), _p(w0), _p(ln_g), _p(ln_b),
                     _p(out), bsz, seq, dd, dtype_flag(q))
        ctx.save_for_backward(q, k, v, eta, w0, ln_g, ln_b)
        return out

    @staticmethod
    def backward(ctx, do):
        q, k, v, eta, w0, ln_g, ln_b = ctx.saved_tensors
        do = do.contiguous().to(q.dtype)
        bsz, seq, dd = q.shape
        grads = [torch.empty_like(t) for t in (q, k, v, eta, w0, ln_g, ln_b)]
        wsb = nat.query("edf_ttt_scan_backward_workspace_bytes", bsz, seq, dd, dtype_flag(q))
        ws = _u8(wsb, q)
        nat.call("edf_fused_ttt_scan_backward_saved", _stream(), _p(q), _p(k), _p(v), _p(eta), _p(w0), _p(ln_g),
                 _p(ln_b), _p(do), *(_p(g) for g in grads), _p(ctx.rec), ctx.recb, _p(ws), wsb, bsz, seq, dd,
                 dtype_flag(q))
        ctx.rec = None
        return tuple(grads)


def ttt_scan(q, k, v, eta, w0, ln_gamma, ln_beta):
    """``FusedScan.ttt_scan/7`` (fused_scan.ex:344-358): TTT-Linear with inner model W [B, D, D]
    (initial w0) trained per step by one LayerNorm-ed reconstruction step; q, k, v, eta
    (post-sigmoid learning rate) [B, T, D], ln_gamma, ln_beta [D]."""
    return _TTT.apply(q, k, v, eta, w0, ln_gamma, ln_beta)


def delta_net_scan(q, k, v, beta):
    """``FusedScan.delta_net_scan/4`` (fused_scan.ex:195-209): q, k, v [B, T, H, d]; k
    L2-normalised, beta post-sigmoid, per element [B, T, H, d] or per head [B, T, H]."""
    return _DeltaRule.apply(q, k, v, beta, None)


def gated_delta_net_scan(q, k, v, beta, alpha):
    """``FusedScan.gated_delta_net_scan/5`` (fused_scan.ex:219-233): as delta_net_scan with a
    per-(b, t, head) decay alpha [B, T, H] applied to the state before each update."""
    return _DeltaRule.apply(q, k, v, beta, alpha)


def selective_scan(x, dt, a, b, c, d=None, z=None, *, dt_mode: str = "channel", dt_softplus: bool = False):
    """``FusedScan.selective_scan/5`` (fused_scan.ex:370-384) plus optional D skip and silu(z) gate.

    x, dt (and z): [B, T, D]; a: [D, N]; b, c: [B, T, N]; d: [D].  dt is clipped to
    [1e-3, 0.1] inside the kernel.  dt_mode="channel" is the kernel semantics
    (B_bar = dt B per channel, fused_selective_scan.cu:68-90); "mean" is the Mamba
    block CPU semantics (B_bar = mean_d(dt) B, common.ex:402-445).  dt_softplus=True (mean
    mode only; the library rejects it with "channel"): dt is the pre-activation and the kernels take softplus(dt) wherever they read it (the Mamba
    block's dt = softplus(dt_proj(.)), common.ex:366), dt's gradient being with respect to
    the pre-activation (no reference counterpart: the block glue's activation without a
    pass and a tensor of its own).
    """
    mode = {"channel": SS_DT_PER_CHANNEL, "mean": SS_DT_MEAN}[dt_mode] | (SS_DT_SOFTPLUS if dt_softplus else 0)
    return _SelectiveScan.apply(x, dt, a, b, c, d, z, mode)
