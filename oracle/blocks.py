"""Block-level restatement of Edifice's sequence-mixing callers — TEST INFRASTRUCTURE ONLY.

Used to pin the scan restatements (and, in GPU tests, the HIP kernels) against the
reference's own model-level fixtures ``test/fixtures/numerical/*_random.safetensors``,
which hold PyTorch-generated weights, inputs, expected outputs and (DeltaNet) the input
gradient.  The models mirror the Edifice blocks:

  MinGRU   lib/edifice/recurrent/min_gru.ex:272-295 (layer), :305-326 (scan)
  MinLSTM  lib/edifice/recurrent/min_lstm.ex:267-292 (layer), :304-334 (scan); no fixture
  DeltaNet lib/edifice/recurrent/delta_net.ex:197-219 (layer), :275-307 (projection split,
           sigmoid beta, key L2 norm with eps 1e-6 inside the sqrt)
  Mamba    lib/edifice/ssm/common.ex:210-279 (block), :333-373 (B/C/dt projections),
           :402-471 (dt-mean discretisation and output)
  GQA      causal grouped-query attention block, fed through the flash-attention op
           (lib/edifice/blocks/sdpa.ex:74-91 routes causal self-attention to flash)

Dense layers use the fixture's PyTorch layout (weight [out, in]).  Layer norm uses
eps 1e-5, the value the fixtures were generated with.  The sequence-mixing op of each
block is pluggable (``ops``) so the same model runs the numpy oracle or the HIP path;
everything around it runs in float64 torch on the CPU (or the device of the input).
"""
from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F

from . import scans

LN_EPS = 1.0e-5


def _np(t):
    return t.detach().cpu().double().numpy()


def _t(a, like):
    return torch.from_numpy(np.ascontiguousarray(a)).to(device=like.device, dtype=like.dtype)


class _OracleMinGRU(torch.autograd.Function):
    @staticmethod
    def forward(ctx, gates, cand):
        ctx.save_for_backward(gates, cand)
        return _t(scans.min_gru_scan(_np(gates), _np(cand)), gates)

    @staticmethod
    def backward(ctx, dy):
        gates, cand = ctx.saved_tensors
        dg, dc = scans.min_gru_scan_backward(_np(gates), _np(cand), _np(dy))
        return _t(dg, gates), _t(dc, cand)


class _OracleMinLSTM(torch.autograd.Function):
    """Logit-level MinLSTM (sigmoids applied inside), forward and the hand-derived backward."""

    @staticmethod
    def forward(ctx, fg, ig, cand):
        ctx.save_for_backward(fg, ig, cand)
        return _t(scans.min_lstm_scan(_np(fg), _np(ig), _np(cand)), fg)

    @staticmethod
    def backward(ctx, dy):
        fg, ig, cand = ctx.saved_tensors
        f, i = scans.sigmoid(_np(fg)), scans.sigmoid(_np(ig))
        fwd = scans.minlstm_scan(f, i, _np(cand))
        df, di, dc, _ = scans.minlstm_scan_backward(f, i, _np(cand), None, fwd, _np(dy))
        return _t(df * f * (1 - f), fg), _t(di * i * (1 - i), ig), _t(dc, cand)


class _OracleDelta(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, beta):
        ctx.save_for_backward(q, k, v, beta)
        return _t(scans.delta_rule(_np(q), _np(k), _np(v), _np(beta)), q)

    @staticmethod
    def backward(ctx, do):
        q, k, v, beta = ctx.saved_tensors
        g = scans.delta_rule_backward(_np(q), _np(k), _np(v), _np(beta), _np(do))
        return _t(g["dq"], q), _t(g["dk"], k), _t(g["dv"], v), _t(g["dbeta"], beta)


class _OracleSelectiveScanMean(torch.autograd.Function):
    """Mean-mode selective scan with the silu(z) gate (the Mamba block's scan), forward and
    the hand-derived backward of scans.selective_scan_backward."""

    @staticmethod
    def forward(ctx, x, dt, A, B, C, z):
        ctx.save_for_backward(x, dt, A, B, C, z)
        return _t(scans.selective_scan(_np(x), _np(dt), _np(A), _np(B), _np(C), None, _np(z), mode="mean"), x)

    @staticmethod
    def backward(ctx, dy):
        x, dt, A, B, C, z = ctx.saved_tensors
        g = scans.selective_scan_backward(_np(x), _np(dt), _np(A), _np(B), _np(C), _np(dy), None, _np(z), mode="mean")
        return (_t(g["dx"], x), _t(g["ddt"], dt), _t(g["dA"], A), _t(g["dB"], B), _t(g["dC"], C), _t(g["dz"], z))


class _OracleCausalAttention(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v):
        ctx.save_for_backward(q, k, v)
        return _t(scans.flash_attention(_np(q), _np(k), _np(v), causal=True), q)

    @staticmethod
    def backward(ctx, do):
        q, k, v = ctx.saved_tensors
        dq, dk, dv = scans.flash_attention_backward(_np(q), _np(k), _np(v), _np(do), causal=True)
        return _t(dq, q), _t(dk, k), _t(dv, v)


class _OracleGatedDelta(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, beta, alpha):
        ctx.save_for_backward(q, k, v, beta, alpha)
        return _t(scans.delta_rule(_np(q), _np(k), _np(v), _np(beta), _np(alpha)), q)

    @staticmethod
    def backward(ctx, do):
        q, k, v, beta, alpha = ctx.saved_tensors
        g = scans.delta_rule_backward(_np(q), _np(k), _np(v), _np(beta), _np(do), _np(alpha))
        return _t(g["dq"], q), _t(g["dk"], k), _t(g["dv"], v), _t(g["dbeta"], beta), _t(g["dalpha"], alpha)


def differentiable_oracle_ops():
    """Every block op as a numpy-oracle autograd Function (forward + hand-derived backward),
    for gradient checks of whole blocks; the Mamba scan takes the z gate inside."""
    return {
        "mingru": _OracleMinGRU.apply,
        "minlstm": _OracleMinLSTM.apply,
        "delta_net": _OracleDelta.apply,
        "gated_delta_net": _OracleGatedDelta.apply,
        "selective_scan_mean_gated": _OracleSelectiveScanMean.apply,
        "causal_attention": _OracleCausalAttention.apply,
    }


def oracle_ops():
    """The numpy oracle as pluggable block ops (forward + hand-derived backward)."""
    return {
        "mingru": _OracleMinGRU.apply,
        "delta_net": _OracleDelta.apply,
        "selective_scan_mean": lambda x, dt, A, B, C: _t(
            scans.selective_scan(_np(x), _np(dt), _np(A), _np(B), _np(C), mode="mean"), x),
        "causal_attention": lambda q, k, v: _t(
            scans.flash_attention(_np(q), _np(k), _np(v), causal=True), q),
    }


def load_fixture(path):
    from safetensors.numpy import load_file

    return {k: torch.from_numpy(v.astype(np.float64)) for k, v in load_file(path).items()}


def _dense(w, prefix, x):
    return F.linear(x, w[prefix + ".weight"], w.get(prefix + ".bias"))


def _ln(w, prefix, x):
    return F.layer_norm(x, (x.shape[-1],), w[prefix + ".weight"], w[prefix + ".bias"], LN_EPS)


def min_gru_model(w, x, ops):
    """MinGRU.build/1: input projection, 2 x (LN -> gate/candidate -> scan -> residual), final LN."""
    h = _dense(w, "weight.input_projection", x)
    for li in range(2):
        p = f"weight.layers.{li}"
        n = _ln(w, p + ".norm", h)
        h = h + ops["mingru"](_dense(w, p + ".gate", n), _dense(w, p + ".candidate", n))
    return _ln(w, "weight.final_norm", h)[:, -1]


def min_lstm_model(w, x, ops):
    """MinLSTM.build/1 (min_lstm.ex:113-162) with embed == hidden: 2 x (LN -> forget, input,
    candidate projections -> scan -> residual, min_lstm.ex:267-292), final LN, last timestep."""
    h = x
    for li in range(2):
        p = f"weight.layers.{li}"
        n = _ln(w, p + ".norm", h)
        h = h + ops["minlstm"](_dense(w, p + ".forget", n), _dense(w, p + ".input", n), _dense(w, p + ".candidate", n))
    return _ln(w, "weight.final_norm", h)[:, -1]


def delta_net_layer(w, p, h, ops, num_heads):
    """One DeltaNet layer (delta_net.ex:197-219, :275-307) under key prefix ``p``, residual
    included: h + out_proj(DeltaRule(q, l2norm(k), v, sigmoid(b)))."""
    bsz, seq, hid = h.shape
    hd = hid // num_heads
    n = _ln(w, p + ".norm", h)
    proj = _dense(w, p + ".qkvb_proj", n)
    q, k, v, bpre = torch.split(proj, hid, dim=-1)
    shp = (bsz, seq, num_heads, hd)
    q, k, v = q.reshape(shp), k.reshape(shp), v.reshape(shp)
    beta = torch.sigmoid(bpre).reshape(shp)
    k = k / torch.sqrt((k * k).sum(-1, keepdim=True) + scans.KEY_NORM_EPS)
    o = ops["delta_net"](q, k, v, beta).reshape(bsz, seq, hid)
    return h + _dense(w, p + ".out_proj", o)


def delta_net_model(w, x, ops, num_heads=4):
    """DeltaNet.build/1 with embed == hidden (no input projection), 2 layers, final LN."""
    h = x
    for li in range(2):
        h = delta_net_layer(w, f"weight.layers.{li}", h, ops, num_heads)
    return _ln(w, "weight.final_norm", h)[:, -1]


def gated_delta_net_model(w, x, ops, num_heads=4, conv_size=4):
    """GatedDeltaNet.build with embed == hidden: per layer LN, short causal depthwise conv +
    SiLU, 6 x hidden projection split into q, k, v, beta, alpha, gate
    (gated_delta_net.ex:230-290, 355-401); alpha = head mean of sigmoid; swish output gate;
    residual; final LN; last timestep.  No reference fixture exists for this family."""
    h = x
    bsz, seq, hid = x.shape
    hd = hid // num_heads
    shp = (bsz, seq, num_heads, hd)
    for li in range(2):
        p = f"weight.layers.{li}"
        n = _ln(w, p + ".norm", h)
        n = F.silu(F.conv1d(n.transpose(1, 2), w[p + ".short_conv.weight"], w[p + ".short_conv.bias"],
                            padding=conv_size - 1, groups=hid)[..., :seq].transpose(1, 2))
        q, k, v, bpre, apre, gpre = torch.split(_dense(w, p + ".qkvbag_proj", n), hid, dim=-1)
        k = k.reshape(shp)
        k = k / torch.sqrt((k * k).sum(-1, keepdim=True) + scans.KEY_NORM_EPS)
        alpha = torch.sigmoid(apre).reshape(shp).mean(-1)
        o = ops["gated_delta_net"](q.reshape(shp), k, v.reshape(shp), torch.sigmoid(bpre).reshape(shp), alpha)
        h = h + _dense(w, p + ".out_proj", o.reshape(bsz, seq, hid) * F.silu(gpre))
    return _ln(w, "weight.final_norm", h)[:, -1]


def mamba_block(w, p, h, ops, state_size, conv_size=4):
    """One Mamba block (common.ex:210-279, SSM :333-471) under key prefix ``p``, WITHOUT the
    residual (Common.build_model adds it)."""
    n = _ln(w, p + ".norm", h)
    xz = _dense(w, p + ".in_proj", n)
    inner = xz.shape[-1] // 2
    xb, zb = xz[..., :inner], xz[..., inner:]
    seq = xb.shape[1]
    conv = F.conv1d(xb.transpose(1, 2), w[p + ".dw_conv.weight"], w[p + ".dw_conv.bias"],
                    padding=conv_size - 1, groups=inner)[..., :seq].transpose(1, 2)
    xa = F.silu(conv)
    bc = _dense(w, p + ".bc_proj", xa)
    Bm, Cm = bc[..., :state_size], bc[..., state_size:]
    dt = F.softplus(_dense(w, p + ".dt_proj", _dense(w, p + ".dt_rank_proj", xa)))
    A = -(torch.arange(state_size, dtype=h.dtype, device=h.device) + 1.0)
    A = A[None, :].expand(inner, state_size).contiguous()
    if "selective_scan_mean_gated" in ops:
        y = ops["selective_scan_mean_gated"](xa, dt, A, Bm, Cm, zb)
    else:
        y = ops["selective_scan_mean"](xa, dt, A, Bm, Cm) * F.silu(zb)
    return _dense(w, p + ".out_proj", y)


def mamba_model(w, x, ops, state_size=8, conv_size=4):
    """Mamba.build/1 via Common.build_model: 2 residual blocks, last timestep (no final LN)."""
    h = x
    for li in range(2):
        h = h + mamba_block(w, f"weight.blocks.{li}", h, ops, state_size, conv_size)
    return h[:, -1]


def gqa_block(w, p, h, ops, num_heads, num_kv_heads):
    """One causal GQA transformer block (attention + GELU FFN, both pre-norm residual)
    under key prefix ``p``."""
    bsz, seq, hid = h.shape
    hd = hid // num_heads
    grp = num_heads // num_kv_heads
    n = _ln(w, p + ".attn_norm", h)
    q = _dense(w, p + ".attn.q_proj", n).reshape(bsz, seq, num_heads, hd).transpose(1, 2)
    k = _dense(w, p + ".attn.k_proj", n).reshape(bsz, seq, num_kv_heads, hd).transpose(1, 2)
    v = _dense(w, p + ".attn.v_proj", n).reshape(bsz, seq, num_kv_heads, hd).transpose(1, 2)
    k = k.repeat_interleave(grp, dim=1).contiguous()
    v = v.repeat_interleave(grp, dim=1).contiguous()
    o = ops["causal_attention"](q.contiguous(), k, v)
    o = o.transpose(1, 2).reshape(bsz, seq, hid)
    h = h + _dense(w, p + ".attn.out_proj", o)
    f = _ln(w, p + ".ffn_norm", h)
    return h + _dense(w, p + ".ffn_down", F.gelu(_dense(w, p + ".ffn_up", f)))


def gqa_model(w, x, ops, num_heads=4, num_kv_heads=2):
    """Causal GQA transformer, 2 blocks (attention + GELU FFN), final LN, last timestep."""
    h = x
    for li in range(2):
        h = gqa_block(w, f"weight.blocks.{li}", h, ops, num_heads, num_kv_heads)
    return _ln(w, "weight.final_norm", h)[:, -1]


def hybrid_decoder_loss(w, tokens, ops, num_heads, state_size=16, conv_size=4, layers=(4, 2, 2)):
    """The config-5 decoder stack (SURVEY 3.5's assembly from blocks that reach the fused
    kernels: ModelBuilder.build_sequence_model with output_mode :all, model_builder.ex:71-132):
    embedding -> Mamba blocks (residual added here) -> DeltaNet layers -> causal attention +
    FFN blocks -> final LN -> LM head (no bias) -> mean next-token cross entropy over
    tokens[:, 1:] (the loss of recipes.ex:158-194).  Keys follow edifice_amd.blocks.HybridDecoder
    under "weight." (embed, mamba.i, delta.i, attn.i, final_norm, lm_head)."""
    n_mamba, n_delta, n_attn = layers
    h = F.embedding(tokens[:, :-1], w["weight.embed.weight"])
    for i in range(n_mamba):
        h = h + mamba_block(w, f"weight.mamba.{i}", h, ops, state_size, conv_size)
    for i in range(n_delta):
        h = delta_net_layer(w, f"weight.delta.{i}", h, ops, num_heads)
    for i in range(n_attn):
        h = gqa_block(w, f"weight.attn.{i}", h, ops, num_heads, num_heads)
    logits = _dense(w, "weight.lm_head", _ln(w, "weight.final_norm", h))
    return F.cross_entropy(logits.reshape(-1, logits.shape[-1]), tokens[:, 1:].reshape(-1))
