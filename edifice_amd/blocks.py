"""Block-level callers of the fused ops: Edifice's sequence-mixing blocks as torch modules.

Each block wires the projections, gates, normalisations and head reshapes of the
reference block around one fused HIP op from :mod:`edifice_amd.fused_scan`, so a
forward and backward through a block runs the HIP kernels for the recurrence and torch
(rocBLAS / MIOpen) for the dense layers around it:

  MinGRULayer        lib/edifice/recurrent/min_gru.ex:272-295 (pre-norm, gate and candidate
                     projections, FusedScan.mingru, residual)
  MinLSTMLayer       lib/edifice/recurrent/min_lstm.ex:267-292 (pre-norm, forget, input and
                     candidate projections, FusedScan.minlstm, residual)
  MambaBlock         lib/edifice/ssm/common.ex:210-279 (norm, in_proj to 2 x inner, x/z split,
                     causal depthwise conv + SiLU, SSM, SiLU(z) gate, out_proj) with the SSM of
                     common.ex:333-373 (B/C and low-rank dt projections, softplus) and the dt-mean
                     discretisation of common.ex:402-471; A = -(1..N) per channel
  DeltaNetLayer      lib/edifice/recurrent/delta_net.ex:197-219, 275-307 (qkvb projection,
                     sigmoid beta, key L2 norm with eps inside the sqrt, per-head recurrence)
  GatedDeltaNetLayer lib/edifice/recurrent/gated_delta_net.ex:230-290, 355-401 (optional short
                     causal conv, 6 x hidden projection, per-head alpha = mean of sigmoid,
                     swish output gate)
  GQABlock           causal grouped-query attention routed to flash attention
                     (lib/edifice/blocks/sdpa.ex:74-91) + GELU feed-forward

``build(name, **opts)`` mirrors ``Edifice.build(name, opts)`` for these families and returns
a model mapping [batch, seq, embed] to the last timestep's hidden state, as the reference's
sequence models do.  Module attributes follow the reference layer names, so
``load_reference_weights`` reads the reference's own weight files (``weight.<layer>...``
keys, PyTorch layout) unchanged.

There is no CPU path: the fused ops raise on CPU tensors.
"""
from __future__ import annotations

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import fused_scan as fs

LN_EPS = 1.0e-5       # layer-norm epsilon the reference fixtures were generated with
KEY_NORM_EPS = 1.0e-6  # inside the sqrt of the key L2 norm (delta_net.ex:291, gated_delta_net.ex:387)


def _heads(t: torch.Tensor, num_heads: int) -> torch.Tensor:
    bsz, seq, hid = t.shape
    return t.reshape(bsz, seq, num_heads, hid // num_heads).contiguous()


class _LinearFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, weight, bias):
        ctx.save_for_backward(x, weight)
        ctx.has_bias = bias is not None
        return F.linear(x, weight, bias)

    @staticmethod
    def backward(ctx, dy):
        x, weight = ctx.saved_tensors
        dy2 = dy.reshape(-1, dy.shape[-1])
        dx = dw = db = None
        if ctx.needs_input_grad[0]:
            dx = dy2.mm(weight).view(x.shape)
        if ctx.needs_input_grad[1]:
            dw = fs.weight_grad(dy2, x.reshape(-1, x.shape[-1]))
        if ctx.has_bias and ctx.needs_input_grad[2]:
            db = fs.bias_grad(dy2)
        return dx, dw, db


class _LinearPair(torch.autograd.Function):
    """y1, y2 = x W[:m1]^T + b[:m1], x W[m1:]^T + b[m1:]: one layer's output rows as two
    products with contiguous outputs.  The backward adds the second product's input gradient
    into the first's (addmm, no separate add) and writes the weight and bias gradients into
    one buffer each (row slices of one output would each be scattered into a zero-filled
    full-size gradient and added)."""

    @staticmethod
    def forward(ctx, x, weight, bias, m1):
        b1, b2 = (None, None) if bias is None else (bias[:m1], bias[m1:])
        ctx.save_for_backward(x, weight)
        ctx.m1, ctx.has_bias = m1, bias is not None
        return F.linear(x, weight[:m1], b1), F.linear(x, weight[m1:], b2)

    @staticmethod
    def backward(ctx, dy1, dy2):
        x, weight = ctx.saved_tensors
        m1 = ctx.m1
        x2 = x.reshape(-1, x.shape[-1])
        g1, g2 = dy1.reshape(-1, dy1.shape[-1]), dy2.reshape(-1, dy2.shape[-1])
        dx = dw = db = None
        if ctx.needs_input_grad[0]:
            dx = g1.mm(weight[:m1])
            dx.addmm_(g2, weight[m1:])
            dx = dx.view(x.shape)
        if ctx.needs_input_grad[1]:
            dw = torch.empty_like(weight)
            fs.weight_grad(g1, x2, out=dw[:m1])
            fs.weight_grad(g2, x2, out=dw[m1:])
        if ctx.has_bias and ctx.needs_input_grad[2]:
            db = torch.empty(weight.shape[0], dtype=weight.dtype, device=weight.device)
            fs.bias_grad(g1, out=db[:m1])
            fs.bias_grad(g2, out=db[m1:])
        return dx, dw, db, None


class Linear(nn.Linear):
    """nn.Linear (same parameters and state-dict names; Axon.dense of the reference blocks)
    whose weight gradient splits the row dimension when that pays (``_weight_grad``)."""

    def forward(self, x):
        return _LinearFn.apply(x, self.weight, self.bias)


class Embedding(nn.Embedding):
    """nn.Embedding (same parameter and state-dict name) whose weight gradient is the HIP
    kernel, ``fs.embedding`` (Axon.embedding of the reference language models)."""

    def forward(self, ids):
        if self.max_norm is not None or self.scale_grad_by_freq or self.sparse:
            raise ValueError("Embedding: max_norm, scale_grad_by_freq and sparse are not supported")
        return fs.embedding(ids, self.weight, self.padding_idx)


class LayerNorm(nn.LayerNorm):
    """nn.LayerNorm over the last dimension (same parameters and state-dict names) run by the
    HIP layer norm, ``fs.layer_norm``: Axon.layer_norm of the reference blocks
    (common.ex:224, delta_net.ex:159,199, model_builder.ex:111,165)."""

    def forward(self, x):
        return fs.layer_norm(x, self.weight, self.bias, self.eps)


def _l2norm_keys(k: torch.Tensor) -> torch.Tensor:
    return fs.l2_normalize(k, KEY_NORM_EPS)


class MinGRULayer(nn.Module):
    """min_gru.ex:272-295: x + MinGRU(gate(norm x), candidate(norm x)); the gate's sigmoid
    and its chain rule run inside the fused kernels."""

    def __init__(self, hidden_size: int):
        super().__init__()
        self.norm = LayerNorm(hidden_size, eps=LN_EPS)
        self.gate = Linear(hidden_size, hidden_size)
        self.candidate = Linear(hidden_size, hidden_size)

    def forward(self, x):
        n = self.norm(x)
        return x + fs.mingru(self.gate(n).contiguous(), self.candidate(n).contiguous())


class MinLSTMLayer(nn.Module):
    """min_lstm.ex:267-292: x + MinLSTM(forget(norm x), input(norm x), candidate(norm x)); the
    two gate sigmoids, their normalisation f / (f + i + 1e-6) and its chain rule run inside
    the fused kernels."""

    def __init__(self, hidden_size: int):
        super().__init__()
        self.norm = LayerNorm(hidden_size, eps=LN_EPS)
        self.forget = Linear(hidden_size, hidden_size)
        self.input = Linear(hidden_size, hidden_size)
        self.candidate = Linear(hidden_size, hidden_size)

    def forward(self, x):
        n = self.norm(x)
        return x + fs.minlstm(self.forget(n).contiguous(), self.input(n).contiguous(),
                              self.candidate(n).contiguous())


class MambaBlock(nn.Module):
    """common.ex:210-279 (block) around the selective SSM of common.ex:333-471.

    The scan runs the fused kernel in dt-mean mode (the block's CPU semantics) with the
    SiLU(z) gate fused in; B, C and A are float32 (the reference's parameter precision),
    x, dt and z keep the model dtype.  Returns the block output without the residual
    (the model adds it, as Common.build_model does)."""

    def __init__(self, hidden_size: int, state_size: int = 16, expand_factor: int = 2, conv_size: int = 4):
        super().__init__()
        inner = hidden_size * expand_factor
        dt_rank = max(hidden_size // 16, 1)  # common.ex:221
        self.inner, self.state_size = inner, state_size
        self.norm = LayerNorm(hidden_size, eps=LN_EPS)
        self.in_proj = Linear(hidden_size, 2 * inner)
        self.dw_conv = nn.Conv1d(inner, inner, conv_size, padding=conv_size - 1, groups=inner)
        self.bc_proj = Linear(inner, 2 * state_size)
        self.dt_rank_proj = Linear(inner, dt_rank)
        self.dt_proj = Linear(dt_rank, inner)
        self.out_proj = Linear(inner, hidden_size)
        a = -(torch.arange(state_size, dtype=torch.float32) + 1.0)
        self.register_buffer("A", a[None, :].expand(inner, state_size).contiguous(), persistent=False)

    def forward(self, x):
        return self.mix(self.norm(x))

    def mix(self, n):
        """The block after its norm: n = norm(x) -> the output the residual adds."""
        # in_proj's two halves as two products over its weight rows (x and z contiguous)
        xb, zb = _LinearPair.apply(n, self.in_proj.weight, self.in_proj.bias, self.inner)
        xa = fs.causal_conv1d_silu(xb, self.dw_conv.weight, self.dw_conv.bias)
        # the B / C and low-rank dt projections as one product over their stacked weight rows
        w1, w2, b1, b2 = self.bc_proj.weight, self.dt_rank_proj.weight, self.bc_proj.bias, self.dt_rank_proj.bias
        wcat = torch.cat([w1, w2], 0)
        bcat = None
        if b1 is not None or b2 is not None:  # a missing bias stacks as zeros
            bcat = torch.cat([b1 if b1 is not None else w1.new_zeros(w1.shape[0]),
                              b2 if b2 is not None else w2.new_zeros(w2.shape[0])], 0)
        y = fs.mamba_ssm(xa, wcat, bcat, self.dt_proj.weight, self.dt_proj.bias, self.A.float(), zb,
                         self.state_size)
        return self.out_proj(y)


class DeltaNetLayer(nn.Module):
    """delta_net.ex:197-219 and :275-307: x + out_proj(DeltaRule(q, l2norm(k), v, sigmoid(b)))."""

    def __init__(self, hidden_size: int, num_heads: int):
        super().__init__()
        self.hidden, self.num_heads = hidden_size, num_heads
        self.norm = LayerNorm(hidden_size, eps=LN_EPS)
        self.qkvb_proj = Linear(hidden_size, 4 * hidden_size)
        self.out_proj = Linear(hidden_size, hidden_size)

    def forward(self, x):
        return x + self.mix(self.norm(x))

    def mix(self, n):
        """The layer after its norm: n = norm(x) -> the output the residual adds."""
        bsz, seq, hid = n.shape
        # q, l2norm(k), v, sigmoid(beta_pre) in the scan's head layout, one pass each way
        q, k, v, beta = fs.delta_net_split(self.qkvb_proj(n), self.num_heads, KEY_NORM_EPS)
        o = fs.delta_net_scan(q, k, v, beta)
        return self.out_proj(o.reshape(bsz, seq, hid))


class GatedDeltaNetLayer(nn.Module):
    """gated_delta_net.ex:230-290 and :355-401: optional short causal conv (+ SiLU), a
    6 x hidden projection to q, k, v, beta, alpha, gate; alpha is the head mean of
    sigmoid(alpha_pre); the output is swish(gate)-gated before out_proj; residual."""

    def __init__(self, hidden_size: int, num_heads: int, use_short_conv: bool = True, conv_size: int = 4):
        super().__init__()
        self.hidden, self.num_heads = hidden_size, num_heads
        self.norm = LayerNorm(hidden_size, eps=LN_EPS)
        self.short_conv = (nn.Conv1d(hidden_size, hidden_size, conv_size, padding=conv_size - 1,
                                     groups=hidden_size) if use_short_conv else None)
        self.qkvbag_proj = Linear(hidden_size, 6 * hidden_size)
        self.out_proj = Linear(hidden_size, hidden_size)

    def forward(self, x):
        bsz, seq, hid = x.shape
        h = self.norm(x)
        if self.short_conv is not None:
            h = fs.causal_conv1d_silu(h, self.short_conv.weight, self.short_conv.bias)
        q, k, v, bpre, apre, gpre = torch.split(self.qkvbag_proj(h), hid, dim=-1)
        nh = self.num_heads
        alpha = _heads(torch.sigmoid(apre), nh).mean(-1).contiguous()
        o = fs.gated_delta_net_scan(_heads(q, nh), _l2norm_keys(_heads(k, nh)), _heads(v, nh),
                                    _heads(torch.sigmoid(bpre), nh), alpha)
        return x + self.out_proj(o.reshape(bsz, seq, hid) * F.silu(gpre))


class GQAttention(nn.Module):
    """Causal grouped-query self-attention on the fused flash kernel; the KV heads are
    repeated to the query heads before the kernel."""

    def __init__(self, hidden_size: int, num_heads: int, num_kv_heads: int):
        super().__init__()
        self.num_heads, self.num_kv_heads = num_heads, num_kv_heads
        hd = hidden_size // num_heads
        self.q_proj = Linear(hidden_size, hidden_size)
        self.k_proj = Linear(hidden_size, num_kv_heads * hd)
        self.v_proj = Linear(hidden_size, num_kv_heads * hd)
        self.out_proj = Linear(hidden_size, hidden_size)

    def forward(self, x):
        bsz, seq, hid = x.shape
        nh, nkv = self.num_heads, self.num_kv_heads
        hd = hid // nh
        if nkv == nh:
            # q, k, v as one product over the stacked weights, split into the kernel's head
            # layout in one pass (the backward merges dq, dk, dv into one gradient, no adds)
            projs = (self.q_proj, self.k_proj, self.v_proj)
            w = torch.cat([m.weight for m in projs], 0)
            b = None
            if any(m.bias is not None for m in projs):
                b = torch.cat([m.bias if m.bias is not None else m.weight.new_zeros(hid) for m in projs], 0)
            q, k, v = fs.split_heads(_LinearFn.apply(x, w, b), 3, nh)
        else:
            q = self.q_proj(x).reshape(bsz, seq, nh, hd).transpose(1, 2).contiguous()
            k = self.k_proj(x).reshape(bsz, seq, nkv, hd).transpose(1, 2)
            v = self.v_proj(x).reshape(bsz, seq, nkv, hd).transpose(1, 2)
            k = k.repeat_interleave(nh // nkv, dim=1).contiguous()
            v = v.repeat_interleave(nh // nkv, dim=1).contiguous()
        o = fs.flash_attention(q, k, v, causal=True)
        return self.out_proj(fs.merge_heads(o))


class GQABlock(nn.Module):
    """Pre-norm transformer block: x + attn(norm x), then + ffn_down(gelu(ffn_up(norm x)))."""

    def __init__(self, hidden_size: int, num_heads: int, num_kv_heads: int, ffn_mult: int = 4):
        super().__init__()
        self.attn_norm = LayerNorm(hidden_size, eps=LN_EPS)
        self.attn = GQAttention(hidden_size, num_heads, num_kv_heads)
        self.ffn_norm = LayerNorm(hidden_size, eps=LN_EPS)
        self.ffn_up = Linear(hidden_size, ffn_mult * hidden_size)
        self.ffn_down = Linear(ffn_mult * hidden_size, hidden_size)

    def forward(self, x):
        x = x + self.attn(self.attn_norm(x))
        return x + self.ffn(self.ffn_norm(x))

    def ffn(self, n):
        return self.ffn_down(F.gelu(self.ffn_up(n)))


class SequenceModel(nn.Module):
    """[batch, seq, embed] -> the last timestep's hidden state [batch, hidden]: an optional
    input projection, a stack of blocks, an optional final layer norm (the shape of the
    reference's MinGRU / DeltaNet / Mamba / GQA builders)."""

    def __init__(self, blocks_name: str, blocks, input_projection=None, final_norm=None, residual=False):
        super().__init__()
        if input_projection is not None:
            self.input_projection = input_projection
        setattr(self, blocks_name, nn.ModuleList(blocks))
        self._blocks_name = blocks_name
        if final_norm is not None:
            self.final_norm = final_norm
        self._residual = residual

    def sequence(self, x):
        """Hidden states of every timestep, [batch, seq, hidden]."""
        h = self.input_projection(x) if hasattr(self, "input_projection") else x
        for blk in getattr(self, self._blocks_name):
            h = h + blk(h) if self._residual else blk(h)
        return self.final_norm(h) if hasattr(self, "final_norm") else h

    def forward(self, x):
        return self.sequence(x)[:, -1]

    def load_reference_weights(self, weights: dict):
        """Load a reference weight file's ``weight.<layer>.<param>`` tensors (PyTorch layout)."""
        sd = {k[len("weight."):]: v for k, v in weights.items() if k.startswith("weight.")}
        ref = self.state_dict()
        missing = sorted(set(ref) - set(sd))
        extra = sorted(set(sd) - set(ref))
        if missing or extra:
            raise KeyError(f"weight keys do not match the model: missing {missing}, unexpected {extra}")
        self.load_state_dict({k: v.to(ref[k].dtype) for k, v in sd.items()})
        return self


def build(name: str, *, embed_size: int, hidden_size: int | None = None, num_layers: int = 2,
          num_heads: int = 4, num_kv_heads: int | None = None, state_size: int = 16, expand_factor: int = 2,
          conv_size: int = 4, use_short_conv: bool = True) -> SequenceModel:
    """``Edifice.build(name, opts)`` for the sequence-mixing families on the fused path.

    name: "min_gru", "min_lstm", "mamba", "delta_net", "gated_delta_net" or "gqa".  hidden_size defaults
    to embed_size; an input projection is added when they differ."""
    hidden = hidden_size or embed_size
    proj = Linear(embed_size, hidden) if hidden != embed_size else None
    if name == "min_gru":
        return SequenceModel("layers", [MinGRULayer(hidden) for _ in range(num_layers)], proj,
                             LayerNorm(hidden, eps=LN_EPS))
    if name == "min_lstm":  # min_lstm.ex:113-162 (the unfused layer stack)
        return SequenceModel("layers", [MinLSTMLayer(hidden) for _ in range(num_layers)], proj,
                             LayerNorm(hidden, eps=LN_EPS))
    if name == "delta_net":
        return SequenceModel("layers", [DeltaNetLayer(hidden, num_heads) for _ in range(num_layers)], proj,
                             LayerNorm(hidden, eps=LN_EPS))
    if name == "gated_delta_net":
        return SequenceModel("layers", [GatedDeltaNetLayer(hidden, num_heads, use_short_conv, conv_size)
                                        for _ in range(num_layers)], proj, LayerNorm(hidden, eps=LN_EPS))
    if name == "mamba":
        return SequenceModel("blocks", [MambaBlock(hidden, state_size, expand_factor, conv_size)
                                        for _ in range(num_layers)], proj, None, residual=True)
    if name == "gqa":
        return SequenceModel("blocks", [GQABlock(hidden, num_heads, num_kv_heads or num_heads)
                                        for _ in range(num_layers)], proj, LayerNorm(hidden, eps=LN_EPS))
    raise ValueError(f"unknown block family {name!r}")


class HybridDecoder(nn.Module):
    """Decoder stack mixing the three fused paths (the hybrid of the benchmark's config 5):
    token embedding -> Mamba blocks (residual) -> DeltaNet layers -> causal attention + FFN
    blocks -> final layer norm -> LM head, with a next-token cross-entropy ``loss``."""

    def __init__(self, vocab_size: int = 32000, embed_size: int = 1024, mamba_layers: int = 4,
                 delta_layers: int = 2, attn_layers: int = 2, num_heads: int = 8, state_size: int = 16,
                 expand_factor: int = 2, conv_size: int = 4):
        super().__init__()
        self.embed = Embedding(vocab_size, embed_size)
        self.mamba = nn.ModuleList(MambaBlock(embed_size, state_size, expand_factor, conv_size)
                                   for _ in range(mamba_layers))
        self.delta = nn.ModuleList(DeltaNetLayer(embed_size, num_heads) for _ in range(delta_layers))
        self.attn = nn.ModuleList(GQABlock(embed_size, num_heads, num_heads) for _ in range(attn_layers))
        self.final_norm = LayerNorm(embed_size, eps=LN_EPS)
        self.lm_head = Linear(embed_size, vocab_size, bias=False)

    def forward(self, tokens: torch.Tensor) -> torch.Tensor:
        # the stack as (norm, mix) stages h <- h + mix(norm h): each residual add runs with the
        # next stage's norm (or the final norm) in one pass, fs.add_layer_norm
        stages = [(b.norm, b.mix) for b in self.mamba] + [(b.norm, b.mix) for b in self.delta]
        for b in self.attn:
            stages += [(b.attn_norm, b.attn), (b.ffn_norm, b.ffn)]
        h = self.embed(tokens)
        n = stages[0][0](h)
        for i, (_, mix) in enumerate(stages):
            nxt = stages[i + 1][0] if i + 1 < len(stages) else self.final_norm
            h, n = fs.add_layer_norm(h, mix(n), nxt.weight, nxt.bias, nxt.eps)
        return self.lm_head(n)

    def loss(self, tokens: torch.Tensor) -> torch.Tensor:
        """Mean next-token cross entropy over tokens[:, 1:] (logits reduced in float32)."""
        logits = self.forward(tokens[:, :-1])
        return fs.cross_entropy(logits.reshape(-1, logits.shape[-1]), tokens[:, 1:].reshape(-1))
