"""GPU parity at the benchmark configurations' full sizes.

The HIP kernels run the whole configuration (every batch row, head and channel tile, the
full sequence, so every chunk carry, checkpoint and partial reduction of the benchmarked
launch is exercised); the float64 oracle then checks slices it can finish in seconds.
Slices are independent of the rest of the launch by construction: heads of the delta rule
and of attention never interact, and for the selective scan's channel sums (dB, dC) and
batch sums (dA, dD) the inputs outside the checked slice are zeroed where they would
contribute (x = 0 makes a channel's state, and so its share of every such sum, zero).
Tolerances are the north-star ones, 1e-4 (f32) and 2e-2 (bf16), relative to the largest
expected magnitude.
"""
import numpy as np
import pytest
import torch

from oracle import scans
from tests.conftest import assert_close
from tests.gpu_util import TOL, announce, host, rounded, to_dev

pytestmark = pytest.mark.gpu

BF16, F32 = torch.bfloat16, torch.float32


def test_c2_selective_scan_full_size_backward(rng):
    """Config 2 (B=8, T=2048, D=1536, N=16; u, dt, z bf16; A, B, C, D f32), forward and
    backward at full size.  Batch row 5, channels 0-255, is checked against the oracle over
    the whole sequence: y, dx, ddt, dz there; dB and dC of row 5 (x = 0 on row 5's other
    channels, so only the checked channels feed those channel sums); dA and dD of channels
    0-255 (x = 0 on those channels in every other row, so only row 5 feeds those batch sums).
    Every other (row, channel) carries random data, so all 24 channel tiles and all 128
    checkpoints per row do real work."""
    from edifice_amd import fused_scan as fs
    from tests.test_gpu_selective_scan import make_inputs
    bsz, T, D, N, b0, W = 8, 2048, 1536, 16, 5, 256
    announce("c2_full_backward", B=bsz, T=T, D=D, N=N)
    x, dt, A, B, C, Dv, z = make_inputs(rng, bsz, T, D, N)
    x[b0, :, W:] = 0.0
    x[np.arange(bsz) != b0, :, :W] = 0.0
    dy = rng.normal(size=x.shape)
    tx, tdt, tz = (to_dev(a, BF16).requires_grad_() for a in (x, dt, z))
    tA, tB, tC, tD = (to_dev(a, F32).requires_grad_() for a in (A, B, C, Dv))
    y = fs.selective_scan(tx, tdt, tA, tB, tC, tD, tz)
    y.backward(to_dev(dy, BF16))
    torch.cuda.synchronize()

    sl = (slice(b0, b0 + 1), slice(None), slice(0, W))
    xr, dtr, zr, dyr = (rounded(a, BF16)[sl] for a in (x, dt, z, dy))
    tol = TOL[BF16]
    assert_close(host(y)[sl], scans.selective_scan(xr, dtr, A[:W], B[b0:b0 + 1], C[b0:b0 + 1], Dv[:W], zr), tol, "y")
    g = scans.selective_scan_backward(xr, dtr, A[:W], B[b0:b0 + 1], C[b0:b0 + 1], dyr, Dv[:W], zr)
    assert_close(host(tx.grad)[sl], g["dx"], tol, "dx")
    assert_close(host(tdt.grad)[sl], g["ddt"], tol, "ddt")
    assert_close(host(tz.grad)[sl], g["dz"], tol, "dz")
    assert_close(host(tB.grad)[b0:b0 + 1], g["dB"], tol, "dB row 5")
    assert_close(host(tC.grad)[b0:b0 + 1], g["dC"], tol, "dC row 5")
    assert_close(host(tA.grad)[:W], g["dA"], tol, "dA channels 0-255")
    assert_close(host(tD.grad)[:W], g["dD"], tol, "dD channels 0-255")


def test_c3_gated_delta_rule_full_size(rng):
    """Config 3 (B=4, H=16, T=4096, d=128, chunk 64, bf16, per-head beta, gated) through the
    chunked MFMA path at full size, forward and backward: heads (b=0, h=0) and (b=3, h=15)
    against the oracle over all 64 chunks (the state and its gradient carried chunk to chunk)."""
    from edifice_amd import fused_scan as fs
    from tests.test_gpu_delta_rule import make_inputs
    Bn, T, H, d = 4, 4096, 16, 128
    announce("c3_full", B=Bn, T=T, H=H, d=d)
    q, k, v, beta, alpha = make_inputs(rng, Bn, T, H, d, True, True)
    do = rng.normal(size=v.shape)
    tq, tk, tv, tb, ta = (to_dev(a, BF16).requires_grad_() for a in (q, k, v, beta, alpha))
    out = fs.gated_delta_net_scan(tq, tk, tv, tb, ta)
    out.backward(to_dev(do, BF16))
    torch.cuda.synchronize()
    tol = TOL[BF16]
    for b, h in ((0, 0), (3, 15)):
        s4 = (slice(b, b + 1), slice(None), slice(h, h + 1))
        qr, kr, vr, dor = (rounded(a, BF16)[s4] for a in (q, k, v, do))
        br, ar = rounded(beta, BF16)[s4], rounded(alpha, BF16)[s4]
        assert_close(host(out)[s4], scans.delta_rule(qr, kr, vr, br, ar), tol, f"o ({b},{h})", mfma_bf16=True)
        g = scans.delta_rule_backward(qr, kr, vr, br, dor, ar)
        for name, t in (("dq", tq), ("dk", tk), ("dv", tv), ("dbeta", tb), ("dalpha", ta)):
            assert_close(host(t.grad)[s4], g[name], tol, f"{name} ({b},{h})", mfma_bf16=True)


def test_c4_flash_attention_full_grid(rng):
    """Config 4 (B=4, H=32, T=4096, d=128, bf16, causal) on the full grid, forward and
    backward: heads (0, 0) and (3, 31), the first and last workgroups of the remapped grid,
    against the oracle."""
    from edifice_amd import fused_scan as fs
    Bn, H, T, d = 4, 32, 4096, 128
    announce("c4_full_grid", B=Bn, H=H, T=T, d=d)
    std = 128 ** -0.25
    q, k, v, do = (rng.normal(scale=std, size=(Bn, H, T, d)) for _ in range(4))
    tq, tk, tv = (to_dev(a, BF16).requires_grad_() for a in (q, k, v))
    out = fs.flash_attention(tq, tk, tv, causal=True)
    out.backward(to_dev(do, BF16))
    torch.cuda.synchronize()
    tol = TOL[BF16]
    for b, h in ((0, 0), (3, 31)):
        s = (slice(b, b + 1), slice(h, h + 1))
        qr, kr, vr, dor = (rounded(a, BF16)[s] for a in (q, k, v, do))
        assert_close(host(out)[s], scans.flash_attention(qr, kr, vr, causal=True), tol, f"o ({b},{h})",
                     mfma_bf16=True)
        dq, dk, dv = scans.flash_attention_backward(qr, kr, vr, dor, causal=True)
        for name, t, e in (("dq", tq, dq), ("dk", tk, dk), ("dv", tv, dv)):
            assert_close(host(t.grad)[s], e, tol, f"{name} ({b},{h})", mfma_bf16=True)


def _hybrid(dtype, seed=5):
    """A reduced config-5 decoder (4 Mamba + 2 DeltaNet + 2 attention blocks, head_dim 128 as
    in config 5; embed 256, vocab 1000) and its float64 copy of the weights for the oracle.
    The Mamba dt biases are drawn so softplus(dt) mostly falls inside the [1e-3, 0.1] clip,
    which keeps the dt-mean discretisation and its gradient active."""
    from edifice_amd import blocks
    torch.manual_seed(seed)
    model = blocks.HybridDecoder(vocab_size=1000, embed_size=256, num_heads=2)
    with torch.no_grad():
        for blk in model.mamba:
            blk.dt_proj.bias.uniform_(-6.0, -2.5)
    w = {"weight." + k: v.detach().double().clone().requires_grad_() for k, v in model.state_dict().items()}
    return model.to("cuda", dtype), w


def _grads_close(pairs, tol, what, floor_frac=1e-3):
    """Each gradient's max error against the larger of its own scale and ``floor_frac`` of the
    largest gradient, since some exact gradients vanish (the attention key bias: softmax
    ignores a shift shared by all keys, so its gradient is rounding noise around 0).  The
    floor is 1e-3 in float32 and 1e-2 in bfloat16, whose 8-bit mantissa cannot resolve a sum
    below ~4e-3 of its terms' scale.  Returns the worst ratio."""
    floor = floor_frac * max(float(e.abs().max()) for _, _, e in pairs)
    worst = 0.0
    for name, got, exp in pairs:
        got, exp = got.detach().double().cpu().numpy(), exp.detach().double().cpu().numpy()
        err = float(np.abs(got - exp).max()) / max(float(np.abs(exp).max()), floor)
        worst = max(worst, err)
        assert err <= tol, f"{what} d_{name}: rel err {err:.3e} > {tol:.0e}"
    return worst


def test_c5_hybrid_decoder_f32_matches_oracle():
    """Config 5's model at reduced size in float32: the next-token loss and every parameter
    gradient of the HIP model against the whole model in float64 on the oracle ops
    (hand-derived backward of each op), at the f32 tolerance."""
    from oracle import blocks as ob
    announce("c5_hybrid_reduced_f32")
    model, w = _hybrid(F32)
    tokens = torch.from_numpy(np.random.default_rng(11).integers(0, 1000, size=(2, 257)))
    loss = model.loss(tokens.cuda())
    loss.backward()
    ref = ob.hybrid_decoder_loss(w, tokens, ob.differentiable_oracle_ops(), num_heads=2)
    ref.backward()
    assert_close(np.array([loss.item()]), np.array([ref.item()]), TOL[F32], "loss")
    pairs = [(k, p.grad, w["weight." + k].grad) for k, p in model.named_parameters()]
    worst = _grads_close(pairs, TOL[F32], "f32")
    print(f"c5 f32: loss {loss.item():.6f} vs {ref.item():.6f}, worst grad err {worst:.2e}", flush=True)


class _OracleOps:
    """Stand-in for edifice_amd.fused_scan inside edifice_amd.blocks: the same calls served
    by the oracle's autograd ops (float64 inside, inputs' dtypes outside)."""

    @staticmethod
    def delta_net_scan(q, k, v, beta):
        from oracle import blocks as ob
        return ob._OracleDelta.apply(q, k, v, beta)

    @staticmethod
    def flash_attention(q, k, v, causal=False):
        from oracle import blocks as ob
        assert causal
        return ob._OracleCausalAttention.apply(q, k, v)

    @staticmethod
    def cross_entropy(logits, targets):
        return torch.nn.functional.cross_entropy(logits.float(), targets)

    @staticmethod
    def causal_conv1d_silu(x, weight, bias=None):
        from tests.gpu_util import torch_causal_conv_silu
        return torch_causal_conv_silu(x, weight, bias)

    @staticmethod
    def layer_norm(x, weight=None, bias=None, eps=1e-5):
        return torch.nn.functional.layer_norm(x, (x.shape[-1],), weight, bias, eps)

    @staticmethod
    def split_heads(x, parts, num_heads):
        bsz, seq, width = x.shape
        return x.reshape(bsz, seq, parts, num_heads, -1).permute(2, 0, 3, 1, 4).contiguous().unbind(0)

    @staticmethod
    def merge_heads(x):
        return x.transpose(1, 2).reshape(x.shape[0], x.shape[2], -1)

    @staticmethod
    def embedding(ids, weight, padding_idx=None):
        return torch.nn.functional.embedding(ids, weight, padding_idx)

    @staticmethod
    def add_layer_norm(x, res, weight=None, bias=None, eps=1e-5):
        s = x + res
        return s, torch.nn.functional.layer_norm(s, (s.shape[-1],), weight, bias, eps)

    @staticmethod
    def mamba_ssm(xa, w_proj, b_proj, w_dt, b_dt, a, z, state_size):
        from oracle import blocks as ob
        proj = torch.nn.functional.linear(xa, w_proj, b_proj)
        n2 = 2 * state_size
        bc = proj[..., :n2].float()
        b, c = bc[..., :state_size].contiguous(), bc[..., state_size:].contiguous()
        dt = torch.nn.functional.softplus(torch.nn.functional.linear(proj[..., n2:], w_dt, b_dt))
        return ob._OracleSelectiveScanMean.apply(xa, dt.contiguous(), a, b, c, z)

    @staticmethod
    def weight_grad(dy, x, out=None):
        r = dy.t().mm(x)
        return r if out is None else out.copy_(r)

    @staticmethod
    def bias_grad(dy, out=None):
        r = dy.sum(0)
        return r if out is None else out.copy_(r)

    @staticmethod
    def delta_net_split(proj, num_heads, eps=1e-6):
        q, k, v, bpre = torch.split(proj, proj.shape[-1] // 4, dim=-1)
        heads = (lambda t: t.reshape(*t.shape[:-1], num_heads, -1).contiguous())
        k = heads(k)
        return heads(q), k / torch.sqrt((k * k).sum(-1, keepdim=True) + eps), heads(v), heads(torch.sigmoid(bpre))

    @staticmethod
    def l2_normalize(x, eps=1e-6):
        return x / torch.sqrt((x * x).sum(-1, keepdim=True) + eps)


def test_c5_hybrid_decoder_bf16_matches_oracle_ops(monkeypatch):
    """Config 5's model at reduced size in bfloat16 (the benchmark's precision): the same bf16
    model (same weights, the same torch bf16 GEMMs) run once on the HIP ops and once with the
    oracle ops (and torch's layer norm, softplus, key norm, convolution, weight- and bias-gradient
    products and loss) swapped in, so the two runs differ only in the ops edifice_amd fuses.  Loss and every
    parameter gradient within the bf16 tolerance."""
    import copy

    from edifice_amd import blocks
    announce("c5_hybrid_reduced_bf16")
    model, _ = _hybrid(BF16)
    ref_model = copy.deepcopy(model)
    tokens = torch.from_numpy(np.random.default_rng(11).integers(0, 1000, size=(2, 257))).cuda()
    loss = model.loss(tokens)
    loss.backward()
    monkeypatch.setattr(blocks, "fs", _OracleOps)
    ref = ref_model.loss(tokens)
    ref.backward()
    assert_close(np.array([loss.item()]), np.array([ref.item()]), TOL[BF16], "loss")
    refp = dict(ref_model.named_parameters())
    pairs = [(k, p.grad, refp[k].grad) for k, p in model.named_parameters()]
    worst = _grads_close(pairs, TOL[BF16], "bf16", floor_frac=1e-2)
    print(f"c5 bf16: loss {loss.item():.6f} vs {ref.item():.6f}, worst grad err {worst:.2e}", flush=True)
