"""Pin of the oracle's GatedDeltaNet model (oracle/blocks.gated_delta_net_model), CPU only.

No reference fixture exists for this family, so the whole layer is written out here a second
way, from the reference source line by line, at T = 2 where the recurrence has a closed form:

  gated_delta_net.ex:233-262  pre-norm (Axon.layer_norm) -> short causal depthwise conv
                              (padding [{K - 1, 0}], one group per channel) -> SiLU ->
                              dense to 6 x hidden -> recurrence -> dense -> residual
  gated_delta_net.ex:355-401  split order q, k, v, beta, alpha, gate; beta = sigmoid per
                              element; alpha = mean over the head of sigmoid(alpha_pre);
                              gate = swish(gate_pre) times the flattened heads; keys L2
                              normalised with 1e-6 inside the sqrt
  gated_delta_net.ex:318-345  per step: S <- alpha S; e = v - S k; S <- S + (beta e) k^T; o = S q
  gated_delta_net.ex:188-203  final layer norm, last timestep

With S_0 = 0 the two outputs of one head are
  o_1 = (b_1 v_1)(k_1 . q_1)
  o_2 = a_2 (b_1 v_1)(k_1 . q_2) + b_2 (v_2 - a_2 (b_1 v_1)(k_1 . k_2)) (k_2 . q_2)
(elementwise products with b, v vectors over the head's value rows).  Layer norm and the
convolution are written as explicit sums, not torch's modules.  The readings a mistake would
most plausibly make are built as variants of the same written-out layer and asserted to
differ from the oracle: alpha as sigmoid of the mean, two split orders, and the convolution
applied to q, k, v after the projection (as some gated-delta-net codes do).
"""
import numpy as np
import pytest
import torch

from oracle import blocks as ob

HID, HEADS, K, LAYERS = 6, 2, 4, 2
HD = HID // HEADS


def _weights(rng):
    w = {}
    for li in range(LAYERS):
        p = f"weight.layers.{li}"
        w[p + ".norm.weight"] = 1.0 + 0.2 * rng.normal(size=HID)
        w[p + ".norm.bias"] = 0.1 * rng.normal(size=HID)
        w[p + ".short_conv.weight"] = 0.6 * rng.normal(size=(HID, 1, K))
        w[p + ".short_conv.bias"] = 0.1 * rng.normal(size=HID)
        w[p + ".qkvbag_proj.weight"] = 0.5 * rng.normal(size=(6 * HID, HID))
        w[p + ".qkvbag_proj.bias"] = 0.1 * rng.normal(size=6 * HID)
        # alpha_pre spread within each head, so that mean(sigmoid) and sigmoid(mean) part
        w[p + ".qkvbag_proj.bias"][4 * HID:5 * HID] += np.tile([3.0, -1.5, 0.5], HEADS)
        w[p + ".out_proj.weight"] = 0.5 * rng.normal(size=(HID, HID))
        w[p + ".out_proj.bias"] = 0.1 * rng.normal(size=HID)
    w["weight.final_norm.weight"] = 1.0 + 0.2 * rng.normal(size=HID)
    w["weight.final_norm.bias"] = 0.1 * rng.normal(size=HID)
    return {k: torch.tensor(v, dtype=torch.float64, requires_grad=True) for k, v in w.items()}


def _layer_norm(x, g, b):
    mu = x.sum(-1, keepdim=True) / x.shape[-1]
    var = ((x - mu) ** 2).sum(-1, keepdim=True) / x.shape[-1]
    return (x - mu) / torch.sqrt(var + ob.LN_EPS) * g + b


def _causal_conv(x, wc, bc):
    """out[t, c] = bc[c] + sum_j wc[c, 0, j] x[t - (K - 1) + j, c], zero before t = 0."""
    seq = x.shape[1]
    cols = []
    for t in range(seq):
        acc = bc.expand(x.shape[0], -1)
        for j in range(K):
            s = t - (K - 1) + j
            if s >= 0:
                acc = acc + wc[:, 0, j] * x[:, s]
        cols.append(acc)
    return torch.stack(cols, 1)


def _silu(x):
    return x / (1 + torch.exp(-x))


def _sig(x):
    return 1 / (1 + torch.exp(-x))


ORDER = ("q", "k", "v", "beta", "alpha", "gate")  # gated_delta_net.ex:360-365


def _layer(w, p, x, alpha_of="mean_sigmoid", order=ORDER, conv="before"):
    bsz, seq, _ = x.shape
    assert seq == 2
    n = _layer_norm(x, w[p + ".norm.weight"], w[p + ".norm.bias"])
    wc, bc = w[p + ".short_conv.weight"], w[p + ".short_conv.bias"]
    a = _silu(_causal_conv(n, wc, bc)) if conv == "before" else n
    proj = a @ w[p + ".qkvbag_proj.weight"].T + w[p + ".qkvbag_proj.bias"]
    part = {name: proj[..., i * HID:(i + 1) * HID] for i, name in enumerate(order)}
    if conv == "after":  # the variant: conv + SiLU on q, k, v after the projection
        for name in ("q", "k", "v"):
            part[name] = _silu(_causal_conv(part[name], wc, bc))
    heads = []
    for h in range(HEADS):
        s = slice(h * HD, (h + 1) * HD)
        q1, q2 = part["q"][:, 0, s], part["q"][:, 1, s]
        k1, k2 = (part["k"][:, t, s] / torch.sqrt((part["k"][:, t, s] ** 2).sum(-1, keepdim=True) + 1e-6)
                  for t in (0, 1))
        v1, v2 = part["v"][:, 0, s], part["v"][:, 1, s]
        b1, b2 = _sig(part["beta"][:, 0, s]), _sig(part["beta"][:, 1, s])
        if alpha_of == "mean_sigmoid":
            a2 = _sig(part["alpha"][:, 1, s]).mean(-1, keepdim=True)
        else:
            a2 = _sig(part["alpha"][:, 1, s].mean(-1, keepdim=True))
        dot = lambda u, v: (u * v).sum(-1, keepdim=True)  # noqa: E731
        o1 = b1 * v1 * dot(k1, q1)
        o2 = a2 * b1 * v1 * dot(k1, q2) + b2 * (v2 - a2 * b1 * v1 * dot(k1, k2)) * dot(k2, q2)
        heads.append(torch.stack([o1, o2], 1))
    raw = torch.cat(heads, -1)
    g = part["gate"]
    out = (g * _sig(g) * raw) @ w[p + ".out_proj.weight"].T + w[p + ".out_proj.bias"]
    return x + out


def _model(w, x, **variant):
    h = x
    for li in range(LAYERS):
        h = _layer(w, f"weight.layers.{li}", h, **variant)
    return _layer_norm(h, w["weight.final_norm.weight"], w["weight.final_norm.bias"])[:, -1]


def _oracle(w, x):
    return ob.gated_delta_net_model(w, x, ob.differentiable_oracle_ops(), num_heads=HEADS, conv_size=K)


@pytest.mark.parametrize("seed", [0, 1])
def test_gated_delta_net_model_matches_written_out_layer(seed):
    rng = np.random.default_rng(seed)
    w = _weights(rng)
    x = torch.tensor(rng.normal(size=(2, 2, HID)), dtype=torch.float64, requires_grad=True)
    r = torch.tensor(rng.normal(size=(2, HID)), dtype=torch.float64)
    got = _oracle(w, x)
    want = _model(w, x)
    assert torch.allclose(got, want, rtol=1e-12, atol=1e-12), (got - want).abs().max()
    # every gradient: the oracle's hand-derived scan backward inside torch autograd, against
    # autograd through the written-out closed form
    names = sorted(w)
    g_got = torch.autograd.grad((got * r).sum(), [x] + [w[k] for k in names])
    g_want = torch.autograd.grad((want * r).sum(), [x] + [w[k] for k in names])
    for name, a, b in zip(["input"] + names, g_got, g_want):
        scale = max(float(b.abs().max()), 1e-12)
        assert float((a - b).abs().max()) / scale < 1e-10, name


@pytest.mark.parametrize("variant", [
    dict(alpha_of="sigmoid_mean"),
    dict(order=("q", "k", "v", "alpha", "beta", "gate")),
    dict(order=("gate", "q", "k", "v", "beta", "alpha")),
    dict(conv="after"),
], ids=["sigmoid_of_mean", "beta_alpha_swapped", "gate_first", "conv_after_projection"])
def test_plausible_misreadings_differ(variant):
    rng = np.random.default_rng(2)
    w = _weights(rng)
    x = torch.tensor(rng.normal(size=(2, 2, HID)), dtype=torch.float64)
    with torch.no_grad():
        ref = _oracle(w, x)
        alt = _model(w, x, **variant)
    rel = float((alt - ref).abs().max() / ref.abs().max())
    assert rel > 1e-3, f"variant {variant} indistinguishable from the oracle (rel {rel:.1e})"
