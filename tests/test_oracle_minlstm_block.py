"""Pin of the oracle's MinLSTM model (oracle/blocks.min_lstm_model), CPU only.  No reference
fixture exists for MinLSTM; the layer is written out a second way from the reference source,
at T = 2:

  min_lstm.ex:267-292  pre-norm -> forget, input, candidate projections -> scan -> residual
  min_lstm.ex:304-334  f = sigmoid(forget), i = sigmoid(input), s = f + (i + 1e-6),
                       c_t = (f / s) c_{t-1} + (i / s) cand_t, c_0 = 0
  min_lstm.ex:152-162  final layer norm, last timestep

so c_1 = (i_1 / s_1) cand_1 and c_2 = (f_2 / s_2) c_1 + (i_2 / s_2) cand_2.  Every gradient of
the oracle (its hand-derived scan backward inside torch autograd) is checked against autograd
of the written-out form, and two misreadings (the gates swapped; no normalisation) are
asserted to differ."""
import numpy as np
import pytest
import torch

from oracle import blocks as ob

HID, LAYERS = 5, 2


def _weights(rng):
    w = {}
    for li in range(LAYERS):
        p = f"weight.layers.{li}"
        w[p + ".norm.weight"] = 1.0 + 0.2 * rng.normal(size=HID)
        w[p + ".norm.bias"] = 0.1 * rng.normal(size=HID)
        for n in ("forget", "input", "candidate"):
            w[f"{p}.{n}.weight"] = 0.6 * rng.normal(size=(HID, HID))
            w[f"{p}.{n}.bias"] = 0.3 * rng.normal(size=HID)
    w["weight.final_norm.weight"] = 1.0 + 0.2 * rng.normal(size=HID)
    w["weight.final_norm.bias"] = 0.1 * rng.normal(size=HID)
    return {k: torch.tensor(v, dtype=torch.float64, requires_grad=True) for k, v in w.items()}


def _layer_norm(x, g, b):
    mu = x.sum(-1, keepdim=True) / x.shape[-1]
    var = ((x - mu) ** 2).sum(-1, keepdim=True) / x.shape[-1]
    return (x - mu) / torch.sqrt(var + ob.LN_EPS) * g + b


def _sig(x):
    return 1 / (1 + torch.exp(-x))


def _model(w, x, variant=None):
    h = x
    for li in range(LAYERS):
        p = f"weight.layers.{li}"
        n = _layer_norm(h, w[p + ".norm.weight"], w[p + ".norm.bias"])
        lin = {k: n @ w[f"{p}.{k}.weight"].T + w[f"{p}.{k}.bias"] for k in ("forget", "input", "candidate")}
        f, i, cand = _sig(lin["forget"]), _sig(lin["input"]), lin["candidate"]
        if variant == "swapped":
            f, i = i, f
        s = f + (i + 1e-6)
        fn, inn = (f, i) if variant == "unnormalised" else (f / s, i / s)
        c1 = inn[:, 0] * cand[:, 0]
        c2 = fn[:, 1] * c1 + inn[:, 1] * cand[:, 1]
        h = h + torch.stack([c1, c2], 1)
    return _layer_norm(h, w["weight.final_norm.weight"], w["weight.final_norm.bias"])[:, -1]


@pytest.mark.parametrize("seed", [0, 1])
def test_min_lstm_model_matches_written_out_layer(seed):
    rng = np.random.default_rng(seed)
    w = _weights(rng)
    x = torch.tensor(rng.normal(size=(3, 2, HID)), dtype=torch.float64, requires_grad=True)
    r = torch.tensor(rng.normal(size=(3, HID)), dtype=torch.float64)
    got = ob.min_lstm_model(w, x, ob.differentiable_oracle_ops())
    want = _model(w, x)
    assert torch.allclose(got, want, rtol=1e-12, atol=1e-12), (got - want).abs().max()
    names = sorted(w)
    g_got = torch.autograd.grad((got * r).sum(), [x] + [w[k] for k in names])
    g_want = torch.autograd.grad((want * r).sum(), [x] + [w[k] for k in names])
    for name, a, b in zip(["input"] + names, g_got, g_want):
        assert float((a - b).abs().max()) / max(float(b.abs().max()), 1e-12) < 1e-10, name


@pytest.mark.parametrize("variant", ["swapped", "unnormalised"])
def test_min_lstm_misreadings_differ(variant):
    rng = np.random.default_rng(3)
    w = _weights(rng)
    x = torch.tensor(rng.normal(size=(3, 2, HID)), dtype=torch.float64)
    with torch.no_grad():
        ref = ob.min_lstm_model(w, x, ob.differentiable_oracle_ops())
        alt = _model(w, x, variant)
    assert float((alt - ref).abs().max() / ref.abs().max()) > 1e-3
