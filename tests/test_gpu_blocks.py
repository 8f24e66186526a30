"""GPU parity of the block API (edifice_amd.blocks): each model runs the
fused HIP ops for its recurrence and is checked
  * forward against the reference's own fixture (expected_output of
    test/fixtures/numerical/*_random.safetensors), and
  * backward (input and every parameter gradient) against the numpy oracle blocks in
    float64 with the hand-derived backward of each op (oracle/blocks.py).
Tolerance: the north-star 1e-4 (f32) relative to the largest magnitude."""
import os

import numpy as np
import pytest
import torch

from oracle import blocks as ob
from tests.conftest import GOLDEN, assert_close
from tests.gpu_util import announce
from tests.test_blocks import FIXTURE_OPTS

pytestmark = pytest.mark.gpu

ORACLE_MODELS = {"min_gru": ob.min_gru_model, "delta_net": ob.delta_net_model, "mamba": ob.mamba_model,
                 "gqa": ob.gqa_model, "gated_delta_net": ob.gated_delta_net_model, "min_lstm": ob.min_lstm_model}


def _grads_match(model, w_ref, x_gpu, x_ref, name, seed=7):
    out = model(x_gpu)
    r = torch.from_numpy(np.random.default_rng(seed).normal(size=tuple(out.shape)))
    (out * r.to(out)).sum().backward()
    ref_out = ORACLE_MODELS[name](w_ref, x_ref, ob.differentiable_oracle_ops())
    (ref_out * r).sum().backward()
    pairs = [("d_input", x_gpu.grad, x_ref.grad)] + [
        ("d_" + k, p.grad, w_ref["weight." + k].grad) for k, p in model.named_parameters()]
    # Some exact gradients vanish (a bias shared by all keys only shifts every score of a
    # query, which softmax ignores): each error is measured against the larger of that
    # gradient's own scale and 1e-3 of the model's largest gradient.
    floor = 1e-3 * max(float(e.abs().max()) for _, _, e in pairs)
    for what, got, exp in pairs:
        got, exp = got.detach().cpu().double().numpy(), exp.numpy()
        err = float(np.abs(got - exp).max()) / max(float(np.abs(exp).max()), floor)
        assert err <= 1e-4, f"{name} {what}: rel err {err:.3e} > 1e-4"


@pytest.mark.parametrize("name", sorted(FIXTURE_OPTS))
def test_block_model_matches_reference_fixture(name):
    from edifice_amd import blocks
    announce("block_fixture", model=name)
    w = ob.load_fixture(os.path.join(GOLDEN, f"{name}_random.safetensors"))
    model = blocks.build(name, **FIXTURE_OPTS[name]).load_reference_weights(w).to("cuda", torch.float32)
    x = w["input.state_sequence"].float().cuda().requires_grad_()
    with torch.no_grad():
        assert_close(model(x).cpu().numpy(), w["expected_output"].numpy(), 1e-4, f"{name} forward")
    w_ref = {k: (v.clone().requires_grad_() if k.startswith("weight.") else v) for k, v in w.items()}
    x_ref = w["input.state_sequence"].clone().requires_grad_()
    _grads_match(model, w_ref, x, x_ref, name)


def test_gated_delta_net_block_matches_oracle():
    """No reference fixture covers GatedDeltaNet: random weights, checked against the oracle block."""
    from edifice_amd import blocks
    announce("block_gated_delta_net")
    torch.manual_seed(3)
    model = blocks.build("gated_delta_net", embed_size=32, num_heads=4)
    w_ref = {"weight." + k: v.detach().double().clone().requires_grad_() for k, v in model.state_dict().items()}
    model = model.to("cuda", torch.float32)
    xn = torch.randn(2, 11, 32, dtype=torch.float64)
    x = xn.float().cuda().requires_grad_()
    x_ref = xn.clone().requires_grad_()
    with torch.no_grad():
        ref = ob.gated_delta_net_model({k: v.detach() for k, v in w_ref.items()}, xn, ob.differentiable_oracle_ops())
        assert_close(model(x).cpu().numpy(), ref.numpy(), 1e-4, "gated_delta_net forward")
    _grads_match(model, w_ref, x, x_ref, "gated_delta_net")


def test_min_lstm_block_matches_oracle():
    """No reference fixture covers MinLSTM: random weights (embed == hidden, two layers),
    checked against the oracle block (pinned by a written-out T = 2 form on the CPU),
    forward and every gradient."""
    from edifice_amd import blocks
    announce("block_min_lstm")
    torch.manual_seed(4)
    model = blocks.build("min_lstm", embed_size=48)
    w_ref = {"weight." + k: v.detach().double().clone().requires_grad_() for k, v in model.state_dict().items()}
    model = model.to("cuda", torch.float32)
    xn = torch.randn(3, 37, 48, dtype=torch.float64)
    x = xn.float().cuda().requires_grad_()
    x_ref = xn.clone().requires_grad_()
    with torch.no_grad():
        ref = ob.min_lstm_model({k: v.detach() for k, v in w_ref.items()}, xn, ob.differentiable_oracle_ops())
        assert_close(model(x).cpu().numpy(), ref.numpy(), 1e-4, "min_lstm forward")
    _grads_match(model, w_ref, x, x_ref, "min_lstm")


@pytest.mark.parametrize("name", ["min_gru", "mamba", "gqa"])
def test_block_model_bf16_forward(name):
    """The same fixtures through bf16 models (dense layers and scans in bf16, f32 math in the
    kernels): within the north-star bf16 tolerance 2e-2."""
    from edifice_amd import blocks
    announce("block_bf16", model=name)
    w = ob.load_fixture(os.path.join(GOLDEN, f"{name}_random.safetensors"))
    model = blocks.build(name, **FIXTURE_OPTS[name]).load_reference_weights(w).to("cuda", torch.bfloat16)
    with torch.no_grad():
        out = model(w["input.state_sequence"].cuda().to(torch.bfloat16)).float().cpu().numpy()
    # a whole bf16 model against the float32 fixture: normalised max-abs only (see assert_close)
    assert_close(out, w["expected_output"].numpy(), 2e-2, f"{name} bf16 forward", elementwise=False)
