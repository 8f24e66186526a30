"""Block API (edifice_amd.blocks) without a GPU: every model the reference fixtures cover
has exactly the fixture's weight keys and shapes, so reference weight files load unchanged."""
import os

import pytest

from oracle import blocks as oracle_blocks
from tests.conftest import GOLDEN

FIXTURE_OPTS = {
    "min_gru": dict(embed_size=32, hidden_size=64),
    "delta_net": dict(embed_size=32, num_heads=4),
    "mamba": dict(embed_size=32, state_size=8),
    "gqa": dict(embed_size=32, num_heads=4, num_kv_heads=2),
}


@pytest.mark.parametrize("name", sorted(FIXTURE_OPTS))
def test_block_models_match_reference_weight_layout(name):
    from edifice_amd import blocks
    w = oracle_blocks.load_fixture(os.path.join(GOLDEN, f"{name}_random.safetensors"))
    model = blocks.build(name, **FIXTURE_OPTS[name])
    ref = {k[len("weight."):]: tuple(v.shape) for k, v in w.items() if k.startswith("weight.")}
    ours = {k: tuple(v.shape) for k, v in model.state_dict().items()}
    assert ours == ref
    model.load_reference_weights(w)  # loads without key errors


def test_gated_delta_net_block_layout():
    from edifice_amd import blocks
    m = blocks.build("gated_delta_net", embed_size=64, num_heads=4)
    sd = m.state_dict()
    assert tuple(sd["layers.0.qkvbag_proj.weight"].shape) == (6 * 64, 64)  # gated_delta_net.ex:249
    assert tuple(sd["layers.0.short_conv.weight"].shape) == (64, 1, 4)


def test_unknown_family_raises():
    from edifice_amd import blocks
    with pytest.raises(ValueError):
        blocks.build("nonexistent", embed_size=8)


def test_hybrid_decoder_oracle_covers_every_parameter():
    """The oracle's config-5 stack reads every HybridDecoder parameter under its own key and
    sends a gradient to each (the GPU test compares those gradients with the HIP model's)."""
    import numpy as np
    import torch

    from edifice_amd import blocks
    from oracle import blocks as ob

    torch.manual_seed(0)
    model = blocks.HybridDecoder(vocab_size=50, embed_size=32, num_heads=2)
    with torch.no_grad():  # softplus(dt) inside the [1e-3, 0.1] clip, else dt's gradient is masked to 0
        for blk in model.mamba:
            blk.dt_proj.bias.uniform_(-6.0, -2.5)
    w = {"weight." + k: v.detach().double().clone().requires_grad_() for k, v in model.state_dict().items()}
    tokens = torch.from_numpy(np.random.default_rng(0).integers(0, 50, size=(2, 9)))
    loss = ob.hybrid_decoder_loss(w, tokens, ob.differentiable_oracle_ops(), num_heads=2)
    loss.backward()
    assert np.isfinite(loss.item())
    names = {k for k, _ in model.named_parameters()}
    assert {k[len("weight."):] for k in w} == names
    assert all(w["weight." + k].grad is not None and w["weight." + k].grad.abs().max() > 0 for k in names)


def test_min_lstm_block_layout():
    """min_lstm.ex:267-292: per layer a norm and three hidden x hidden projections named
    forget, input, candidate (the names pack_block_weights reads, min_lstm.ex:212-219)."""
    from edifice_amd import blocks
    m = blocks.build("min_lstm", embed_size=24, hidden_size=32)
    sd = m.state_dict()
    assert tuple(sd["input_projection.weight"].shape) == (32, 24)
    for proj in ("forget", "input", "candidate"):
        assert tuple(sd[f"layers.1.{proj}.weight"].shape) == (32, 32)
    assert {k for k in sd if k.startswith("layers.0.")} == {
        f"layers.0.{n}.{p}" for n in ("norm", "forget", "input", "candidate") for p in ("weight", "bias")}
