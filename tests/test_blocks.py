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
