"""The decode-chain configuration has the expected shapes
and byte count: 28 Qwen3-0.6B layers + 151936-row head = 398,060,544
weight bytes per step, 197 projection launches (113 with fused q/k/v and
gate/up)."""
from edgerunner_amd.chain import ChainSpec


def test_chain_bytes_and_launches():
    s = ChainSpec()
    assert s.weight_bytes() == 398_060_544
    per_layer = ChainSpec(layers=1, vocab=0).weight_bytes()
    assert per_layer == 9_658_368
    assert s.launches(False) == 197 and s.launches(True) == 113
    names = [n for n, *_ in s.layer_projections()]
    assert names == ["q", "k", "v", "o", "gate", "up", "down"]
