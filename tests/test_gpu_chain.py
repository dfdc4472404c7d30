"""Decode-step projection chain (28 Qwen3-0.6B layers in a
Q4_K_M mix + 151936-row Q6_K head) on the GPU: every projection of the first
and last layer and the head against the CPU oracle (1e-3 relative L2); the
fused form (triple q/k/v, dual gate/up) bit-identical to per-projection
launches; graph replays -- three, with eager work in between, outputs cleared
before each -- bit-identical to the eager encode."""
import numpy as np
import pytest

from edgerunner_amd.chain import ChainSpec, DecodeChain, make_inputs, make_weights
from oracle import ref
from conftest import rel_l2

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def chain(ctx):
    spec = ChainSpec()
    ws, xs = make_weights(spec), make_inputs(spec)
    s = ctx.stream()
    ch = DecodeChain(ctx, spec, ws, xs, s)
    s.synchronize()
    yield spec, ws, xs, ch, s
    ch.free()
    s.destroy()


def clear(ch, s):
    for b in ch.y.values():
        b.upload(np.zeros(b.length // 4, np.float32), stream=s)


def test_chain_matches_oracle(chain):
    spec, ws, xs, ch, s = chain
    clear(ch, s)
    ch.encode(s, fused=False)
    s.synchronize()
    out = ch.outputs(s)
    th = ref.max_threads()
    keys = [(l, n) for l in (0, spec.layers - 1) for n, *_ in spec.layer_projections()] + [(-1, "head")]
    for key in keys:
        f, M, K, src = ch.meta[key]
        exp = ref.gemv(f, ws[key], xs[src], M, K, threads=th)
        err = rel_l2(out[key], exp)
        assert err < 1e-3, (key, err)
    assert all(np.all(np.isfinite(v)) for v in out.values())


def test_fused_equals_per_projection(chain):
    spec, ws, xs, ch, s = chain
    clear(ch, s)
    ch.encode(s, fused=False)
    s.synchronize()
    a = ch.outputs(s)
    clear(ch, s)
    ch.encode(s, fused=True)
    s.synchronize()
    b = ch.outputs(s)
    for k in a:
        assert np.array_equal(a[k], b[k]), k


@pytest.mark.parametrize("fused", [False, True])
def test_graph_replays_equal_eager(chain, fused):
    spec, ws, xs, ch, s = chain
    clear(ch, s)
    ch.encode(s, fused=fused)
    s.synchronize()
    eager = ch.outputs(s)
    g = ch.capture(s, fused=fused)
    try:
        for rep in range(3):
            clear(ch, s)
            g.launch(s)
            s.synchronize()
            got = ch.outputs(s)
            for k in eager:
                assert np.array_equal(got[k], eager[k]), (rep, k)
            ch.encode(s, fused=not fused)  # eager work between replays
            s.synchronize()
    finally:
        g.destroy()
