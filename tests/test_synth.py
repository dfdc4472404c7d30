"""The synthetic workload generator: RNG pinned against splitmix64's published
first outputs and an independent restatement of xoshiro256**; block fields
within BASELINE.json's distributions."""
import numpy as np

import edgerunner_amd.synth as synth
from oracle import restate_np as rn

MASK = (1 << 64) - 1


def splitmix(seed, n):
    out, s = [], seed
    for _ in range(n):
        s = (s + 0x9E3779B97F4A7C15) & MASK
        z = s
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & MASK
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & MASK
        out.append(z ^ (z >> 31))
    return out


def xoshiro(state, n):
    s = list(state)
    rotl = lambda x, k: ((x << k) | (x >> (64 - k))) & MASK  # noqa: E731
    out = []
    for _ in range(n):
        out.append((rotl((s[1] * 5) & MASK, 7) * 9) & MASK)
        t = (s[1] << 17) & MASK
        s[2] ^= s[0]
        s[3] ^= s[1]
        s[1] ^= s[2]
        s[0] ^= s[3]
        s[2] ^= t
        s[3] = rotl(s[3], 45)
    return out


def test_splitmix64_published_values():
    # splitmix64 from state 0: first outputs published with the algorithm
    assert splitmix(0, 3) == [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F]
    # xoshiro256** first output from state {1,2,3,4}: rotl(2*5, 7)*9 = 11520
    assert xoshiro([1, 2, 3, 4], 1) == [11520]


def test_generator_matches_restatement():
    for seed in (0, 1, synth.seed(2, 0)):
        got = [int(v) for v in synth.rng_outputs(seed, 16)]
        assert got == xoshiro(splitmix(seed, 4), 16)


def test_distributions():
    q8 = synth.q8_0(synth.seed(1, 0), 64, 1024).reshape(-1, 34)
    q = q8[:, 2:].view(np.int8)
    assert q.min() == -127 and q.max() == 127
    d = q8[:, :2].copy().view(np.float16).astype(np.float32)
    assert np.all(d >= 0) and 0.01 < float(np.mean(d)) / 0.02 < 1.0
    q4 = synth.q4_k(synth.seed(2, 0), 64, 1024).reshape(-1, 144)
    sc, mn = rn.q4k_scale_min(q4)
    assert sc.min() == 0 and sc.max() == 63 and mn.min() == 0 and mn.max() == 63
    q6 = synth.q6_k(synth.seed(3, 0), 64, 1024).reshape(-1, 210)
    s6 = q6[:, 192:208].view(np.int8)
    assert s6.min() == -32 and s6.max() == 31
    v6 = rn.q6k_values(q6)
    assert v6.min() == 0 and v6.max() == 63
    x = synth.normal_f32(5, 100000)
    assert abs(float(x.mean())) < 0.02 and abs(float(x.std()) - 1) < 0.02


def test_deterministic():
    a = synth.q4_k(synth.seed(2, 0), 8, 512)
    b = synth.q4_k(synth.seed(2, 0), 8, 512)
    c = synth.q4_k(synth.seed(2, 1), 8, 512)
    assert np.array_equal(a, b) and not np.array_equal(a, c)
