"""Pins the CPU oracle (oracle/er_oracle.c) for dequantisation.

Checks, none of which retype the oracle's formula:
  * hand-derived values of the reference's own formula fillers
    (GEMVTests.swift:136-170), worked out in the comments below;
  * bit-exact agreement with an independent numpy statement written from the
    bit layout (oracle/restate_np.py);
  * exhaustive fp16 widening vs numpy, fp32->fp16 narrowing vs numpy;
  * single-field brute force: every value of every scale byte / quant byte;
  * zero blocks and pack->dequant round trips with the reference tests'
    tolerances (DequantQ*Tests.swift).
"""
import numpy as np
import pytest

from oracle import ref
from oracle import restate_np as rn


def bits(a):
    return np.asarray(a, dtype=np.float32).view(np.uint32)


# ---- hand-derived known answers -------------------------------------------
# makeQ4KWeights block 0: d = 0.03125, dmin = 2^-8,
#   scale bytes s[i] = 13 i -> [0,13,26,39,52,65,78,91,104,117,130,143]
#   sc = [0,13,26,39, 104&15=8, 117&15=5, 130&15=2, 143&15=15]   (s[0..3] >> 6 = 0)
#   m  = [52, 65&63=1, 78&63=14, 91&63=27, 104>>4=6, (117>>4)|16=23, (130>>4)|16=24, (143>>4)|16=24]
#   qs[i] = 7 i mod 256
# w[0]   j=0 l=0 : q=0                 -> -2^-8*52           = -0.203125
# w[32]  j=1 l=0 : qs[0]>>4 = 0         -> -2^-8*1            = -0.00390625
# w[35]  j=1 l=3 : qs[3]=21>>4 = 1      -> 0.03125*13 - 2^-8  = 0.40234375
# w[69]  j=2 l=5 : qs[37]=3 &15 = 3     -> 0.03125*26*3 - 14/256 = 2.3828125
# w[234] j=7 l=10: qs[106]=230>>4 = 14  -> 0.03125*15*14 - 24/256 = 6.46875
# w[129] j=4 l=1 : qs[65]=199 &15 = 7   -> 0.03125*8*7 - 6/256 = 1.7265625
# w[162] j=5 l=2 : qs[66]=206>>4 = 12   -> 0.03125*5*12 - 23/256 = 1.78515625
Q4K_KNOWN = {0: -0.203125, 32: -0.00390625, 35: 0.40234375, 69: 2.3828125, 234: 6.46875,
             129: 1.7265625, 162: 1.78515625}

# makeQ6KWeights block 0: ql[i] = 5i, qh[i] = 3i, sc[i] = (i%7)-3, d = 2^-6
# w[0]   h0 l0 q1: ql0=0, qh0=0 -> q=-32, sc[0]=-3          -> 2^-6*-3*-32 = 1.5
# w[1]   h0 l1 q1: ql1=5, qh1=3 -> (5|48)-32 = 21, sc[0]=-3  -> -0.984375
# w[65]  h0 l1 q3: ql1>>4=0, (qh1>>4)&3=0 -> -32, sc[4]=1   -> -0.5
# w[244] h1 l20 q4: ql[116]=68>>4=4, (qh[52]=156>>6)&3=2 -> 36-32=4, sc[15]=-2 -> -0.125
# w[199] h1 l7 q3: ql[71]=99>>4=6, (qh[39]=117>>4)&3=3 -> 54-32=22, sc[12]=2 -> 0.6875
Q6K_KNOWN = {0: 1.5, 1: -0.984375, 65: -0.5, 244: -0.125, 199: 0.6875}


def test_q4k_known_answers():
    w = ref.dequant("q4_k", ref.make_q4k_weights(1, 256))
    for i, v in Q4K_KNOWN.items():
        assert w[i] == np.float32(v), (i, w[i], v)


def test_q6k_known_answers():
    w = ref.dequant("q6_k", ref.make_q6k_weights(1, 256))
    for i, v in Q6K_KNOWN.items():
        assert w[i] == np.float32(v), (i, w[i], v)


def test_q8_0_known_answers():
    blk = np.zeros(34, np.uint8)
    blk[0:2] = [0x00, 0x3C]            # d = 1.0
    blk[2:34] = np.arange(32, dtype=np.int8).view(np.uint8) - 16
    w = ref.dequant("q8_0", blk)
    assert np.array_equal(w, (np.arange(32) - 16).astype(np.float32))
    blk[0:2] = [0x00, 0xB8]            # d = -0.5
    blk[2] = 0x80                      # q = -128
    assert ref.dequant("q8_0", blk)[0] == np.float32(64.0)


# ---- independent statement -------------------------------------------------
@pytest.mark.parametrize("fmt", ["q8_0", "q4_k", "q6_k"])
def test_c_oracle_matches_numpy_statement_random(fmt):
    rng = np.random.default_rng(1234)
    bb = rn.BLOCK[fmt][0]
    blocks = rng.integers(0, 256, size=(500, bb), dtype=np.uint8)
    # keep d/dmin finite: clear the fp16 exponent's top bit
    if fmt == "q8_0":
        blocks[:, 1] &= 0xBF
    elif fmt == "q4_k":
        blocks[:, 1] &= 0xBF
        blocks[:, 3] &= 0xBF
    else:
        blocks[:, 209] &= 0xBF
    a = ref.dequant(fmt, blocks)
    b = rn.DEQUANT[fmt](blocks)
    assert np.array_equal(bits(a), bits(b))


def test_c_oracle_matches_numpy_statement_fillers():
    for rows, cols in [(9, 512), (7, 512), (12, 768)]:
        w = ref.make_q4k_weights(rows, cols)
        assert np.array_equal(bits(ref.dequant("q4_k", w)), bits(rn.dequant_q4_k(w)))
        w = ref.make_q6k_weights(rows, cols)
        assert np.array_equal(bits(ref.dequant("q6_k", w)), bits(rn.dequant_q6_k(w)))


# ---- exhaustive scale/min unpack and quant fields ---------------------------
def test_q4k_scale_field_brute_force():
    """Every value of every one of the 12 scale bytes, alone in an otherwise
    zero field, with d = dmin = 1 and all nibbles = 1: w = sc[j] - m[j]."""
    blocks = np.zeros((12 * 256, 144), np.uint8)
    blocks[:, 0:2] = [0x00, 0x3C]
    blocks[:, 2:4] = [0x00, 0x3C]
    blocks[:, 16:] = 0x11
    for pos in range(12):
        blocks[pos * 256:(pos + 1) * 256, 4 + pos] = np.arange(256)
    w = ref.dequant("q4_k", blocks).reshape(-1, 8, 32)
    sc, mn = rn.q4k_scale_min(blocks)
    assert np.array_equal(w[:, :, 0], (sc - mn).astype(np.float32))
    # closed form for a single set byte v at position pos:
    v = np.arange(256)
    for pos in range(12):
        got = w[pos * 256:(pos + 1) * 256, :, 0]
        exp = np.zeros((256, 8))
        if pos < 4:        # s[pos]: sc[pos] = v & 63, sc[pos+4] high bits = v >> 6
            exp[:, pos] += v & 63
            exp[:, pos + 4] += (v >> 6) << 4
        elif pos < 8:      # s[pos] = mins: m[pos-4] = v & 63, m[pos] high bits = v >> 6
            exp[:, pos - 4] -= v & 63
            exp[:, pos] -= (v >> 6) << 4
        else:              # s[pos]: sc[pos-4] low nibble, m[pos-4] low nibble
            exp[:, pos - 4] += (v & 15) - (v >> 4)
        assert np.array_equal(got, exp.astype(np.float32)), pos


def test_q4k_nibble_positions_brute_force():
    """A single nonzero qs byte at every position, d = 1, sc = 1, no mins:
    exactly weights (32*(i//32)*2 + i%32) = lo and +32 = hi are set."""
    blocks = np.zeros((128, 144), np.uint8)
    blocks[:, 0:2] = [0x00, 0x3C]
    blocks[:, 4:8] = 1      # sc[0..3] = 1
    blocks[:, 12:16] = 1    # sc[4..7] = 1 (low nibble), m = 0
    for i in range(128):
        blocks[i, 16 + i] = 0x52   # lo nibble 2, hi nibble 5
    w = ref.dequant("q4_k", blocks).reshape(128, 256)
    for i in range(128):
        p, l = divmod(i, 32)
        exp = np.zeros(256, np.float32)
        exp[64 * p + l] = 2.0
        exp[64 * p + 32 + l] = 5.0
        assert np.array_equal(w[i], exp), i


def test_q6k_single_bit_positions():
    """Each ql / qh byte alone (others zero) with d = 1 and all scales 1: the
    quant at the byte's destination changes from -32 by the byte's bits."""
    n = 192
    blocks = np.zeros((n, 210), np.uint8)
    blocks[:, 192:208] = 1
    blocks[:, 208:210] = [0x00, 0x3C]
    for i in range(n):
        blocks[i, i] = 0xFF
    w = ref.dequant("q6_k", blocks).reshape(n, 256)
    for i in range(n):
        exp = np.full(256, -32.0, np.float32)
        if i < 128:                     # ql byte: h = i//64, r = i%64
            h, r = divmod(i, 64)
            l = r % 32
            base = 128 * h + l
            if r < 32:
                exp[base] += 15       # q1 low nibble
                exp[base + 64] += 15  # q3 high nibble
            else:
                exp[base + 32] += 15  # q2
                exp[base + 96] += 15  # q4
        else:                           # qh byte: h = (i-128)//32, l
            h, l = divmod(i - 128, 32)
            for k in range(4):
                exp[128 * h + 32 * k + l] += 48
        assert np.array_equal(w[i], exp), i


def test_zero_blocks():
    # DequantQ4KMTests.swift:181-196, DequantQ6KTests.swift:175-190, DequantQ8_0Tests.swift:96-111
    for fmt, n in (("q8_0", 32), ("q4_k", 256), ("q6_k", 256)):
        blk = ref.pack_block(fmt, np.zeros(n, np.float32))
        assert np.all(ref.dequant(fmt, blk) == 0.0), fmt


# ---- fp16 conversions -------------------------------------------------------
def test_f16_widening_exhaustive():
    allbits = np.arange(65536, dtype=np.uint16)
    exp = allbits.view(np.float16).astype(np.float32)
    blocks = np.zeros((65536, 34), np.uint8)
    blocks[:, 0] = allbits & 0xFF
    blocks[:, 1] = allbits >> 8
    blocks[:, 2] = 1
    got = ref.dequant("q8_0", blocks).reshape(-1, 32)[:, 0]
    finite = np.isfinite(exp)
    assert np.array_equal(bits(got[finite]), bits(exp[finite]))
    assert np.array_equal(np.isnan(got), np.isnan(exp))
    assert np.array_equal(got[np.isinf(exp)], exp[np.isinf(exp)])


def test_f32_to_f16_matches_numpy_rne():
    rng = np.random.default_rng(7)
    vals = np.concatenate([
        rng.normal(size=20000).astype(np.float32) * 10 ** rng.uniform(-9, 5, 20000),
        np.array([0.0, -0.0, 65504, 65519.99, 65520, 1e-8, 2.0 ** -25, 2.0 ** -24, 3 * 2.0 ** -26,
                  np.inf, -np.inf], dtype=np.float32)]).astype(np.float32)
    with np.errstate(over="ignore"):
        exp = vals.astype(np.float16).view(np.uint16)
    got = np.array([ref.f32_to_f16(float(v)) for v in vals], dtype=np.uint16)
    assert np.array_equal(got, exp)


# ---- reference tests' pack patterns ----------------------------------------
def _patterns():
    yield "q8_0", [np.arange(32) * 0.1 - 1.6], 1e-3, 0.06
    yield "q8_0", [((b * 31 + np.arange(32)) % 19 - 9) * 0.22 for b in range(32)], 1e-3, 0.06
    # the reference's Q4_K packer clamps mins at 0, so all-positive sub-blocks
    # saturate; its tests compare GPU vs CPU dequant of the packed bytes only
    yield "q4_k", [np.arange(256) * 0.01 - 1.28], 1e-2, None
    yield "q4_k", [((b * 17 + np.arange(256)) % 29 - 14) * 0.14 for b in range(8)], 1e-2, None
    yield "q6_k", [np.arange(256) * 0.01 - 1.28], 1e-2, 0.06
    yield "q6_k", [((b * 17 + np.arange(256)) % 29 - 14) * 0.14 for b in range(8)], 1e-2, 0.2


@pytest.mark.parametrize("case", list(_patterns()), ids=lambda c: c[0])
def test_pack_round_trip(case):
    fmt, vals, _, bound = case
    for v in vals:
        v = np.asarray(v, np.float32)
        blk = ref.pack_block(fmt, v)
        w = ref.dequant(fmt, blk)
        assert np.array_equal(bits(w), bits(rn.DEQUANT[fmt](blk)))
        if bound is not None:
            assert np.max(np.abs(w - v)) <= bound


def test_quantise_error_bounds_reference():
    # DequantQ8_0Tests.swift:113-127 (MAE < 0.02), DequantQ4KMTests.swift:198-212 (< 0.15)
    v8 = (np.arange(32) % 13) / 12.0 - 0.45
    assert np.mean(np.abs(ref.dequant("q8_0", ref.pack_block("q8_0", v8)) - v8)) < 0.02
    v4 = (np.arange(256) % 23) / 11.0 - 1.0
    assert np.mean(np.abs(ref.dequant("q4_k", ref.pack_block("q4_k", v4)) - v4)) < 0.15
