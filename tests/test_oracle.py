"""Pins the CPU oracle: the reference's own known-answer tests, closed forms,
brute force, and the reference's scalar sources compiled here (oracle/_ref).

None of these tests need a GPU.
"""
import numpy as np
import pytest

from tsac_hip.synthetic import Geometry, bf16_bits, bf16_float, pattern_tokens, random_model

SCALE_128 = np.float32(0.0883883461356163)


# ---------------------------------------------------------------- BF16 / FTZ / exp

def test_bf16_exhaustive_kat(oracle):
    """tests/numeric.cpp:172-188: every BF16 upper half x six lower halves."""
    upper = np.arange(65536, dtype=np.uint32)
    assert np.array_equal(bf16_float(upper.astype(np.uint16)).view(np.uint32), upper << 16)
    for lower in (0, 0x7FFE, 0x7FFF, 0x8000, 0x8001, 0xFFFF):
        bits = (upper << 16) | lower
        expected = (upper + ((lower > 0x8000) | ((lower == 0x8000) & (upper & 1)))).astype(np.uint16)
        got = oracle.bf16_batch(bits.view(np.float32))
        assert np.array_equal(got, expected), hex(lower)


def test_exp_matches_reference_over_strided_float_space(oracle, reference):
    """original_exp over ~8.6M bit patterns spanning every exponent, both signs,
    NaNs and infinities (src/common/numeric/probability.hpp:14-33)."""
    bits = np.arange(0, 1 << 32, 499, dtype=np.uint64).astype(np.uint32)
    z = bits.view(np.float32)
    a, b = oracle.exp_batch(z), reference.exp_batch(z)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_exp_dense_working_range(oracle, reference):
    """Every float in the softmax/attention working range [-88, 0]."""
    lo = np.float32(-88.0).view(np.uint32)
    bits = np.arange(0x80000000, lo + 1, 3, dtype=np.uint64).astype(np.uint32)
    z = bits.view(np.float32)
    a, b = oracle.exp_batch(z), reference.exp_batch(z)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_exp_closed_form_points(oracle):
    """exp(0) = 1 exactly; exp is close to e^z over the clamp range."""
    assert oracle.exp(0.0) == 1.0
    z = np.linspace(-87, 87, 10001, dtype=np.float32)
    got = oracle.exp_batch(z).astype(np.float64)
    assert np.max(np.abs(got / np.exp(z.astype(np.float64)) - 1)) < 4e-7


def test_gelu_exhaustive_against_reference_table(oracle, reference):
    """All 65,536 BF16 inputs vs the reference's LUT (src/common/probability.cpp:65-85)."""
    x = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    assert np.array_equal(oracle.gelu_batch(x), reference.gelu_table(x))


def test_gelu_closed_form(oracle):
    """tanh-GELU: gelu(0)=0, gelu(x) ~ x for large x, ~0 for very negative x."""
    assert oracle.gelu(0) == 0
    for v in (4.0, 8.0, 100.0):
        assert bf16_float(np.array([oracle.gelu(int(bf16_bits(np.float32(v))))]))[0] == v
    assert abs(bf16_float(np.array([oracle.gelu(int(bf16_bits(np.float32(-20.0))))]))[0]) < 1e-30


# ---------------------------------------------------------------- reductions

@pytest.mark.parametrize("count", [1, 2, 5, 8, 9, 33, 63, 64, 65, 127, 128, 129, 192, 256, 511,
                                   512, 513, 1000, 1024, 2048, 3000])
def test_probability_sum_matches_reference(oracle, reference, count):
    rng = np.random.default_rng(count)
    for scale in (1.0, 1e-36, 1e30):
        v = (rng.standard_normal(count) * scale).astype(np.float32)
        a, b = oracle.probability_sum(v), reference.probability_sum(v)
        assert np.float32(a).view(np.uint32) == np.float32(b).view(np.uint32)


def test_probability_sum_closed_form(oracle):
    """For 2^k x 64 values the carry merge is a balanced pair tree; integers sum exactly."""
    v = np.arange(1024, dtype=np.float32)
    assert oracle.probability_sum(v) == 1023 * 1024 / 2
    # FTZ: subnormal inputs are flushed before adding.
    assert oracle.probability_sum(np.full(16, 1e-40, np.float32)) == 0.0


def test_conditional_q15(oracle, reference):
    rng = np.random.default_rng(5)
    for left, mass in [(0.0, 1.0), (1.0, 1.0), (0.5, 1.0), (1e-9, 1.0), (0.3, 0.0),
                       (float("nan"), 1.0)] + [tuple(rng.random(2).astype(np.float32)) for _ in range(200)]:
        assert oracle.conditional_q15(left, mass) == reference.conditional_q15(left, mass)
    assert oracle.conditional_q15(0.5, 1.0) == 16384


# ---------------------------------------------------------------- BF8L / qlinear

def test_bf8l_kat(oracle):
    """tests/scalar.cpp:44-53: nearest-even quantisation."""
    values = np.zeros(256, np.float32)
    values[:4] = [127, 0.5, 1.5, -1.5]
    q, s = oracle.bf8l(values)
    assert list(s) == [int(bf16_bits(np.float32(1)))]
    assert list(q[:4]) == [127, 0, 2, -2]


def test_bf8l_matches_reference(oracle, reference):
    rng = np.random.default_rng(11)
    for scale in (1.0, 1e-38, 3e37, 0.0):
        v = (rng.standard_normal(1024) * scale).astype(np.float32)
        v = bf16_float(bf16_bits(v))
        qa, sa = oracle.bf8l(v)
        qb, sb = reference.bf8l(v)
        assert np.array_equal(qa, qb) and np.array_equal(sa, sb)


def test_bf8l_rejects_nonfinite(oracle):
    from oracle import OracleError

    v = np.zeros(256, np.float32)
    v[7] = np.inf
    with pytest.raises(OracleError):
        oracle.bf8l(v)


def _fma32(a, b, c):
    # float32 fma via exact float64 product (24+24 bits fit in 53) and one
    # float32 rounding of an exactly-representable sum candidate.
    import fractions
    exact = fractions.Fraction(float(a)) * fractions.Fraction(float(b)) + fractions.Fraction(float(c))
    return np.float32(_round_fraction_to_f32(exact))


def _round_fraction_to_f32(fr):
    # Round an exact rational to the nearest float32 (ties to even).
    if fr == 0:
        return 0.0
    f64 = float(fr)
    lo = np.float32(f64)
    cands = [np.nextafter(lo, np.float32(-np.inf)), lo, np.nextafter(lo, np.float32(np.inf))]
    import fractions
    best = min(cands, key=lambda c: (abs(fractions.Fraction(float(c)) - fr),
                                     int(np.float32(c).view(np.uint32)) & 1))
    return float(best)


def test_qlinear_brute_force_tiny(oracle):
    rng = np.random.default_rng(3)
    for k, n, m in [(256, 4, 2), (512, 8, 3), (1024, 4, 1)]:
        w = rng.integers(-127, 128, size=(n, k), dtype=np.int8)
        ws = bf16_float(bf16_bits(rng.uniform(0.001, 0.02, (k // 256, n)).astype(np.float32))).reshape(k // 256, n)
        bias = (rng.standard_normal(n) * 0.1).astype(np.float32)
        x = bf16_bits(rng.standard_normal((m, k)).astype(np.float32) * 3)
        assert np.array_equal(oracle.qlinear(w, ws, bias, x), _brute_qlinear_fraction(oracle, w, ws, bias, x))


def _brute_qlinear_fraction(oracle, w, ws, bias, x):
    n, k = w.shape
    out = np.zeros((x.shape[0], n), np.uint16)
    for m in range(x.shape[0]):
        q, s = oracle.bf8l(bf16_float(x[m]))
        a = bf16_float(s)
        dots = (w.reshape(n, k // 256, 256).astype(np.int64) *
                q.reshape(1, k // 256, 256).astype(np.int64)).sum(-1)
        for j in range(n):
            acc = np.float32(0)
            for b in range(k // 256):
                scale = np.float32(np.float32(ws[b, j]) * np.float32(a[b]))
                acc = _fma32(np.float32(dots[j, b]), scale, acc)
            out[m, j] = bf16_bits(np.float32(np.float32(acc) + np.float32(bias[j])))
    return out


@pytest.mark.parametrize("k,n,m", [(512, 1536, 3), (2048, 512, 2), (1024, 512, 5), (512, 1024, 1)])
def test_qlinear_matches_reference(oracle, reference, k, n, m):
    rng = np.random.default_rng(k + n + m)
    w = rng.integers(-127, 128, size=(n, k), dtype=np.int8)
    ws = bf16_float(bf16_bits(rng.uniform(0.001, 0.02, (k // 256, n)).astype(np.float32))).reshape(k // 256, n)
    bias = (rng.standard_normal(n) * 0.1).astype(np.float32)
    x = bf16_bits(rng.standard_normal((m, k)).astype(np.float32))
    x[0, :256] = 0  # an all-zero block exercises the 1e-35 minimum scale
    assert np.array_equal(oracle.qlinear(w, ws, bias, x), reference.qlinear(w, ws, bias, x))


# ---------------------------------------------------------------- elementwise

EDGE_BITS = np.array([0, 0x8000, 0x0001, 0x8001, 0x3F00, 0xBF00, 0x3FC0, 0xBFC0, 0x42FE, 0xC300,
                      0x2F80, 0xAF80], np.uint16)  # tests/metal_optimized.cpp:152-153


def test_layer_norm_matches_reference(oracle, reference):
    rng = np.random.default_rng(2)
    for width in (512, 1024):
        for trial in range(20):
            x = bf16_bits((rng.standard_normal(width) * 10 ** rng.uniform(-3, 3)).astype(np.float32))
            if trial == 0:
                x = np.resize(EDGE_BITS, width)
            g = bf16_bits((1 + 0.1 * rng.standard_normal(width)).astype(np.float32))
            b = bf16_bits((0.1 * rng.standard_normal(width)).astype(np.float32))
            assert np.array_equal(oracle.layer_norm(x, g, b), reference.layer_norm(x, g, b))


def test_softmax_matches_reference(oracle, reference):
    rng = np.random.default_rng(4)
    for amplitude in (0.0, 1 / 32, 1.0, 40.0, 300.0):  # tests/metal_range.cpp:144
        for n in (1024, 37, 128):
            x = bf16_bits((rng.standard_normal(n) * amplitude).astype(np.float32))
            assert np.array_equal(oracle.softmax(x), reference.softmax(x))


def test_rotary_and_add_match_reference(oracle, reference):
    rng = np.random.default_rng(9)
    v = bf16_bits(rng.standard_normal(128).astype(np.float32) * 4)
    c = bf16_bits(rng.uniform(-1, 1, 128).astype(np.float32))
    assert np.array_equal(oracle.rotary(v, c), reference.rotary(v, c))
    pairs = rng.integers(0, 65536, size=(5000, 2))
    for a, b in pairs:
        if (a & 0x7F80) == 0x7F80 or (b & 0x7F80) == 0x7F80:
            continue
        assert oracle.add_bf16(int(a), int(b)) == reference.add_bf16(int(a), int(b))


# ---------------------------------------------------------------- attention

def _attention_inputs(heads, coordinates, frames):
    """tests/attention.cpp:56-69 integer-pattern inputs."""
    width = heads * coordinates
    i = np.arange(width)
    q = bf16_bits((((i * 37 + 19) % 257) - 128).astype(np.float32) / np.float32(128))
    i = np.arange(frames * width)
    k = bf16_bits((((i * 73 + i // 17) % 257) - 128).astype(np.float32) / np.float32(64))
    v = bf16_bits((((i * 31 + i // 7) % 127) - 63).astype(np.float32) / np.float32(32))
    return q, k, v


def test_attention_checksum_kat(oracle):
    """tests/attention.cpp:83-104: FNV-1a over every geometry == 15737425383056432415."""
    checksum, mask = 14695981039346656037, (1 << 64) - 1
    for heads in (1, 2, 4):
        for coordinates in (3, 4, 7, 16, 128):
            for frames in (1, 3, 4, 15, 16, 17, 31, 32, 33, 63, 64, 65, 127, 128, 129, 257):
                q, k, v = _attention_inputs(heads, coordinates, frames)
                for prefill in (False, True):
                    for value in oracle.attention(q, k, v, heads, coordinates, SCALE_128, prefill):
                        value = int(value)
                        checksum = ((checksum ^ (value & 255)) * 1099511628211) & mask
                        checksum = ((checksum ^ (value >> 8)) * 1099511628211) & mask
    assert checksum == 15737425383056432415


def test_attention_matches_reference_random(oracle, reference):
    rng = np.random.default_rng(6)
    for heads, hw, frames in [(4, 128, 1), (4, 128, 200), (16, 64, 300), (2, 64, 64), (1, 8, 1030)]:
        w = heads * hw
        q = bf16_bits(rng.standard_normal(w).astype(np.float32))
        k = bf16_bits(rng.standard_normal(frames * w).astype(np.float32))
        v = bf16_bits(rng.standard_normal(frames * w).astype(np.float32))
        scale = np.float32(1 / np.sqrt(hw))
        for prefill in (False, True):
            assert np.array_equal(oracle.attention(q, k, v, heads, hw, scale, prefill),
                                  reference.attention(q, k, v, heads, hw, scale, prefill))


# ---------------------------------------------------------------- range coder / container

def test_token_crc_kat(oracle, reference):
    """tests/sanitation.cpp:36,86: the fast stream f6 c5 a0 holds tokens [987, 90]
    and the matching normal stream carries CRC 0x895ce095."""
    tokens = np.array([987, 90], np.uint16)
    assert oracle.token_crc32(tokens) == 0x895CE095 == reference.token_crc32(tokens)


def test_parse_header_literal_streams(oracle):
    normal = bytes([0x46, 0x42, 0x41, 0x5A, 0, 1, 1, 1, 0, 0, 0, 2, 0, 1, 0, 0x89, 0x5C, 0xE0, 0x95])
    h, offset, payload, crc = oracle.parse_header(normal)
    assert (h.method, h.groups, h.model_channels, h.codebooks, h.frames, h.batch) == (1, 1, 1, 1, 2, 1)
    assert (offset, payload, crc) == (14, 1, 0x895CE095)
    from oracle import OracleError

    for size in range(len(normal)):
        with pytest.raises(OracleError):
            oracle.parse_header(normal[:size])
    bad = bytearray(normal)
    bad[13] = 0  # zero batch
    with pytest.raises(OracleError):
        oracle.parse_header(bytes(bad))
    fast = bytes([0x46, 0x42, 0x41, 0x5A, 0, 0, 1, 1, 0xF6, 0xC5, 0xA0])
    h, offset, payload, crc = oracle.parse_header(fast)
    assert (h.method, h.frames) == (0, 2)


def test_range_coder_matches_reference_and_round_trips(oracle, reference):
    rng = np.random.default_rng(8)
    for amplitude in (0.0, 1 / 32, 1.0, 40.0):
        logits = bf16_bits((rng.standard_normal((40, 1024)) * amplitude).astype(np.float32))
        probs = bf16_float(np.stack([oracle.softmax(row) for row in logits]))
        symbols = rng.integers(0, 1024, 40).astype(np.uint16)
        symbols[:5] = np.argmax(probs[:5], axis=1)
        a = oracle.range_encode(probs, symbols)
        assert a == reference.range_encode(probs, symbols)
        assert np.array_equal(oracle.range_decode(probs, a), symbols)


# ---------------------------------------------------------------- composition
#
# The oracle's layer sequence, predictor schedule, rollover and stream order are
# pinned against the reference's own CpuTransformer and pack_normal at the
# reference geometry in test_reference_composition.py (and, through committed
# reference streams, on the GPU). Here: the oracle's own invariants at reduced
# widths, which the GPU tests use as shapes.

SMALL = Geometry(width=256, heads=2, head_width=128, ffn=512, temporal_layers=2, codebook_layers=1,
                 latent=256)


@pytest.fixture(scope="module")
def small_model():
    return random_model(SMALL, seed=3)


@pytest.mark.parametrize("frames,batch,groups,books", [(17, 8, 16, 12), (101, 3, 1, 12), (35, 3, 2, 12),
                                                       (17, 1, 1, 12), (3, 8, 2, 12), (5, 3, 1, 7)])
def test_pack_unpack_round_trip(oracle, small_model, frames, batch, groups, books):
    """unpack_normal(pack_normal(t)) == t, with lanes prepared on several threads
    or one (the stream does not depend on the lane executor)."""
    from oracle import header

    h = header(frames, batch, groups, books)
    tokens = pattern_tokens(frames * groups * books)
    om = oracle.model(small_model)
    stream = om.pack_normal(h, tokens, threads=3)
    assert stream == om.pack_normal(h, tokens, threads=1)
    assert np.array_equal(om.unpack_normal(stream, threads=2), tokens)


def test_decode_rejects_corrupt_crc(oracle, small_model):
    from oracle import OracleError, header

    h = header(9, 3, 1, 12)
    tokens = pattern_tokens(9 * 12)
    om = oracle.model(small_model)
    stream = bytearray(om.pack_normal(h, tokens))
    stream[-1] ^= 1
    with pytest.raises(OracleError, match="CRC"):
        om.unpack_normal(bytes(stream))
