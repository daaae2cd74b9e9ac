"""The DAC/RVQ oracle pinned on the CPU: Snake, convolutions (every stride,
dilation and transposition the DAC uses), DAC weight-norm folding and the RVQ
search and projection against the reference's own compiled scalar sources;
BF8 expansion and PCM16 conversion against their closed forms; the graphs'
shapes and finiteness on random-init weights."""
import numpy as np
import pytest

from tsac_hip.synthetic import bf16_bits, bf16_float, dac_shape, random_dac


def _conv_config(oracle, kind):
    from oracle import OrcConv

    c = OrcConv()
    c.input, c.output, c.kernel, c.stride, c.dilation, c.transposed = kind
    c.padding = (c.kernel - 1) * c.dilation // 2 if c.stride == 1 else (c.stride + 1) // 2
    return c


# in, out, kernel, stride, dilation, transposed (channel counts reduced; the
# DAC's kernels, strides and dilations).
CONV_KINDS = [(5, 7, 7, 1, 1, 0), (6, 4, 7, 1, 3, 0), (3, 5, 7, 1, 9, 0), (8, 6, 1, 1, 1, 0),
              (4, 9, 3, 1, 1, 0), (6, 12, 4, 2, 1, 0), (5, 10, 8, 4, 1, 0), (3, 6, 16, 8, 1, 0),
              (12, 6, 16, 8, 1, 1), (8, 4, 8, 4, 1, 1), (6, 3, 4, 2, 1, 1), (2, 64, 7, 1, 1, 0)]


@pytest.mark.parametrize("kind", CONV_KINDS)
def test_conv1d_matches_reference(oracle, reference, kind):
    rng = np.random.default_rng(sum(kind))
    c = _conv_config(oracle, kind)
    w = rng.standard_normal(c.input * c.kernel * c.output).astype(np.float32)
    bias = rng.standard_normal(c.output).astype(np.float32)
    for frames, groups in ((8, 1), (37, 1), (64, 2)):
        x = rng.standard_normal(frames * groups * c.input).astype(np.float32)
        a = oracle.conv1d(c, w, bias, x, frames, groups, threads=3)
        b = reference.conv1d(c, w, bias, x, frames, groups)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), (kind, frames, groups)


def test_snake_matches_reference(oracle, reference):
    rng = np.random.default_rng(4)
    channels = 96
    x = np.concatenate([rng.standard_normal(96 * 50) * 3, rng.uniform(-1e4, 1e4, 96 * 20),
                        np.array([0.0, -0.0, 1e-40, -1e-40, 3e4, -3e4] * 16)]).astype(np.float32)
    x[:channels] = np.float32(np.pi / 2) * np.arange(channels, dtype=np.float32)  # quadrant boundaries
    alpha = rng.uniform(0.05, 3.0, channels).astype(np.float32)
    assert np.array_equal(oracle.snake(x, channels, alpha).view(np.uint32),
                          reference.snake(x, channels, alpha).view(np.uint32))


def test_sine_squared_close_to_sine(oracle):
    """The restated polynomial is sin(x)^2 to within a few ulp on [-100, 100]."""
    phases = np.linspace(-100, 100, 20001).astype(np.float32)
    got = np.array([oracle.dac_sine_squared(float(p)) for p in phases], np.float64)
    assert np.max(np.abs(got - np.sin(phases.astype(np.float64)) ** 2)) < 2e-6


@pytest.mark.parametrize("fan_in,columns", [(7, 5), (448, 3), (1024, 8), (8, 64), (5376, 2), (96, 7), (33, 4)])
def test_fold_dac_weight_norm_matches_reference(oracle, reference, fan_in, columns):
    rng = np.random.default_rng(fan_in)
    v = rng.standard_normal(fan_in * columns).astype(np.float32)
    g = rng.uniform(0.1, 2.0, columns).astype(np.float32)
    assert np.array_equal(oracle.fold_dac_weight_norm(v, g, fan_in).view(np.uint32),
                          reference.fold_dac_weight_norm(v, g, fan_in).view(np.uint32))


def test_rvq_search_and_projection_match_reference(oracle, reference):
    rng = np.random.default_rng(8)
    codebook = rng.standard_normal((1024, 8)).astype(np.float32)
    vectors = np.stack([reference.normalize_search(row) for row in codebook])
    assert np.array_equal(vectors, np.stack([oracle.normalize_search(row) for row in codebook]))
    vectors[700] = vectors[12]  # a tie: the lower index wins
    weights = rng.standard_normal(8192).astype(np.float32)
    bias = rng.standard_normal(1024).astype(np.float32)
    for trial in range(200):
        query = rng.standard_normal(8).astype(np.float32) * (10.0 ** rng.uniform(-3, 3))
        if trial == 0:
            query = codebook[700].copy()
        expected = reference.nearest_rvq(query, vectors)
        assert oracle.nearest_rvq(query, vectors) == expected
        if trial < 20:
            assert np.array_equal(oracle.project_codebook(expected, codebook, weights, bias),
                                  reference.project_codebook(expected, codebook, weights, bias))
    assert oracle.nearest_rvq(codebook[12], vectors) == 12


def test_expand_bf8_closed_form(oracle):
    rng = np.random.default_rng(3)
    rows, cols, outer = 64, 7, 3
    values = rng.integers(-128, 128, rows * cols * outer, dtype=np.int8)
    padded = 8
    scales = bf16_bits(rng.uniform(0.001, 0.1, (outer, rows // 32, padded)).astype(np.float32))
    got = oracle.expand_bf8(values, scales, (rows, cols, outer))
    v = values.reshape(outer, cols, rows // 32, 32).astype(np.float32)
    s = bf16_float(scales)[:, :, :cols].transpose(0, 2, 1)[:, :, :, None]
    assert np.array_equal(got, (v * s).reshape(-1))


def test_pcm16_closed_form(oracle):
    xs = np.array([0.0, -0.0, 1.0, -1.0, 2.0, -2.0, 0.5 / 32768, 1.5 / 32768, 2.5 / 32768, -0.5 / 32768,
                   32767.5 / 32768, -32768.5 / 32768, 0.3], np.float32)
    want = []
    for x in xs:
        scaled = min(max(float(x) * 32768.0, -32768.0), 32767.0)
        want.append(int(np.rint(scaled)))  # numpy rint: ties to even
    assert [oracle.pcm16(float(x)) for x in xs] == want


def test_dac_conv_configs_match_the_contract_shapes(oracle):
    for synthesis in (False, True):
        for channels in (1, 2):
            for i in range(30):
                c = oracle.dac_conv_config(synthesis, channels, i)
                rows, kernel, last = dac_shape(synthesis, channels, i)
                assert c.kernel == kernel
                assert (c.output, c.input) == ((rows, last) if c.transposed else (last, rows))


def test_dac_graphs_run_end_to_end(oracle):
    """Analysis of 2 latent frames and synthesis of 1, on random-init weights:
    shapes as the contract fixes them and finite values."""
    model = random_dac(channels=2, books=12, seed=1)
    dm = oracle.dac_model(model)
    rng = np.random.default_rng(0)
    pcm = (0.3 * rng.standard_normal(1024 * 2)).astype(np.float32)
    latent = dm.apply(False, pcm, 1024)
    assert latent.shape == (2 * 1024,) and np.all(np.isfinite(latent))
    tokens = dm.rvq_encode(latent, 2)
    assert tokens.shape == (24,) and tokens.max() < 1024
    decoded = dm.rvq_decode(tokens, 2)
    assert np.all(np.isfinite(decoded))
    audio = dm.apply(True, decoded[:1024], 1)
    assert audio.shape == (512 * 2,) and np.all(np.isfinite(audio))


def test_library_prepare_rvq_matches_oracle_and_reference(oracle, reference):
    """tsac_hip_prepare_rvq (host code of the library, no device needed) gives the
    oracle's and the compiled reference's search vectors and folded projections."""
    from tsac_hip import native

    rng = np.random.default_rng(21)
    codebook = rng.standard_normal((1024, 8)).astype(np.float32)
    in_v = rng.standard_normal(8 * 1024).astype(np.float32)
    in_g = rng.uniform(0.1, 2.0, 8).astype(np.float32)
    out_v = rng.standard_normal(1024 * 8).astype(np.float32)
    out_g = rng.uniform(0.1, 2.0, 1024).astype(np.float32)
    search, input_weights, output_weights = native.prepare_rvq(codebook, in_v, in_g, out_v, out_g)
    expected_search = np.stack([reference.normalize_search(row) for row in codebook]).ravel()
    assert np.array_equal(search.view(np.uint32), expected_search.view(np.uint32))
    assert np.array_equal(search, np.stack([oracle.normalize_search(row) for row in codebook]).ravel())
    for got, v, g, fan_in in ((input_weights, in_v, in_g, 1024), (output_weights, out_v, out_g, 8)):
        assert np.array_equal(got.view(np.uint32), reference.fold_dac_weight_norm(v, g, fan_in).view(np.uint32))
        assert np.array_equal(got.view(np.uint32), oracle.fold_dac_weight_norm(v, g, fan_in).view(np.uint32))
