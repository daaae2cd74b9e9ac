"""Operator parity on the MI355X: every HIP kernel, called through the C ABI,
against the CPU oracle on the same seeded inputs. Bit-exact throughout."""
import numpy as np
import pytest

from tsac_hip.synthetic import bf16_bits, bf16_float, random_linear

pytestmark = pytest.mark.gpu

EDGE_BITS = np.array([0, 0x8000, 0x0001, 0x8001, 0x3F00, 0xBF00, 0x3FC0, 0xBFC0, 0x42FE, 0xC300,
                      0x2F80, 0xAF80], np.uint16)  # tests/metal_optimized.cpp:152-153


@pytest.fixture(scope="module")
def torch():
    import torch

    assert torch.cuda.is_available(), "GPU tests need a visible MI355X"
    return torch


@pytest.fixture(scope="module")
def native():
    from tsac_hip import native

    native.library()
    return native


def dev(torch, array):
    a = np.ascontiguousarray(array)
    if a.dtype == np.uint16:
        a = a.view(np.int16)
    return torch.from_numpy(a.copy()).cuda()


def host(tensor, dtype=np.uint16):
    return tensor.cpu().numpy().view(dtype)


def empty(torch, shape, dtype):
    return torch.empty(shape, dtype=dtype, device="cuda")


# ---------------------------------------------------------------- qlinear

def _activations(rng, m, k, pattern=False):
    if pattern:  # tests/metal_optimized.cpp:105-108
        i = np.arange(m * k)
        return bf16_bits(((i * 73 + i // 17) % 257 - 128).astype(np.float32) * np.float32(0.03125)).reshape(m, k)
    return bf16_bits(rng.standard_normal((m, k)).astype(np.float32))


@pytest.mark.parametrize("n", [1024, 4096])
@pytest.mark.parametrize("m", [1, 3, 64, 1024, 4096])
def test_qlinear_config_shapes_match_oracle(torch, native, oracle, n, m):
    """K=1024 qlinear, GEMV, small-M and GEMM paths, against the oracle (rows sampled for large M)."""
    rng = np.random.default_rng(n * 7 + m)
    values, scales, bias = random_linear(rng, 1024, n, bias_std=0.1, row_scales=True)
    x = _activations(rng, m, 1024)
    linear = native.DeviceLinear(values, scales, bias)
    dx = dev(torch, x)
    outputs = {}
    paths = [native.PATH_GEMM] + ([native.PATH_GEMV] if m <= 8 else []) + ([native.PATH_SMALL] if m <= 1024 else [])
    for path in paths:
        y = empty(torch, (m, n), torch.int16)
        linear.apply(dx, y, path)
        outputs[path] = host(y)
    if m > 8:  # the GEMV path in blocks of 8 columns covers every row too
        y = empty(torch, (m, n), torch.int16)
        for r in range(0, m, 8):
            linear.apply(dx[r:r + 8], y[r:r + 8], native.PATH_GEMV)
        outputs[native.PATH_GEMV] = host(y)
    assert np.array_equal(outputs[native.PATH_GEMM], outputs[native.PATH_GEMV])
    if m <= 1024:
        assert np.array_equal(outputs[native.PATH_GEMM], outputs[native.PATH_SMALL])
    rows = np.arange(m) if m <= 64 else np.unique(np.r_[0, 1, 127, 128, m - 1, rng.integers(0, m, 40)])
    expected = oracle.qlinear(values, scales, bias, x[rows])
    assert np.array_equal(outputs[native.PATH_GEMM][rows], expected)


@pytest.mark.parametrize("k,n", [(512, 1536), (512, 512), (512, 2048), (2048, 512), (1024, 512), (512, 1024),
                                 (256, 256), (4096, 1024)])
@pytest.mark.parametrize("columns", [1, 2, 3, 6, 8, 14, 33, 64, 96])
def test_qlinear_reference_projection_shapes(torch, native, oracle, k, n, columns):
    """Projection shapes of the reference model at the column counts of
    tests/metal_optimized.cpp:96-146, with the integer-pattern activations."""
    rng = np.random.default_rng(k + n + columns)
    values, scales, bias = random_linear(rng, k, n, bias_std=0.1)
    x = _activations(rng, columns, k, pattern=True)
    linear = native.DeviceLinear(values, scales, bias)
    y = empty(torch, (columns, n), torch.int16)
    linear.apply(dev(torch, x), y, native.PATH_GEMM)
    expected = oracle.qlinear(values, scales, bias, x)
    assert np.array_equal(host(y), expected)
    if columns <= 8:
        linear.apply(dev(torch, x), y, native.PATH_GEMV)
        assert np.array_equal(host(y), expected)
    if columns <= 64 and k <= 2048:
        y.zero_()
        linear.apply(dev(torch, x), y, native.PATH_SMALL)
        assert np.array_equal(host(y), expected)


def test_qlinear_edge_bits_and_zero_blocks(torch, native, oracle):
    """BF16 edge patterns with whole zero blocks (tests/metal_optimized.cpp:148-203)."""
    rng = np.random.default_rng(1)
    values, scales, bias = random_linear(rng, 1024, 512)
    for columns in (3, 1, 3, 2, 6, 3, 40):
        i = np.arange(columns * 1024)
        x = np.where((i // 256) % 3 == 0, 0, EDGE_BITS[i % EDGE_BITS.size]).astype(np.uint16).reshape(columns, 1024)
        expected = oracle.qlinear(values, scales, bias, x)
        linear = native.DeviceLinear(values, scales, bias)
        for path in (native.PATH_GEMM, native.PATH_SMALL) + ((native.PATH_GEMV,) if columns <= 8 else ()):
            y = empty(torch, (columns, 512), torch.int16)
            linear.apply(dev(torch, x), y, path)
            assert np.array_equal(host(y), expected)


def test_qlinear_rejects_nonfinite(torch, native):
    rng = np.random.default_rng(2)
    linear = native.DeviceLinear(*random_linear(rng, 512, 512))
    for bad in (0x7F80, 0x7FC1):
        x = np.zeros((3, 512), np.uint16)
        x[0, 0] = bad
        y = empty(torch, (3, 512), torch.int16)
        with pytest.raises(native.HipError, match="finite"):
            linear.apply(dev(torch, x), y)


def test_qlinear_fused_residual(torch, native, oracle):
    rng = np.random.default_rng(3)
    values, scales, bias = random_linear(rng, 2048, 512)
    # 77 and 300 rows at N = 512 take the small-M kernel automatically (few GEMM tiles).
    for m, path in ((3, native.PATH_AUTO), (77, native.PATH_AUTO), (40, native.PATH_SMALL), (64, native.PATH_AUTO),
                    (300, native.PATH_AUTO), (300, native.PATH_GEMM)):
        x = _activations(rng, m, 2048)
        skip = bf16_bits(((np.arange(m * 512) % 31) - 15).astype(np.float32) / 32).reshape(m, 512)
        q = empty(torch, (m, 2048), torch.int8)
        s = empty(torch, (m, 8), torch.float32)
        native.bf8l(dev(torch, x), m, 2048, q, s)
        linear = native.DeviceLinear(values, scales, bias)
        y = dev(torch, skip)
        linear.apply_quantized(q, s, m, y, residual=y, path=path)
        plain = oracle.qlinear(values, scales, bias, x)
        expected = np.array([[oracle.add_bf16(int(a), int(b)) for a, b in zip(r1, r2)]
                             for r1, r2 in zip(skip, plain)], np.uint16)
        assert np.array_equal(host(y), expected)


def _tile_offsets(m, k):
    """Byte offset of (row, k) in the MFMA operand-tile layout of bf8l_tiles."""
    r = np.arange(m)[:, None]
    c = np.arange(k)[None, :]
    return ((r // 32) * (k // 32) + c // 32) * 1024 + ((r % 32) + 32 * ((c // 16) % 2)) * 16 + c % 16


@pytest.mark.parametrize("m,k,n", [(9, 256, 64), (130, 512, 192), (77, 2048, 512), (300, 512, 1536),
                                   (129, 4096, 1024), (1000, 1024, 320)])
def test_gemm_tiles_and_rows_layouts_agree(torch, native, oracle, m, k, n):
    """The GEMM on operand tiles (encode path), on row-major activations, and
    the GEMV in blocks of eight columns agree bit for bit with the oracle, with
    and without a residual, at row and column counts that leave partial tiles."""
    rng = np.random.default_rng(m * 31 + k + n)
    values, scales, bias = random_linear(rng, k, n, bias_std=0.1)
    x = _activations(rng, m, k)
    linear = native.DeviceLinear(values, scales, bias)
    padded = native.tile_rows(m)
    assert padded % 128 == 0 and padded >= m
    q_rows = empty(torch, (m, k), torch.int8)
    s_rows = empty(torch, (m, k // 256), torch.float32)
    native.bf8l(dev(torch, x), m, k, q_rows, s_rows)
    q_tiles = empty(torch, (padded * k,), torch.int8)
    s_tiles = empty(torch, (k // 256, padded), torch.float32)
    native.bf8l_tiles(dev(torch, x), m, k, q_tiles, s_tiles)
    # The tile layout holds the same bytes and scales as the rows.
    assert np.array_equal(host(q_tiles, np.int8)[_tile_offsets(m, k)], host(q_rows, np.int8))
    assert np.array_equal(host(s_tiles, np.float32)[:, :m].T, host(s_rows, np.float32))
    expected = oracle.qlinear(values, scales, bias, x)
    skip = bf16_bits(rng.standard_normal((m, n)).astype(np.float32))
    with_skip = np.array([[oracle.add_bf16(int(a), int(b)) for a, b in zip(r1, r2)]
                          for r1, r2 in zip(skip, expected)], np.uint16)
    for residual, want in ((False, expected), (True, with_skip)):
        results = []
        for q, s, path in ((q_tiles, s_tiles, native.PATH_GEMM_TILES), (q_rows, s_rows, native.PATH_GEMM)):
            y = dev(torch, skip) if residual else empty(torch, (m, n), torch.int16)
            linear.apply_quantized(q, s, m, y, residual=y if residual else None, path=path)
            results.append(host(y))
        y = dev(torch, skip) if residual else empty(torch, (m, n), torch.int16)
        for r in range(0, m, 8):
            linear.apply_quantized(q_rows[r:r + 8], s_rows[r:r + 8], min(8, m - r), y[r:r + 8],
                                   residual=y[r:r + 8] if residual else None, path=native.PATH_GEMV)
        results.append(host(y))
        for got in results:
            assert np.array_equal(got, want)


@pytest.mark.parametrize("k,n,with_residual", [(512, 1536, False), (2048, 512, True)])
def test_gemm_many_tiles_per_workgroup(torch, native, k, n, with_residual):
    """At the encode's 2580 x 12 rows every persistent workgroup walks several
    tiles (LDS reuse across tiles, output staging between them); the GEMM on
    operand tiles must equal the GEMV in blocks of eight columns, on two runs."""
    rng = np.random.default_rng(k + n)
    m = 30960
    linear = native.DeviceLinear(*random_linear(rng, k, n, bias_std=0.1))
    x = dev(torch, _activations(rng, m, k))
    skip = dev(torch, bf16_bits(rng.standard_normal((m, n)).astype(np.float32)))
    padded = native.tile_rows(m)
    q_tiles = empty(torch, (padded * k,), torch.int8)
    s_tiles = empty(torch, (k // 256 * padded,), torch.float32)
    native.bf8l_tiles(x, m, k, q_tiles, s_tiles)
    q_rows = empty(torch, (m, k), torch.int8)
    s_rows = empty(torch, (m, k // 256), torch.float32)
    native.bf8l(x, m, k, q_rows, s_rows)
    want = skip.clone()
    for r in range(0, m, 8):
        native_rows = min(8, m - r)
        linear.apply_quantized(q_rows[r:r + 8], s_rows[r:r + 8], native_rows, want[r:r + 8],
                               residual=want[r:r + 8] if with_residual else None, path=native.PATH_GEMV)
    want = host(want)
    for _ in range(2):
        y = skip.clone()
        linear.apply_quantized(q_tiles, s_tiles, m, y, residual=y if with_residual else None,
                               path=native.PATH_GEMM_TILES)
        assert np.array_equal(host(y), want)


def test_gemm_output_beyond_32bit_byte_range(torch, native, oracle):
    """Outputs are addressed through 32-bit buffer ranges, so an output matrix
    past 2^31 bytes takes several launches of row chunks (K=256, N=8192: 130,944
    rows per launch); rows on both sides of the chunk boundary, in both
    activation layouts and with a residual, must match the oracle."""
    rng = np.random.default_rng(31)
    k, n = 256, 8192
    m = 131072 + 300
    assert m * n * 2 > 2 ** 31
    values, scales, bias = random_linear(rng, k, n, bias_std=0.1)
    linear = native.DeviceLinear(values, scales, bias)
    x = _activations(rng, m, k)
    dx = dev(torch, x)
    rows = np.unique(np.r_[0, 1, 130943, 130944, 130945, 131071, 131072, m - 1, rng.integers(0, m, 24)])
    expected = oracle.qlinear(values, scales, bias, x[rows])
    index = torch.from_numpy(rows).cuda()
    padded = native.tile_rows(m)
    q_tiles = empty(torch, (padded * k,), torch.int8)
    s_tiles = empty(torch, (k // 256 * padded,), torch.float32)
    native.bf8l_tiles(dx, m, k, q_tiles, s_tiles)
    q_rows = empty(torch, (m, k), torch.int8)
    s_rows = empty(torch, (m, k // 256), torch.float32)
    native.bf8l(dx, m, k, q_rows, s_rows)
    y = empty(torch, (m, n), torch.int16)
    for q, s, path in ((q_tiles, s_tiles, native.PATH_GEMM_TILES), (q_rows, s_rows, native.PATH_GEMM)):
        y.zero_()
        linear.apply_quantized(q, s, m, y, path=path)
        assert np.array_equal(host(y.index_select(0, index)), expected)
    skip = bf16_bits(rng.standard_normal((rows.size, n)).astype(np.float32))
    y.zero_()
    y.index_copy_(0, index, dev(torch, skip))
    linear.apply_quantized(q_tiles, s_tiles, m, y, residual=y, path=native.PATH_GEMM_TILES)
    with_skip = np.array([[oracle.add_bf16(int(a), int(b)) for a, b in zip(r1, r2)]
                          for r1, r2 in zip(skip, expected)], np.uint16)
    assert np.array_equal(host(y.index_select(0, index)), with_skip)
    del y, q_tiles, q_rows
    torch.cuda.empty_cache()


def test_gemm_repeatable(torch, native):
    """Two launches of the persistent GEMM give identical bytes."""
    rng = np.random.default_rng(8)
    m, k, n = 4000, 512, 1536
    linear = native.DeviceLinear(*random_linear(rng, k, n))
    x = dev(torch, _activations(rng, m, k))
    outputs = []
    for _ in range(2):
        y = empty(torch, (m, n), torch.int16)
        linear.apply(x, y, native.PATH_GEMM)
        outputs.append(host(y))
    assert np.array_equal(outputs[0], outputs[1])


def test_bf8l_matches_oracle(torch, native, oracle):
    rng = np.random.default_rng(4)
    for k in (256, 512, 1024, 2048, 4096):
        x = bf16_bits((rng.standard_normal((5, k)) * 10.0 ** rng.uniform(-30, 30, (5, 1))).astype(np.float32))
        q = empty(torch, (5, k), torch.int8)
        s = empty(torch, (5, k // 256), torch.float32)
        native.bf8l(dev(torch, x), 5, k, q, s)
        for r in range(5):
            eq, es = oracle.bf8l(bf16_float(x[r]))
            assert np.array_equal(host(q, np.int8)[r], eq)
            assert np.array_equal(host(s, np.float32)[r], bf16_float(es))


# ---------------------------------------------------------------- elementwise

def test_gelu_exhaustive(torch, native, oracle):
    x = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    out = empty(torch, 65536, torch.int16)
    native.gelu(dev(torch, x), out)
    assert np.array_equal(host(out), oracle.gelu_batch(x))


def test_layer_norm_matches_oracle(torch, native, oracle):
    rng = np.random.default_rng(5)
    for width in (256, 512, 1024, 2048):
        rows = 9
        x = bf16_bits((rng.standard_normal((rows, width)) * 10.0 ** rng.uniform(-3, 3, (rows, 1))).astype(np.float32))
        x[0] = np.resize(EDGE_BITS, width)
        g = bf16_bits((1 + 0.1 * rng.standard_normal(width)).astype(np.float32))
        b = bf16_bits((0.1 * rng.standard_normal(width)).astype(np.float32))
        out = empty(torch, (rows, width), torch.int16)
        native.layer_norm(dev(torch, x), rows, width, dev(torch, g), dev(torch, b), out)
        expected = np.stack([oracle.layer_norm(r, g, b) for r in x])
        assert np.array_equal(host(out), expected)


def _tiny_rows(rng, width):
    """Rows around the magnitudes where FTZ sums start to differ from plain sums:
    values at and just below 2^-56, squares that are subnormal, sums that cancel
    to subnormals, BF16 subnormals, signed zeros and the largest finite values."""
    rows = []
    for exponent in (-56, -57, -63, -64, -70, -100, -126, -130):
        rows.append(bf16_bits((rng.standard_normal(width) * 2.0 ** exponent).astype(np.float32)))
    mixed = bf16_bits(rng.standard_normal(width).astype(np.float32))
    mixed[::3] = bf16_bits((rng.standard_normal(mixed[::3].size) * 1e-30).astype(np.float32))
    rows.append(mixed)
    boundary = np.where(rng.random(width) < 0.5, 0x2380, 0x237F).astype(np.uint16)
    boundary |= (rng.random(width) < 0.5).astype(np.uint16) << 15
    rows.append(boundary)
    cancel = bf16_bits((rng.standard_normal(width) * 2.0 ** -120).astype(np.float32))
    cancel[1::2] = cancel[0::2] ^ 0x8000  # pairs sum to signed zeros
    cancel[-1] = 0x0003
    rows.append(cancel)
    rows.append(np.resize(np.array([0x0001, 0x8001, 0x007F, 0x807F, 0x0000, 0x8000], np.uint16), width))
    rows.append(np.resize(np.array([0x7F7F, 0xFF7F, 0x0080, 0x8080], np.uint16), width))
    return np.stack(rows)


def test_layer_norm_small_magnitudes(torch, native, oracle):
    rng = np.random.default_rng(15)
    for width in (256, 512, 2048):
        x = _tiny_rows(rng, width)
        rows = x.shape[0]
        g = bf16_bits((1 + 0.1 * rng.standard_normal(width)).astype(np.float32))
        b = bf16_bits((0.1 * rng.standard_normal(width)).astype(np.float32))
        out = empty(torch, (rows, width), torch.int16)
        native.layer_norm(dev(torch, x), rows, width, dev(torch, g), dev(torch, b), out)
        expected = np.stack([oracle.layer_norm(r, g, b) for r in x])
        assert np.array_equal(host(out), expected)


def test_bf8l_small_magnitudes(torch, native, oracle):
    rng = np.random.default_rng(16)
    for k in (256, 512, 2048):
        x = _tiny_rows(rng, k)
        rows = x.shape[0]
        q = empty(torch, (rows, k), torch.int8)
        s = empty(torch, (rows, k // 256), torch.float32)
        native.bf8l(dev(torch, x), rows, k, q, s)
        for r in range(rows):
            eq, es = oracle.bf8l(bf16_float(x[r]))
            assert np.array_equal(host(q, np.int8)[r], eq), r
            assert np.array_equal(host(s, np.float32)[r], bf16_float(es)), r


def test_softmax_matches_oracle(torch, native, oracle):
    rng = np.random.default_rng(6)
    for amplitude in (0.0, 1 / 32, 1.0, 40.0, 300.0):  # tests/metal_range.cpp:144
        x = bf16_bits((rng.standard_normal((7, 1024)) * amplitude).astype(np.float32))
        out = empty(torch, (7, 1024), torch.int16)
        native.softmax(dev(torch, x), 7, 1024, out)
        assert np.array_equal(host(out), np.stack([oracle.softmax(r) for r in x]))
    bad = np.zeros((1, 1024), np.uint16)
    bad[0, 5] = 0x7F80
    with pytest.raises(native.HipError):
        native.softmax(dev(torch, bad), 1, 1024, out)


def test_rotary_and_add_match_oracle(torch, native, oracle):
    rng = np.random.default_rng(7)
    v = bf16_bits(rng.standard_normal(4096).astype(np.float32) * 4)
    c = bf16_bits(rng.uniform(-1, 1, 4096).astype(np.float32))
    out = empty(torch, 4096, torch.int16)
    native.rotary(dev(torch, v), dev(torch, c), out)
    assert np.array_equal(host(out), oracle.rotary(v, c))
    a = bf16_bits(rng.standard_normal((6, 512)).astype(np.float32))
    b = bf16_bits(rng.standard_normal((3, 512)).astype(np.float32))
    out = empty(torch, (6, 512), torch.int16)
    native.add(dev(torch, a), dev(torch, b), 6, 512, 3, out)
    expected = np.array([[oracle.add_bf16(int(x), int(y)) for x, y in zip(a[r], b[r % 3])] for r in range(6)],
                        np.uint16)
    assert np.array_equal(host(out), expected)


# ---------------------------------------------------------------- attention

def _pattern_attention(heads, hw, frames):
    width = heads * hw
    i = np.arange(width)
    q = bf16_bits((((i * 37 + 19) % 257) - 128).astype(np.float32) / np.float32(128))
    i = np.arange(frames * width)
    k = bf16_bits((((i * 73 + i // 17) % 257) - 128).astype(np.float32) / np.float32(64))
    v = bf16_bits((((i * 31 + i // 7) % 127) - 63).astype(np.float32) / np.float32(32))
    return q, k, v


@pytest.mark.parametrize("heads,hw", [(4, 128), (16, 64), (1, 128), (2, 64)])
def test_attention_decode_matches_oracle(torch, native, oracle, heads, hw):
    """One query over T cached keys (tests/attention.cpp frame sweep + the long histories)."""
    rng = np.random.default_rng(heads * hw)
    scale = np.float32(1 / np.sqrt(hw))
    for frames in (1, 3, 4, 8, 9, 15, 16, 17, 33, 63, 64, 65, 127, 128, 129, 257, 1024, 1290):
        for pattern in (True, False):
            if pattern:
                q, k, v = _pattern_attention(heads, hw, frames)
            else:
                w = heads * hw
                q = bf16_bits(rng.standard_normal(w).astype(np.float32) * 2)
                k = bf16_bits(rng.standard_normal(frames * w).astype(np.float32) * 2)
                v = bf16_bits(rng.standard_normal(frames * w).astype(np.float32))
            for prefill in (False, True):
                out = empty(torch, heads * hw, torch.int16)
                native.attention(dev(torch, q), dev(torch, k), dev(torch, v), 0, 1, frames, heads, hw, scale,
                                 prefill, out)
                assert np.array_equal(host(out), oracle.attention(q, k, v, heads, hw, scale, prefill)), \
                    (frames, pattern, prefill)


@pytest.mark.parametrize("heads,hw", [(1, 128), (2, 64)])
def test_attention_decode_long_histories(torch, native, oracle, heads, hw):
    """Histories past 64 blocks (the merge's running-maximum scan carried from
    one chunk of 64 blocks to the next), the longest one workgroup's LDS holds
    (256 blocks), one block more (partials in scratch and a merge launch), and
    a block whose scores are all NaN (the merge's plain sequential loop)."""
    rng = np.random.default_rng(21 + hw)
    scale = np.float32(1 / np.sqrt(hw))
    w = heads * hw
    cases = [(frames, False) for frames in (4097, 8191, 16384, 16385)] + [(5000, True)]
    for frames, poisoned in cases:
        q = bf16_bits(rng.standard_normal(w).astype(np.float32) * 2)
        k = bf16_bits(rng.standard_normal(frames * w).astype(np.float32) * 2)
        v = bf16_bits(rng.standard_normal(frames * w).astype(np.float32))
        if poisoned:
            q[3] = 0  # 0 * inf = NaN in every score of block 70
            k.reshape(frames, w)[70 * 64:71 * 64, 3] = 0x7F80
        out = empty(torch, w, torch.int16)
        native.attention(dev(torch, q), dev(torch, k), dev(torch, v), 0, 1, frames, heads, hw, scale, False, out)
        assert np.array_equal(host(out), oracle.attention(q, k, v, heads, hw, scale, False)), (frames, poisoned)


def test_attention_decode_batched_sequences(torch, native, oracle):
    """Three lanes with their own caches, as the decode step runs them."""
    rng = np.random.default_rng(11)
    heads, hw, frames, lanes, extent = 4, 128, 200, 3, 256
    w = heads * hw
    q = bf16_bits(rng.standard_normal((lanes, w)).astype(np.float32))
    k = bf16_bits(rng.standard_normal((lanes, extent, w)).astype(np.float32))
    v = bf16_bits(rng.standard_normal((lanes, extent, w)).astype(np.float32))
    out = empty(torch, (lanes, w), torch.int16)
    scale = np.float32(0.0883883461356163)
    native.attention(dev(torch, q), dev(torch, k), dev(torch, v), extent * w, lanes, frames, heads, hw, scale,
                     False, out)
    for lane in range(lanes):
        expected = oracle.attention(q[lane], k[lane, :frames], v[lane, :frames], heads, hw, scale, False)
        assert np.array_equal(host(out)[lane], expected)


def test_attention_decode_split_scratch_and_capture(torch, native, oracle):
    """Histories split over several workgroups per (sequence, head), in shapes
    that grow, shrink and grow the per-stream scratch in turn (its arrival
    counters must be zero again after every launch), then one such call
    captured in a graph and replayed with eager calls on the same stream
    between the replays."""
    rng = np.random.default_rng(31)

    def case(sequences, heads, hw, frames):
        w = heads * hw
        q = bf16_bits(rng.standard_normal((sequences, w)).astype(np.float32) * 2)
        k = bf16_bits(rng.standard_normal((sequences, frames, w)).astype(np.float32) * 2)
        v = bf16_bits(rng.standard_normal((sequences, frames, w)).astype(np.float32))
        scale = np.float32(1 / np.sqrt(hw))
        expected = np.stack([oracle.attention(q[s], k[s], v[s], heads, hw, scale, False) for s in range(sequences)])
        args = (dev(torch, q), dev(torch, k), dev(torch, v), frames * w, sequences, frames, heads, hw, scale, False)
        return args, expected

    shapes = [(1, 2, 64, 1290), (3, 16, 64, 2580), (1, 2, 64, 700), (2, 4, 128, 5000), (3, 16, 64, 2580),
              (2, 1, 128, 257)]
    cases = [case(*shape) for shape in shapes]
    for shape, (args, expected) in zip(shapes, cases):
        out = empty(torch, expected.shape, torch.int16)
        native.attention(*args, out)
        assert np.array_equal(host(out), expected), shape
    (args, expected), (other, other_expected) = cases[1], cases[3]
    out = empty(torch, expected.shape, torch.int16)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        native.attention(*args, out)
    for replay in range(3):
        out.zero_()
        other_out = empty(torch, other_expected.shape, torch.int16)
        native.attention(*other, other_out)
        graph.replay()
        torch.cuda.synchronize()
        assert np.array_equal(host(out), expected), replay
        assert np.array_equal(host(other_out), other_expected), replay


@pytest.mark.parametrize("heads,hw,rotary", [(4, 128, True), (4, 128, False), (16, 64, True)])
def test_attention_causal_matches_oracle(torch, native, oracle, heads, hw, rotary):
    """Every query of several causal sequences (one with a replay prefix) against
    the oracle's single-query attention over keys 0..t."""
    rng = np.random.default_rng(heads + hw + rotary)
    w = heads * hw
    lengths = [1, 12, 70, 300, 129]
    replays = [0, 0, 0, 256, 5]
    starts = np.cumsum([0] + lengths[:-1]).astype(np.int32)
    rows = sum(lengths)
    qkv = bf16_bits(rng.standard_normal((rows, 3 * w)).astype(np.float32))
    context = max(lengths)
    rotations = bf16_bits(rng.uniform(-1, 1, (context, hw)).astype(np.float32)) if rotary else None
    scale = np.float32(1 / np.sqrt(hw))
    out = empty(torch, (rows, w), torch.int16)
    native.attention_causal(dev(torch, qkv), heads, hw, dev(torch, starts), dev(torch, np.array(lengths, np.int32)),
                            dev(torch, np.array(replays, np.int32)), len(lengths), max(lengths),
                            dev(torch, rotations) if rotary else None, scale, out)
    got = host(out)
    for s, (start, length, replay) in enumerate(zip(starts, lengths, replays)):
        seq = qkv[start:start + length]
        q, k, v = seq[:, :w].copy(), seq[:, w:2 * w].copy(), seq[:, 2 * w:].copy()
        if rotary:
            for t in range(length):
                for h in range(heads):
                    q[t, h * hw:(h + 1) * hw] = oracle.rotary(q[t, h * hw:(h + 1) * hw], rotations[t])
                    k[t, h * hw:(h + 1) * hw] = oracle.rotary(k[t, h * hw:(h + 1) * hw], rotations[t])
        for t in range(length):
            expected = oracle.attention(q[t], k[:t + 1], v[:t + 1], heads, hw, scale, t < replay)
            assert np.array_equal(got[start + t], expected), (s, t)


def test_calibration_probes(torch, native):
    """The calibration kernels run, report their operation count, and reject
    sizes they cannot stream."""
    data = torch.zeros(1 << 20, dtype=torch.uint8, device="cuda")
    native.probe_read(data)
    assert native.probe_mfma(8, 3) == 8 * 4 * 4 * 3 * 65536
    torch.cuda.synchronize()
    with pytest.raises(native.HipError, match="multiple of 64 KiB"):
        native.probe_read(data[:1000])
