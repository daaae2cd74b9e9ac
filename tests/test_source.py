"""The original model files on the CPU: the record parser against the
reference's own compiled SourceModel and the fixture of tests/sanitation.cpp:119-203,
dequantization of every storage against its closed form, the shape and
inventory checks, and the packer's preparation (projections, norms, positions,
rotary table, codebook-projection embeddings, DAC planes and quantizer)
against the synthetic model the files were written from."""
import struct

import numpy as np
import pytest

from tsac_hip import native
from tsac_hip import synthetic as syn


def _fixture():
    """The one-tensor file of tests/sanitation.cpp:119-132: metadata "{}", a
    float32 tensor "f" of one element 1.0."""
    head = struct.pack("<II", 0x23F4AEFB, 2) + b"{}"
    record = struct.pack("<IIIII", 0x23F4AEFA, 0, 1, 1, 1) + b"f" + struct.pack("<I", 0x3F800000)
    return head + record, len(head)


def _accepts(data, limits=None):
    try:
        native.SourceFile(data, limits=limits).close()
        return True
    except native.HipError:
        return False


def test_fixture_parses(reference):
    data, _ = _fixture()
    with native.SourceFile(data) as f:
        assert f.tensors() == [("f", 0, (1,), 1)]
        assert f.metadata() == b"{}"
        assert f.dequantize("f").tolist() == [1.0]
        for call in (f.dac_config, f.transformer_books, lambda: f.dequantize("absent")):
            with pytest.raises(native.HipError):
                call()
    assert reference.source_parse(data) == 1
    assert reference.source_configs(data) == (0, 0, 0)


def test_fixture_rejections_match_reference(reference):
    """tests/sanitation.cpp:133-203: every truncation but the one at the record
    boundary (which leaves a file without tensors), bad metadata length, bad
    storage, rank 9, empty and oversized axes, a trailing byte, a duplicated
    record, and the file and metadata size limits."""
    data, record = _fixture()
    cases = [data[:size] for size in range(len(data)) if size != record]
    for offset, value in ((4, 0xFFFFFFFF), (14, 0x10000), (18, 9), (26, 0), (26, 0xFFFFFFFF)):
        bad = bytearray(data)
        bad[offset:offset + 4] = struct.pack("<I", value)
        cases.append(bytes(bad))
    cases += [data + b"\0", data + data[record:], data[:record]]
    for case in cases:
        assert not _accepts(case), case
        assert reference.source_parse(case) is None, case
    assert not _accepts(data, native.SourceLimits(file_bytes=len(data) - 1))
    assert reference.source_parse(data, file_bytes=len(data) - 1) is None
    assert not _accepts(data, native.SourceLimits(metadata_bytes=1))
    assert reference.source_parse(data, metadata_bytes=1) is None
    assert _accepts(data, native.SourceLimits(file_bytes=len(data), metadata_bytes=2))


def test_dequantize_every_storage(reference):
    """float32, BF16, BF8 (3 axes, columns not a multiple of 8) and BF8L against
    the closed form value = int8 * scale[(outer*rows/block + b)*align8(cols) + col],
    and against the reference's SourceModel::dequantize."""
    rng = np.random.default_rng(5)
    f32 = rng.standard_normal(12).astype(np.float32)
    bf16 = syn.bf16_bits(rng.standard_normal(10).astype(np.float32))
    q8 = rng.integers(-128, 128, 64 * 5 * 3, dtype=np.int8)
    s8 = syn.bf16_bits(rng.uniform(0.001, 0.1, (3, 2, 8)).astype(np.float32))
    q8l = rng.integers(-128, 128, 512 * 9, dtype=np.int8)
    s8l = syn.bf16_bits(rng.uniform(0.001, 0.1, (1, 2, 16)).astype(np.float32))
    tensors = [syn.f32_tensor("a", (3, 4), f32), syn.bf16_tensor("b", (10,), bf16),
               syn.quantized_tensor("c", (64, 5, 3), q8, s8, 32), syn.quantized_tensor("d", (512, 9), q8l, s8l, 256)]
    data = syn.source_file(tensors)
    want = {
        "a": f32,
        "b": syn.bf16_float(bf16),
        "c": (q8.reshape(3, 5, 2, 32).astype(np.float32) *
              syn.bf16_float(s8)[:, :, :5].transpose(0, 2, 1)[:, :, :, None]).ravel(),
        "d": (q8l.reshape(1, 9, 2, 256).astype(np.float32) *
              syn.bf16_float(s8l)[:, :, :9].transpose(0, 2, 1)[:, :, :, None]).ravel(),
    }
    with native.SourceFile(data) as f:
        assert [t[1] for t in f.tensors()] == [syn.F32, syn.BF16, syn.BF8, syn.BF8L]
        for name, values in want.items():
            got = f.dequantize(name)
            assert np.array_equal(got.view(np.uint32), values.astype(np.float32).view(np.uint32)), name
            assert np.array_equal(got, reference.source_dequantize(data, name, got.size)), name


@pytest.fixture(scope="module")
def stereo_files():
    model = syn.random_model(syn.REFERENCE, seed=4)
    dac = syn.random_dac(channels=2, books=12, seed=4)
    return model, dac, syn.source_file(syn.transformer_source(model)), syn.source_file(syn.dac_source(dac))


def test_configs_match_reference(reference, stereo_files):
    _, _, transformer, dac = stereo_files
    with native.SourceFile(transformer) as t, native.SourceFile(dac) as d:
        assert t.transformer_books() == 12
        assert d.dac_config() == (2, 12)
        for f in (t, d):
            assert f.metadata() == b'{"producer": "tsac_hip.synthetic"}'
    assert reference.source_configs(transformer) == (0, 0, 12)
    assert reference.source_configs(dac) == (2, 12, 0)


def test_transformer_preparation(oracle, reference, stereo_files):
    """Projections, norms, positions and rotary table come back as written; the
    feedback embeddings are bf16(project_codebook(symbol)) through the folded
    out_proj, equal to the oracle's and the reference's own preparation."""
    model, dac, transformer, dac_file = stereo_files
    with native.SourceFile(transformer) as t, native.SourceFile(dac_file) as d:
        prepared = native.prepare_transformer(t, d)
    assert prepared.geometry == syn.REFERENCE
    for i, (a, b) in enumerate(zip(model.projections, prepared.projections)):
        for x, y in zip(a, b):
            assert np.array_equal(x, y), i
    for a, b in zip(model.norm_gain + model.norm_bias, prepared.norm_gain + prepared.norm_bias):
        assert np.array_equal(a, b)
    assert np.array_equal(model.positions, prepared.positions)
    assert np.array_equal(model.rotations, prepared.rotations)
    for book in (0, 7, 11):
        w = oracle.fold_dac_weight_norm(dac.out_v[book], dac.out_g[book], 8)
        assert np.array_equal(w, reference.fold_dac_weight_norm(dac.out_v[book], dac.out_g[book], 8))
        for symbol in (0, 1, 511, 1023):
            column = oracle.project_codebook(symbol, dac.codebook[book], w, dac.out_bias[book])
            assert np.array_equal(column, reference.project_codebook(symbol, dac.codebook[book], w,
                                                                     dac.out_bias[book]))
            assert np.array_equal(prepared.embeddings[book, symbol], syn.bf16_bits(column)), (book, symbol)


def test_dac_preparation(stereo_files):
    """Convolution planes, gains, biases and alphas come back as written; the
    quantizer is prepare_rvq of the written tensors."""
    _, dac, _, dac_file = stereo_files
    with native.SourceFile(dac_file) as d:
        prepared = native.prepare_dac(d)
    assert (prepared["channels"], prepared["books"]) == (2, 12)
    for graph, convs, alphas in (("analysis", dac.analysis, dac.analysis_alpha),
                                 ("synthesis", dac.synthesis, dac.synthesis_alpha)):
        for i, (c, (dims, values, gain, bias)) in enumerate(zip(convs, prepared[graph])):
            assert dims == tuple(c.dims), (graph, i)
            if c.bf8:
                assert np.array_equal(values[0], c.values) and np.array_equal(values[1], c.scales), (graph, i)
            else:
                assert np.array_equal(values, c.values), (graph, i)
            assert np.array_equal(gain, c.gain) and np.array_equal(bias, c.bias), (graph, i)
        for a, b in zip(alphas, prepared[graph + "_alpha"]):
            assert np.array_equal(a, b)
    for book in (0, 11):
        search, input_weights, output_weights = native.prepare_rvq(dac.codebook[book], dac.in_v[book], dac.in_g[book],
                                                                   dac.out_v[book], dac.out_g[book])
        want = (dac.codebook[book].ravel(), search, input_weights, dac.in_bias[book], output_weights,
                dac.out_bias[book])
        for x, y in zip(prepared["rvq"][book], want):
            assert np.array_equal(x, y), book


def test_mono_variant(reference):
    """Mono: one output channel, 9 codebooks (src/weights/source_model.cpp:176-180)."""
    dac = syn.random_dac(channels=1, books=9, seed=6)
    data = syn.source_file(syn.dac_source(dac))
    with native.SourceFile(data) as d:
        assert d.dac_config() == (1, 9)
        prepared = native.prepare_dac(d)
    assert prepared["analysis"][0][0] == (1, 7, 64) and prepared["synthesis"][29][0] == (96, 7, 1)
    assert reference.source_configs(data)[:2] == (1, 9)


def test_inventory_checks(reference, stereo_files):
    """An extra, a missing or a reshaped tensor fails transformer_config as it
    fails the reference's; a projection stored as float32 fails the packer's
    preparation; a quantizer book with a leading zero fails dac_config; the
    two files must agree on the codebook count."""
    model, dac, _, dac_file = stereo_files
    base = syn.transformer_source(model)
    extra = base + [syn.f32_tensor("extra", (1,), np.zeros(1, np.float32))]
    missing = [t for t in base if t.name != "h3/ln_2/b"]
    reshaped = [syn.bf16_tensor(t.name, (256, 2), np.frombuffer(t.payload, np.uint16))
                if t.name == "h0/ln_1/g" else t for t in base]
    for tensors in (extra, missing, reshaped):
        data = syn.source_file(tensors)
        with native.SourceFile(data) as t:
            with pytest.raises(native.HipError):
                t.transformer_books()
        assert reference.source_configs(data)[2] == 0
    values, scales, bias = model.projections[0]
    float_weights = [syn.f32_tensor(t.name, t.dims, (values.astype(np.float32) * 0.01).ravel())
                     if t.name == "h0/attn/c_attn/w" else t for t in base]
    with native.SourceFile(syn.source_file(float_weights)) as t, native.SourceFile(dac_file) as d:
        assert t.transformer_books() == 12
        with pytest.raises(native.HipError, match="BF8L"):
            native.prepare_transformer(t, d)
    zero_book = syn.dac_source(dac) + [syn.f32_tensor("quantizer.quantizers.01.extra", (1,), np.zeros(1, np.float32))]
    data = syn.source_file(zero_book)
    with native.SourceFile(data) as d:
        with pytest.raises(native.HipError, match="inventory"):
            d.dac_config()
    assert reference.source_configs(data)[:2] == (0, 0)
    mono_dac = syn.source_file(syn.dac_source(syn.random_dac(channels=1, books=9, seed=2)))
    with native.SourceFile(syn.source_file(base)) as t, native.SourceFile(mono_dac) as d:
        with pytest.raises(native.HipError, match="codebook count"):
            native.prepare_transformer(t, d)


def test_load_from_path(tmp_path):
    data, _ = _fixture()
    path = tmp_path / "tsac_fixture.bin"
    path.write_bytes(data)
    with native.SourceFile(path=path) as f:
        assert f.tensors() == [("f", 0, (1,), 1)]
    with pytest.raises(native.HipError, match="cannot open"):
        native.SourceFile(path=tmp_path / "absent.bin")
    with pytest.raises(native.HipError, match="size limit"):
        native.SourceFile(path=path, limits=native.SourceLimits(file_bytes=len(data) - 1))
