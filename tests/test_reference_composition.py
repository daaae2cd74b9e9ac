"""The oracle's composition pinned against the reference's own classes.

oracle/Makefile builds the reference's packer from its sources, packs the seeded
original-format files of oracle/seeded_models.py, and compiles the reference's
CpuTransformer<scalar::Kernels>, TransformerPredictor, pack_normal /
unpack_normal, DacAnalysis, DacSynthesis, RvqEncoder and RvqDecoder against the
adapter_offsets.hpp the packer generated (oracle/_ref/libtsacmodel.so). Here:

* the packed TransformerModel and DAC adapters hold what the seeded files hold,
  and the feedback embeddings the packer derives equal the oracle's derivation
  and the HIP library's preparation (tsac_hip_prepare_transformer / _prepare_dac);
* the oracle's streams and distributions equal the reference's for the
  known-token shapes of tests/metal_optimized.cpp:253-259 at the reference
  geometry, stereo and two-group mono, and the committed reference fixtures
  (tests/golden/reference_streams) are what the reference produces now;
* the oracle's DAC graphs and chunked pipeline equal DacAnalysis::apply /
  apply_chunked, DacSynthesis::apply / apply_chunked, RvqEncoder and RvqDecoder.

Shapes whose reference run takes minutes (1026-frame rollover, 3074 frames,
2584 frames at 12 books) are checked through their fixtures by the GPU tests.
Everything here skips where the reference tree was not compiled.
"""
import dataclasses
import json
import pathlib

import numpy as np
import pytest

import seeded_models
from tsac_hip import native
from tsac_hip.synthetic import pattern_tokens

GOLDEN = pathlib.Path(__file__).resolve().parent / "golden"
STREAMS = GOLDEN / "reference_streams"


@pytest.fixture(scope="module")
def composition():
    from oracle import ReferenceComposition

    if not ReferenceComposition.available():
        pytest.skip("reference composition not compiled here (oracle/_ref absent)")
    return ReferenceComposition()


def feedback_embeddings(oracle, dac):
    """bf16(project_codebook(symbol)) through each book's folded out_proj: what the
    packer stores as embeddings.<book> (src/weights/pack_main.cpp:368-385)."""
    from tsac_hip.synthetic import bf16_bits

    out = np.zeros((len(dac.codebook), 1024, 1024), np.uint16)
    for book in range(len(dac.codebook)):
        w = oracle.fold_dac_weight_norm(dac.out_v[book], dac.out_g[book], 8)
        for symbol in range(1024):
            out[book, symbol] = bf16_bits(oracle.project_codebook(symbol, dac.codebook[book], w, dac.out_bias[book]))
    return out


_MODELS = {}


def oracle_model(oracle, channels):
    """The seeded probability model as the reference's packer prepares it."""
    if channels not in _MODELS:
        model = seeded_models.transformer(channels)
        _MODELS[channels] = dataclasses.replace(
            model, embeddings=feedback_embeddings(oracle, seeded_models.dac(channels)))
    return _MODELS[channels]


@pytest.mark.parametrize("channels", [2, 1])
def test_packed_transformer_holds_the_seeded_model(oracle, composition, channels):
    """Every projection, norm and constant the reference's TransformerModel reads
    from the packed files equals the seeded model; the packer's feedback embeddings
    equal the oracle's derivation and the HIP library's preparation of the same
    original-format files."""
    books = seeded_models.BOOKS[channels]
    model = oracle_model(oracle, channels)
    with composition.transformer(channels, books) as reference, \
            native.SourceFile(seeded_models.transformer_file(channels)) as t, \
            native.SourceFile(seeded_models.dac_file(channels)) as d:
        prepared = native.prepare_transformer(t, d)
        for i in range(63):
            for a, b, c in zip(reference.projection(i), model.projections[i], prepared.projections[i]):
                assert np.array_equal(a, b) and np.array_equal(a, c), i
        for i in range(32):
            gain, bias = reference.norm(i)
            assert np.array_equal(gain, model.norm_gain[i]) and np.array_equal(bias, model.norm_bias[i]), i
            assert np.array_equal(gain, prepared.norm_gain[i]) and np.array_equal(bias, prepared.norm_bias[i]), i
        positions, rotations, embeddings = reference.constants()
    assert np.array_equal(positions, model.positions) and np.array_equal(positions, prepared.positions)
    assert np.array_equal(rotations, model.rotations) and np.array_equal(rotations, prepared.rotations)
    assert np.array_equal(embeddings, model.embeddings)
    assert np.array_equal(embeddings, prepared.embeddings)


@pytest.mark.parametrize("channels", [2, 1])
def test_packed_codec_holds_the_seeded_codec(composition, channels):
    """The reference's DAC adapters read the seeded convolutions, gains, biases and
    alphas back as stored, and the RVQ adapters the packer's search vectors and
    folded projections; the HIP library's preparation of the same file equals them."""
    books = seeded_models.BOOKS[channels]
    dac = seeded_models.dac(channels)
    with composition.dac(channels, books) as reference, \
            native.SourceFile(seeded_models.dac_file(channels)) as d:
        prepared = native.prepare_dac(d)
        for synthesis, graph in ((False, "analysis"), (True, "synthesis")):
            convs = dac.synthesis if synthesis else dac.analysis
            alphas = dac.synthesis_alpha if synthesis else dac.analysis_alpha
            for i, conv in enumerate(convs):
                payload, plane, gains, biases = reference.convolution(synthesis, i)
                dims, values, gain, bias = prepared[graph][i]
                if conv.bf8:
                    assert np.array_equal(payload[:conv.values.size].view(np.int8), values[0]), (graph, i)
                    scales = payload[plane:plane + 2 * values[1].size].view(np.uint16)
                    assert np.array_equal(scales, values[1].ravel()), (graph, i)
                else:
                    assert np.array_equal(payload.view(np.float32), values), (graph, i)
                assert np.array_equal(gains, gain) and np.array_equal(biases, bias), (graph, i)
                assert np.array_equal(gains, conv.gain) and np.array_equal(biases, conv.bias), (graph, i)
            for i, alpha in enumerate(alphas):
                a = reference.activation(synthesis, i)
                assert np.array_equal(a, alpha) and np.array_equal(a, prepared[graph + "_alpha"][i]), (graph, i)
        for book in range(books):
            codebook, search, in_w, in_b, out_w, out_b = reference.rvq_tensors(book)
            p_codebook, p_search, p_in_w, p_in_b, p_out_w, p_out_b = prepared["rvq"][book]
            assert np.array_equal(codebook.ravel(), p_codebook.ravel()), book
            assert np.array_equal(search.ravel(), p_search.ravel()), book
            assert np.array_equal(in_b, p_in_b) and np.array_equal(out_b, p_out_b), book
            assert np.array_equal(out_w.ravel(), p_out_w.ravel()), book
            assert np.array_equal(np.sort(in_w.ravel()), np.sort(p_in_w.ravel())), book
            assert (np.array_equal(in_w.ravel(), p_in_w.ravel())
                    or np.array_equal(in_w.T.ravel(), p_in_w.ravel())), book


KNOWN = [(2, (17, 8, 16, 12)), (2, (35, 3, 2, 12)), (2, (17, 1, 1, 12)), (2, (3, 8, 2, 12)), (1, (35, 3, 2, 9)),
         (1, (7, 2, 2, 9)), (2, (5, 3, 1, 7))]


@pytest.mark.parametrize("channels,shape", KNOWN)
def test_oracle_stream_equals_reference_composition(oracle, composition, channels, shape):
    """The oracle's pack_normal == the reference's CpuTransformer driven by its own
    TransformerPredictor and pack_normal, byte for byte, at the reference geometry;
    the reference's unpack_normal recovers the tokens."""
    from oracle import header

    h = header(*shape, model_channels=channels)
    tokens = pattern_tokens(shape[0] * shape[2] * shape[3])
    stream = oracle.model(oracle_model(oracle, channels)).pack_normal(h, tokens, threads=8)
    with composition.transformer(channels, seeded_models.BOOKS[channels]) as reference:
        assert stream == reference.pack_normal(h, tokens, threads=8)
        if shape[0] <= 17:
            assert np.array_equal(reference.unpack_normal(stream, tokens.size, threads=8), tokens)


@pytest.mark.parametrize("shape", [(17, 3, 1, 12), (35, 3, 2, 12), (3, 8, 2, 12)])
def test_observer_bits_and_order_equal_reference(oracle, composition, shape):
    """What an EntropyObserver sees during pack_normal: every symbol's position in
    the order the reference's pack_normal visits them and the bits after_symbol
    reports (RangeEncoder::bit_position deltas, src/format/entropy.cpp:86-100)."""
    from oracle import header

    h = header(*shape)
    tokens = pattern_tokens(shape[0] * shape[2] * shape[3])
    stream, bits, positions = oracle.model(oracle_model(oracle, 2)).pack_normal_observed(h, tokens, threads=8)
    with composition.transformer(2, 12) as reference:
        ref_stream, ref_bits, ref_positions = reference.pack_normal_observed(h, tokens)
    assert stream == ref_stream
    assert np.array_equal(positions, ref_positions)
    assert np.array_equal(bits, ref_bits)
    assert sorted(positions[:, 5].tolist()) == list(range(tokens.size))
    payload_bits = (len(stream) - 18) * 8
    assert payload_bits - 32 <= int(bits.sum()) <= payload_bits


@pytest.mark.parametrize("channels,shape", [(2, (4, 3, 1, 12)), (1, (3, 2, 2, 9)), (2, (70, 2, 1, 1))])
def test_oracle_distributions_equal_reference_composition(oracle, composition, channels, shape):
    """Every symbol's BF16 distribution, oracle == reference."""
    from oracle import header

    h = header(*shape, model_channels=channels)
    tokens = pattern_tokens(shape[0] * shape[2] * shape[3])
    a = oracle.model(oracle_model(oracle, channels)).distributions(h, tokens, threads=8)
    with composition.transformer(channels, seeded_models.BOOKS[channels]) as reference:
        assert np.array_equal(a, reference.distributions(h, tokens, threads=8))


def _fixtures():
    return sorted(p.stem for p in STREAMS.glob("*.json"))


def _fixture(name):
    case = json.loads((STREAMS / f"{name}.json").read_text())
    return case, (STREAMS / f"{name}.bin").read_bytes()


FAST_FIXTURES = ["known_35_3_2", "known_3_8_2", "known_17_1_1", "mono_35_3_2", "bounded_90_3_1", "decode_197_3_1"]


def test_fixture_set_is_complete():
    import hashlib

    names = _fixtures()
    for name in ("known_17_8_16", "known_101_3_1", "known_51_3_1", "known_35_3_2", "known_17_1_1", "known_3_8_2",
                 "rollover_1026_1_1", "bounded_90_3_1", "decode_197_3_1", "decode_197_3_2", "decode_3074_3_1",
                 "mono_35_3_2", "stereo_2584_3_1"):
        assert name in names
        case, stream = _fixture(name)
        assert len(stream) == case["bytes"] and hashlib.sha256(stream).hexdigest() == case["sha256"]
        assert stream[:4] == b"FBAZ"


@pytest.mark.parametrize("name", FAST_FIXTURES)
def test_fixtures_are_the_reference_composition(oracle, composition, name):
    """The committed reference streams are what the reference composition produces
    for the seeded model now (the bounded-lookahead case with the reference's
    cache limit of 2,300,000 bytes), and the oracle produces the same bytes."""
    from oracle import header

    case, stream = _fixture(name)
    shape = (case["frames"], case["batch"], case["groups"], case["codebooks"])
    h = header(*shape, model_channels=case["channels"])
    tokens = pattern_tokens(shape[0] * shape[2] * shape[3])
    books = seeded_models.BOOKS[case["channels"]]
    with composition.transformer(case["channels"], books, case["cache_bytes"]) as reference:
        assert reference.pack_normal(h, tokens, threads=8) == stream
    assert oracle.model(oracle_model(oracle, case["channels"])).pack_normal(h, tokens, threads=8) == stream


# ---------------------------------------------------------------- the codec


def _bits(x):
    return np.ascontiguousarray(x, np.float32).view(np.uint32)


@pytest.mark.parametrize("channels", [2, 1])
def test_dac_graphs_equal_reference(oracle, composition, channels):
    """DacAnalysis::apply and DacSynthesis::apply on one window, bit for bit."""
    rng = np.random.default_rng(channels)
    dac_model = seeded_models.dac(channels)
    od = oracle.dac_model(dac_model)
    with composition.dac(channels, seeded_models.BOOKS[channels]) as reference:
        frames = 5
        pcm = (0.3 * rng.standard_normal(frames * 512 * channels)).astype(np.float32)
        assert np.array_equal(_bits(od.apply(False, pcm, frames * 512)), _bits(reference.analysis(pcm, frames * 512)))
        latent = (0.5 * rng.standard_normal(3 * 1024)).astype(np.float32)
        assert np.array_equal(_bits(od.apply(True, latent, 3)), _bits(reference.synthesis(latent, 3)))


def test_chunked_analysis_and_quantizer_equal_reference(oracle, composition):
    """The oracle's chunked analysis + RVQ (10-frame chunks, 8 + 9 context frames)
    == the reference's DacAnalysis::apply_chunked then RvqEncoder::encode; the
    oracle's RVQ decode == RvqDecoder::decode."""
    from tsac_hip.synthetic import synthetic_audio

    frames, books = 13, 12
    od = oracle.dac_model(seeded_models.dac(2))
    audio = synthetic_audio(frames * 512 / 44100, channels=2, seed=9).astype(np.float32) / np.float32(32768)
    pcm = np.zeros((frames * 512, 2), np.float32)
    pcm[:audio.shape[0]] = audio
    with composition.dac(2, books) as reference:
        latent = reference.analysis(pcm, frames * 512, chunk=10)
        tokens = reference.rvq_encode(latent, frames)
        assert np.array_equal(od.analyze_audio(pcm, frames, chunk=10), tokens)
        assert np.array_equal(_bits(od.rvq_decode(tokens, frames)), _bits(reference.rvq_decode(tokens, frames)))


def test_chunked_synthesis_equals_reference(oracle, composition):
    """The oracle's chunked synthesis (12-frame chunks, 11 context frames each
    side, the second chunk's left context clipped at frame 1) == the reference's
    RvqDecoder::decode then DacSynthesis::apply_chunked, bit for bit."""
    frames, books = 13, 12
    od = oracle.dac_model(seeded_models.dac(2))
    tokens = np.random.default_rng(3).integers(0, 1024, frames * books).astype(np.uint16)
    with composition.dac(2, books) as reference:
        latent = reference.rvq_decode(tokens, frames)
        want = reference.synthesis(latent, frames, chunk=12)
    assert np.array_equal(_bits(od.synthesize_audio(tokens, frames, chunk=12)), _bits(want))


def test_two_group_mono_pipeline_equals_reference(oracle, composition):
    """Two independent mono groups (stereo coded with separate channels): tokens
    [frame][group][book] and PCM interleaved by group, oracle == reference."""
    frames, books, groups = 3, 9, 2
    od = oracle.dac_model(seeded_models.dac(1))
    rng = np.random.default_rng(5)
    pcm = (0.2 * rng.standard_normal((groups, frames * 512, 1))).astype(np.float32)
    with composition.dac(1, books) as reference:
        tokens = reference.rvq_encode(reference.analysis(pcm, frames * 512, groups=groups, chunk=400), frames, groups)
        got = od.analyze_audio(np.ascontiguousarray(pcm), frames, groups=groups, chunk=400)
        assert np.array_equal(got, tokens)
        want = reference.synthesis(reference.rvq_decode(tokens, frames, groups), frames, groups, chunk=400)
    # reference [group][sample][channel] -> oracle [sample][group * channels]
    want = want.reshape(groups, frames * 512).T.ravel()
    assert np.array_equal(_bits(od.synthesize_audio(tokens, frames, groups=groups, chunk=400)), _bits(want))
