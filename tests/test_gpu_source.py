"""Models created straight from original-format files (tsac_hip_model_create_from_source,
tsac_hip_dac_create_from_source) on the MI355X: the probability model codes a
token stream to the oracle's pack_normal bytes of the packer-prepared model and
decodes it back; the codec analyses and synthesises bit for bit like the codec
created from the tensors the files were written from."""
import numpy as np
import pytest

from tsac_hip import synthetic as syn

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def native():
    import torch

    assert torch.cuda.is_available(), "GPU tests need a visible MI355X"
    from tsac_hip import native

    native.library()
    return native


@pytest.fixture(scope="module")
def files(native):
    model = syn.random_model(syn.REFERENCE, seed=8)
    dac = syn.random_dac(channels=2, books=12, seed=8)
    transformer = native.SourceFile(syn.source_file(syn.transformer_source(model)))
    codec = native.SourceFile(syn.source_file(syn.dac_source(dac)))
    yield dac, transformer, codec
    transformer.close()
    codec.close()


def test_model_from_source_codes_like_the_prepared_model(native, oracle, files):
    from oracle import header as oracle_header

    _, transformer, codec = files
    frames, batch, books = 7, 2, 12
    tokens = syn.random_tokens(frames, 1, books, seed=9)
    prepared = native.prepare_transformer(transformer, codec)
    expected = oracle.model(prepared).pack_normal(oracle_header(frames, batch, 1, books), tokens)
    with native.HipModel.from_source(transformer, codec) as model, model.session() as session:
        stream = session.encode(native.header(frames, batch, 1, books), tokens)
        assert stream == expected
        assert np.array_equal(session.decode(stream), tokens)


def test_dac_from_source_matches_the_written_codec(native, files):
    dac_model, transformer, codec = files
    audio = syn.synthetic_audio(1.0, 2, seed=3).astype(np.float32) / np.float32(32768)
    frames = -(-len(audio) // 512)
    padded = np.zeros((frames * 512, 2), np.float32)
    padded[:len(audio)] = audio
    with native.HipModel.from_source(transformer, codec) as model, model.session() as session, \
            native.HipDac.from_source(codec) as from_file, native.HipDac(dac_model) as direct:
        assert (from_file.channels, from_file.books) == (2, 12)
        tokens = from_file.analyze(session, padded, frames)
        assert np.array_equal(tokens, direct.analyze(session, padded, frames))
        pcm = from_file.synthesize(session, tokens, frames)
        assert np.array_equal(pcm.view(np.uint32), direct.synthesize(session, tokens, frames).view(np.uint32))
