"""The DAC codec on the MI355X through the C ABI against the oracle, bit for
bit: one analysis and one synthesis window (DacAnalysis/DacSynthesis::apply),
the chunked pipelines with their context frames (analyze_audio and
synthesize_audio, chunks shrunk to 10 frames by the element limit so that
short inputs cross chunk boundaries), stereo and mono with two channel groups,
and whole recordings through AudioAnalyzer encode/decode in normal and fast
framing: the GPU stream equals the oracle's, and the decoded PCM equals the
oracle decoder's (so its PCM16 does too)."""
import numpy as np
import pytest

from tsac_hip.synthetic import Geometry, random_dac, random_model, random_tokens, synthetic_audio

pytestmark = pytest.mark.gpu

#: Limits whose element budget makes audio_chunk_frames 10 (96 * 512 * (10 + 22)).
SMALL_CHUNKS = 96 * 512 * 32


@pytest.fixture(scope="module")
def native():
    import torch

    assert torch.cuda.is_available(), "GPU tests need a visible MI355X"
    from tsac_hip import native

    native.library()
    return native


def _setup(native, oracle, channels, books, seed):
    model = random_dac(channels=channels, books=books, seed=seed)
    geometry = Geometry(channels=channels, books=books) if channels == 1 else Geometry()
    transformer = random_model(geometry, seed=seed)
    hip_model = native.HipModel(transformer)
    hip_model.source = transformer
    session = hip_model.session()
    dac = native.HipDac(model)
    small = native.HipDac(model, native.Limits(0, 0, 0, 0, SMALL_CHUNKS))
    return model, hip_model, session, dac, small, oracle.dac_model(model)


@pytest.fixture(scope="module")
def stereo(native, oracle):
    parts = _setup(native, oracle, 2, 12, 1)
    yield parts
    _, hip_model, session, dac, small, _ = parts
    for p in (small, dac, session, hip_model):
        p.close()


@pytest.fixture(scope="module")
def mono(native, oracle):
    parts = _setup(native, oracle, 1, 9, 2)
    yield parts
    _, hip_model, session, dac, small, _ = parts
    for p in (small, dac, session, hip_model):
        p.close()


def _pcm(seconds, channels, seed, frames):
    audio = synthetic_audio(seconds, channels, seed).astype(np.float32) / np.float32(32768)
    padded = np.zeros((frames * 512, channels), np.float32)
    padded[:len(audio)] = audio[:frames * 512]
    return padded


def _bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def test_analysis_window_matches_oracle(stereo):
    model, _, session, dac, _, dm = stereo
    pcm = _pcm(0.1, 2, 3, 7)
    got = dac.apply(session, False, pcm, 7 * 512)
    assert np.array_equal(_bits(got), _bits(dm.apply(False, pcm, 7 * 512)))


def test_synthesis_window_matches_oracle(stereo):
    model, _, session, dac, _, dm = stereo
    frames = 5
    latent = dm.rvq_decode(random_tokens(frames, 1, 12, seed=4), frames)
    got = dac.apply(session, True, latent, frames)
    assert np.array_equal(_bits(got), _bits(dm.apply(True, latent, frames)))
    assert 0.05 < np.abs(got).max() < 4.0, "random-init synthesis should stay near full scale"


@pytest.mark.parametrize("frames", [1, 10, 25])
def test_chunked_analysis_matches_oracle(stereo, frames):
    model, _, session, _, small, dm = stereo
    pcm = _pcm(frames * 512 / 44100 + 0.01, 2, frames, frames)
    tokens = small.analyze(session, pcm, frames)
    assert np.array_equal(tokens, dm.analyze_audio(pcm, frames, 1, chunk=10))


@pytest.mark.parametrize("frames", [1, 10, 25])
def test_chunked_synthesis_matches_oracle(stereo, frames):
    model, _, session, _, small, dm = stereo
    tokens = random_tokens(frames, 1, 12, seed=frames)
    got = small.synthesize(session, tokens, frames)
    assert np.array_equal(_bits(got), _bits(dm.synthesize_audio(tokens, frames, 1, chunk=10)))


def test_mono_two_groups_match_oracle(mono):
    """Separate channels: a mono model run once per channel group."""
    model, _, session, _, small, dm = mono
    frames, groups = 13, 2
    pcm = _pcm(0.2, 2, 5, frames)  # interleaved [T][groups * 1]
    tokens = small.analyze(session, pcm, frames, groups)
    grouped = np.ascontiguousarray(pcm.reshape(frames * 512, groups, 1).transpose(1, 0, 2))
    assert np.array_equal(tokens, dm.analyze_audio(grouped, frames, groups, chunk=10))
    audio = small.synthesize(session, tokens, frames, groups)
    assert np.array_equal(_bits(audio), _bits(dm.synthesize_audio(tokens, frames, groups, chunk=10)))


@pytest.mark.timeout(600)
def test_audio_round_trip_matches_oracle(native, oracle, stereo):
    """AudioAnalyzer::encode then ::decode of 2 s of joint stereo, 12 codebooks:
    the normal stream equals the oracle's (its DAC analysis, RVQ and pack_normal),
    the decoded PCM equals the oracle's synthesis bit for bit, so every PCM16
    sample does; fast framing decodes to the same PCM."""
    from oracle import header

    model, hip_model, session, dac, _, dm = stereo
    audio = synthetic_audio(2.0, 2, 7).astype(np.float32) / np.float32(32768)
    frames = -(-len(audio) // 512)
    padded = np.zeros((frames * 512, 2), np.float32)
    padded[:len(audio)] = audio
    stream = dac.encode(session, audio, 2, method=1)
    tokens = dm.analyze_audio(padded, frames, 1)
    expected = oracle.model(hip_model.source).pack_normal(header(frames, 1, 1, 12), tokens)
    assert stream == expected
    pcm, channels = dac.decode(session, stream)
    assert channels == 2 and pcm.shape == (frames * 512, 2)
    reference_pcm = dm.synthesize_audio(tokens, frames, 1).reshape(frames * 512, 2)
    assert np.array_equal(_bits(pcm), _bits(reference_pcm))
    pcm16 = np.array([oracle.pcm16(float(x)) for x in pcm.ravel()[:4096]])
    assert np.array_equal(pcm16, [oracle.pcm16(float(x)) for x in reference_pcm.ravel()[:4096]])
    fast = dac.encode(session, audio, 2, method=0)
    assert len(fast) == 8 + (frames * 12 * 10 + 7) // 8
    fast_pcm, _ = dac.decode(session, fast)
    assert np.array_equal(_bits(fast_pcm), _bits(pcm))
