"""The HIP library held byte for byte against the reference's own outputs.

tests/golden/reference_streams and reference_audio hold what the reference's
compiled CpuTransformer + TransformerPredictor + pack_normal, DacAnalysis,
RvqEncoder, RvqDecoder and DacSynthesis produce for the seeded model files of
oracle/seeded_models.py (written by the scripts beside them). Here the library
is created from the same original-format files through the C ABI
(tsac_hip_model_create_from_source, tsac_hip_dac_create_from_source) and must
reproduce them on the MI355X:

* encode: the stream of every fixture shape, including the reference tests'
  known-token shapes (tests/metal_optimized.cpp:253-259), 1026 frames in one
  lane (context rollover and 256-frame replay), the bounded-lookahead case
  under a 2,300,000-byte cache limit (:277-292), 197- and 3074-frame resident
  decode shapes (:519-523), two mono channel groups, and 2584 frames at 12
  codebooks in lanes of 862/861/861;
* decode: the reference's streams back to their tokens on the frame-step path
  (whose last steps run with one active lane where the lanes are uneven);
* audio: the 30 s joint-stereo recording at 12 codebooks and entropy batch 3,
  the 10 s recording at 3 codebooks with the automatic batch, and stereo coded
  as two mono groups: analysis tokens equal the reference's, every 400-frame
  synthesis chunk's float PCM equals the reference's bit for bit, the
  AudioAnalyzer encode writes the reference's stream and its decode returns
  the reference's PCM.
"""
import hashlib
import json
import pathlib

import numpy as np
import pytest

import seeded_models
from tsac_hip import synthetic as syn

pytestmark = pytest.mark.gpu

GOLDEN = pathlib.Path(__file__).resolve().parent / "golden"
STREAMS = GOLDEN / "reference_streams"
AUDIO = GOLDEN / "reference_audio"


@pytest.fixture(scope="module")
def native():
    import torch

    assert torch.cuda.is_available(), "GPU tests need a visible MI355X"
    from tsac_hip import native

    native.library()
    return native


@pytest.fixture(scope="module")
def sources(native):
    files = {}
    for channels in (1, 2):
        files[channels] = (native.SourceFile(seeded_models.transformer_file(channels)),
                           native.SourceFile(seeded_models.dac_file(channels)))
    yield files
    for pair in files.values():
        for f in pair:
            f.close()


@pytest.fixture(scope="module")
def models(native, sources):
    made = {}

    def get(channels, cache_bytes=0):
        key = (channels, cache_bytes)
        if key not in made:
            limits = native.Limits()
            limits.cache_bytes = cache_bytes
            made[key] = native.HipModel.from_source(*sources[channels], limits=limits if cache_bytes else None)
        return made[key]

    yield get
    for model in made.values():
        model.close()


def _case(name):
    return json.loads((STREAMS / f"{name}.json").read_text()), (STREAMS / f"{name}.bin").read_bytes()


def _pattern(case):
    return syn.pattern_tokens(case["frames"] * case["groups"] * case["codebooks"])


PATTERN_CASES = ["known_17_8_16", "known_101_3_1", "known_51_3_1", "known_35_3_2", "known_17_1_1", "known_3_8_2",
                 "rollover_1026_1_1", "bounded_90_3_1", "decode_197_3_1", "decode_197_3_2", "decode_3074_3_1",
                 "mono_35_3_2", "stereo_2584_3_1"]


@pytest.mark.parametrize("name", PATTERN_CASES)
def test_encode_writes_the_reference_stream(native, models, name):
    case, stream = _case(name)
    print(f"encode {name}", flush=True)
    h = native.header(case["frames"], case["batch"], case["groups"], case["codebooks"],
                      model_channels=case["channels"])
    with models(case["channels"], case["cache_bytes"]).session() as session:
        got = session.encode(h, _pattern(case))
    assert len(got) == len(stream)
    assert got == stream


@pytest.mark.parametrize("name", PATTERN_CASES)
def test_decode_reads_the_reference_stream(native, models, name):
    case, stream = _case(name)
    print(f"decode {name}", flush=True)
    with models(case["channels"], case["cache_bytes"]).session() as session:
        tokens = session.decode(stream)
    assert np.array_equal(tokens, _pattern(case))


# ---------------------------------------------------------------- audio

AUDIO_CASES = ["stereo_30s_q12", "stereo_10s_q3", "mono_groups_3s_q9"]


def _audio(name):
    path = AUDIO / f"{name}.json"
    if not path.exists():
        pytest.skip(f"reference audio fixture {name} not generated")
    case = json.loads(path.read_text())
    tokens = np.fromfile(AUDIO / f"{name}.tokens", np.uint16)
    assert hashlib.sha256(tokens.tobytes()).hexdigest() == case["tokens_sha256"]
    pcm16 = syn.synthetic_audio(case["seconds"], channels=case["audio_channels"], seed=case["audio_seed"])
    return case, tokens, pcm16


def _padded(case, pcm16):
    """Interleaved float PCM [frames*512][groups*channels], zero-padded."""
    out = np.zeros((case["frames"] * 512, case["audio_channels"]), np.float32)
    out[:pcm16.shape[0]] = pcm16.astype(np.float32) / np.float32(32768)
    return out


def _check_chunks(case, pcm):
    """Every synthesis chunk's float PCM equals the reference's (SHA-256 of its bits)."""
    groups, channels = case["groups"], case["model_channels"]
    pcm = np.ascontiguousarray(pcm, np.float32).reshape(case["frames"] * 512, groups, channels)
    for chunk in case["synthesis"]:
        part = np.ascontiguousarray(pcm[chunk["begin"] * 512:(chunk["begin"] + chunk["frames"]) * 512,
                                        chunk["group"], :])
        assert hashlib.sha256(part.tobytes()).hexdigest() == chunk["sha256"], chunk


@pytest.mark.parametrize("name", AUDIO_CASES)
def test_codec_reproduces_the_reference_audio(native, models, sources, name):
    """Analysis tokens and every synthesis chunk, bit for bit."""
    case, tokens, pcm16 = _audio(name)
    print(f"codec {name}", flush=True)
    channels = case["model_channels"]
    with native.HipDac.from_source(sources[channels][1]) as dac, models(channels).session() as session:
        got = dac.analyze(session, _padded(case, pcm16), case["frames"], case["groups"], case["codebooks"])
        assert np.array_equal(got, tokens)
        pcm = dac.synthesize(session, tokens, case["frames"], case["groups"], case["codebooks"])
    _check_chunks(case, pcm)


@pytest.mark.parametrize("name", AUDIO_CASES)
def test_audio_round_trip_is_the_reference(native, models, sources, name):
    """AudioAnalyzer encode of the recording writes the reference's stream of the
    reference's tokens (entropy batch 3 at 30 s, automatic otherwise), and its
    decode returns the reference's synthesis."""
    case, tokens, pcm16 = _audio(name)
    stream_path = STREAMS / f"audio_{name}.bin"
    if not stream_path.exists():
        pytest.skip(f"reference stream for {name} not generated")
    want = stream_path.read_bytes()
    print(f"audio round trip {name}", flush=True)
    channels = case["model_channels"]
    x = pcm16.astype(np.float32) / np.float32(32768)
    batch = 3 if case["seconds"] == 30.0 else 0
    with native.HipDac.from_source(sources[channels][1]) as dac, models(channels).session() as session:
        stream = dac.encode(session, x, case["audio_channels"], codebooks=case["codebooks"],
                            separate_channels=channels == 1, entropy_batch=batch)
        assert stream == want
        pcm, out_channels = dac.decode(session, want)
    assert out_channels == case["audio_channels"]
    _check_chunks(case, pcm[:case["frames"] * 512])
