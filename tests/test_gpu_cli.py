"""The tsac-hip binary end to end on the MI355X with seeded original-format
model files: compression writes the stream the library's AudioAnalyzer entry
point writes for the same PCM and options; decompression writes the WAVE of
the library's decoded PCM; "t" equals "c" then "d"; -v / -vv print the
statistics lines; fast framing, separate channels (the mono model with two
groups), raw .sw input and a forced entropy batch go through the same path."""
import os
import pathlib
import subprocess

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
def models(native, tmp_path_factory):
    directory = tmp_path_factory.mktemp("models")
    for channels, books, variant in ((2, 12, "stereo"), (1, 9, "mono")):
        geometry = syn.Geometry(channels=channels, books=books)
        (directory / f"tsac_{variant}_q8.bin").write_bytes(
            syn.source_file(syn.transformer_source(syn.random_model(geometry, seed=channels))))
        (directory / f"dac_{variant}_q8.bin").write_bytes(
            syn.source_file(syn.dac_source(syn.random_dac(channels=channels, books=books, seed=channels))))
    return directory


def _run(models, *args):
    binary = pathlib.Path(__file__).resolve().parent.parent / "tsac-metal_amd" / "tsac-hip"
    print("tsac-hip", *args, flush=True)
    return subprocess.run([str(binary), *map(str, args)], capture_output=True, text=True, timeout=240,
                          env={**os.environ, "TSAC_HIP_MODELS": str(models)})


def _library(native, models, variant):
    transformer = native.SourceFile(path=models / f"tsac_{variant}_q8.bin")
    codec = native.SourceFile(path=models / f"dac_{variant}_q8.bin")
    model = native.HipModel.from_source(transformer, codec)
    return model, model.session(), native.HipDac.from_source(codec), (transformer, codec)


def _close(parts):
    model, session, dac, sources = parts
    for p in (dac, session, model, *sources):
        p.close()


def test_compress_decompress_round_trip(native, models, tmp_path):
    audio = syn.synthetic_audio(2.0, 2, seed=5).astype(np.float32) / np.float32(32768)
    wav = tmp_path / "in.wav"
    wav.write_bytes(native.wave_write(audio))
    pcm = native.wave_read(wav.read_bytes())
    r = _run(models, "-q", "4", "c", wav, tmp_path / "out.tsac")
    assert r.returncode == 0, r.stderr
    stream = (tmp_path / "out.tsac").read_bytes()
    parts = _library(native, models, "stereo")
    try:
        model, session, dac, _ = parts
        assert stream == dac.encode(session, pcm, 2, codebooks=4)
        decoded, channels = dac.decode(session, stream)
        assert channels == 2
    finally:
        _close(parts)
    r = _run(models, "d", tmp_path / "out.tsac", tmp_path / "out.wav")
    assert r.returncode == 0, r.stderr
    assert (tmp_path / "out.wav").read_bytes() == native.wave_write(decoded)
    r = _run(models, "-q", "4", "t", wav, tmp_path / "rt.wav")
    assert r.returncode == 0, r.stderr
    assert (tmp_path / "rt.wav").read_bytes() == (tmp_path / "out.wav").read_bytes()


def test_statistics_and_options(native, models, tmp_path):
    audio = syn.synthetic_audio(1.0, 2, seed=6).astype(np.float32) / np.float32(32768)
    wav = tmp_path / "in.wav"
    wav.write_bytes(native.wave_write(audio))
    r = _run(models, "-vv", "-q", "3", "--batch_size", "4", "c", wav, tmp_path / "a.tsac")
    assert r.returncode == 0, r.stderr
    assert "batch_size=4 bs=1 n_cb=3 block_len=22" in r.stdout
    assert "CB AVG_BITS" in r.stdout and "bitrate=" in r.stdout and " kb/s, max_memory=" in r.stdout
    header = native.parse_header((tmp_path / "a.tsac").read_bytes())
    assert (header.batch, header.codebooks, header.model_channels) == (4, 3, 2)
    r = _run(models, "-f", "c", wav, tmp_path / "fast.tsac")
    assert r.returncode == 0, r.stderr
    frames = -(-audio.shape[0] // 512)
    assert len((tmp_path / "fast.tsac").read_bytes()) == 8 + (frames * 12 * 10 + 7) // 8
    r = _run(models, "d", tmp_path / "fast.tsac", tmp_path / "fast.wav")
    assert r.returncode == 0, r.stderr
    assert native.wave_read((tmp_path / "fast.wav").read_bytes()).shape == (frames * 512, 2)
    # Separate channels: the mono model, two groups; decoded back to two channels.
    r = _run(models, "-s", "-q", "2", "t", wav, tmp_path / "sep.wav")
    assert r.returncode == 0, r.stderr
    assert native.wave_read((tmp_path / "sep.wav").read_bytes()).shape == (frames * 512, 2)
    # Raw 16-bit input with a forced channel count.
    raw = tmp_path / "in.sw"
    raw.write_bytes((np.clip(np.round(audio * 32768), -32768, 32767).astype("<i2")).tobytes())
    r = _run(models, "-c", "2", "-q", "4", "c", raw, tmp_path / "raw.tsac")
    assert r.returncode == 0, r.stderr
    assert (tmp_path / "raw.tsac").read_bytes() == _compress_bytes(native, models, wav)


def _compress_bytes(native, models, wav):
    parts = _library(native, models, "stereo")
    try:
        _, session, dac, _ = parts
        return dac.encode(session, native.wave_read(wav.read_bytes()), 2, codebooks=4)
    finally:
        _close(parts)
