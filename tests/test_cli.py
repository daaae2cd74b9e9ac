"""The command-line codec on the CPU: option parsing against the reference's
compiled parse_cli (including the rejections of tests/sanitation.cpp:279-309),
the audio files against the reference's compiled pcm16_input, wave_input and
pcm16_wave (including the rejections of tests/sanitation.cpp:204-238), the
stream header the encoder will write, and the tsac-hip binary's behaviour up
to the point where it needs a GPU."""
import os
import pathlib
import struct
import subprocess

import numpy as np
import pytest

from tsac_hip import native
from tsac_hip import synthetic as syn

BINARY = pathlib.Path(native.PACKAGE) / "tsac-hip"

PARSE_CASES = [
    ["c", "in.wav", "out.tsac"],
    ["-v", "-v", "-q", "3", "d", "in.tsac", "out.wav"],
    ["-vv", "t", "in.wav", "out.wav"],
    ["-vq", "3", "c", "in.wav", "out.tsac"],
    ["-q", "+7", "-T", "8", "c", "in.wav", "out.tsac"],
    ["--n_codebooks", "12", "--channels", "2", "--batch_size", "5", "c", "in.sw", "out.tsac"],
    ["-f", "-s", "c", "in.wav", "out.tsac"],
    ["-fs", "--metal", "c", "in.wav", "out.tsac"],
    ["--fast", "--separate_channels", "c", "in.wav", "out.tsac"],
    ["c", "-", "out.tsac"],
    ["--", "c", "-input.wav", "-out.tsac"],
    ["c", "in.wav"],
    ["c", "in.wav", "out.tsac", "extra"],
    [],
    ["-h"],
    ["--help", "--cpu"],
    ["c", "in.wav", "out.tsac", "-h"],
    ["-q", "-3", "c", "in.wav", "out.tsac"],
    # rejected
    ["-q1", "c", "in.wav", "out.tsac"],
    ["-q", "1x", "c", "input"],
    ["-q"],
    ["-x", "c", "in.wav", "out.tsac"],
    ["-vx", "c", "in.wav", "out.tsac"],
    ["--verbose", "c", "in.wav", "out.tsac"],
    ["-q", "", "c", "in.wav", "out.tsac"],
    ["-q", "99999999999", "c", "in.wav", "out.tsac"],
    ["x", "in.wav", "out.tsac"],
] + [[option, "c", "input.wav", "output.tsac"] for option in
     ("--cpu", "--scalar", "--full", "--cuda", "--model", "--trf_model")] + [
    [command, "input", "output"] for command in ("inspect", "tokens", "export-audio", "decode-fast")]


def _mine(arguments):
    try:
        return native.cli_parse(arguments)
    except native.HipError:
        return None


@pytest.mark.parametrize("arguments", PARSE_CASES, ids=lambda a: " ".join(a) or "(none)")
def test_parse_matches_reference(reference, arguments):
    got, want = _mine(arguments), reference.parse_cli(arguments)
    assert (got is None) == (want is None), (got, want)
    if got is None:
        return
    for key in ("threads", "quality", "channels", "batch", "verbose"):
        assert got[key] == want[key], key
    for key in ("fast", "separate", "help", "metal"):
        assert got[key] == bool(want[key]), key
    assert got["command"] == (chr(want["command"]) if want["command"] else "")
    for key in ("input", "output"):
        assert got[key] == (arguments[want[key]] if want[key] >= 0 else None), key


def test_help_text():
    text = native.cli_help()
    for line in ("c infile outfile", "d infile outfile", "t infile outfile", "-q --n_codebooks n",
                 "-s --separate_channels", "-c --channels n", "-f --fast", "--batch_size n", "-v "):
        assert line in text


def _wave(channels, data, rate=44100, bits=16, form=1, chunks=(), fmt_extra=b"", data_size=None, order="fd"):
    fmt = struct.pack("<HHIIHH", form, channels, rate, rate * channels * bits // 8, channels * bits // 8, bits)
    fmt += fmt_extra
    parts = {"f": b"fmt " + struct.pack("<I", len(fmt)) + fmt,
             "d": b"data" + struct.pack("<I", len(data) if data_size is None else data_size) + data}
    body = b"WAVE" + b"".join(chunks) + b"".join(parts[c] for c in order)
    return b"RIFF" + struct.pack("<I", len(body)) + body


def _mine_wave(data):
    try:
        return native.wave_read(data)
    except native.HipError:
        return None


def test_wave_input_matches_reference(reference):
    rng = np.random.default_rng(3)
    pcm = lambda n: rng.integers(-32768, 32768, n, dtype=np.int16).tobytes()
    good = [
        _wave(2, pcm(2 * 700)),
        _wave(1, pcm(1)),
        _wave(8, pcm(8 * 513)),
        _wave(2, pcm(2 * 600) + b"\x01"),                       # incomplete last frame
        _wave(2, pcm(2 * 300), data_size=12),                   # data size ignored
        _wave(2, pcm(2 * 200), chunks=(b"LIST" + struct.pack("<I", 6) + b"abcdef",)),
        _wave(1, pcm(100), fmt_extra=b"\0\0"),                  # 18-byte fmt
        _wave(3, b""),                                          # no samples
    ]
    bad = [
        b"",
        b"RIFX" + _wave(2, pcm(4))[4:],
        _wave(2, pcm(4))[:8] + b"WAVX" + _wave(2, pcm(4))[12:],
        _wave(2, pcm(4), form=3),
        _wave(2, pcm(6), bits=24),
        _wave(0, pcm(4)),
        _wave(9, pcm(18)),
        _wave(2, pcm(4), rate=48000),
        _wave(2, pcm(4), order="df"),                           # data before fmt
        _wave(2, pcm(4), order="f"),                            # no data chunk
        _wave(2, pcm(4))[:38],                                  # truncated chunk header
        _wave(2, pcm(4), chunks=(b"LIST" + struct.pack("<I", 1000) + b"ab",)),
    ]
    for data in good:
        got, want = _mine_wave(data), reference.wave_input(data)
        assert got is not None and want is not None
        assert np.array_equal(got, want)
        assert got.shape[0] % 512 == 0
    for data in bad:
        assert _mine_wave(data) is None and reference.wave_input(data) is None, data[:48]


def test_pcm16_input_matches_reference(reference):
    rng = np.random.default_rng(4)
    for channels in (1, 2, 3, 127):
        data = rng.integers(0, 256, 2 * channels * 700 + 3, dtype=np.uint8).tobytes()
        got = native.pcm16_read(data, channels)
        assert np.array_equal(got, reference.pcm16_input(data, channels))
        assert got.shape == (1024, channels)
    for channels in (0, 128):
        with pytest.raises(native.HipError):
            native.pcm16_read(b"", channels)
        assert reference.pcm16_input(b"", channels) is None


def test_pcm16_wave_matches_reference(reference):
    rng = np.random.default_rng(5)
    ties = (np.arange(-8, 8) + 0.5) / 32768
    edges = [0.0, -0.0, 1.0, -1.0, 1.5, -1.5, 32767.5 / 32768, -32768.5 / 32768, 1e30, -1e30, 1e-40]
    samples = np.concatenate([rng.uniform(-1.2, 1.2, 2000), ties, edges]).astype(np.float32)
    samples = samples[:samples.size // 2 * 2].reshape(-1, 2)
    got = native.wave_write(samples)
    assert got == reference.pcm16_wave(samples)
    assert got[:4] == b"RIFF" and got[8:16] == b"WAVEfmt " and len(got) == 44 + samples.size * 2
    assert np.array_equal(native.wave_read(got)[:samples.shape[0]],
                          np.clip(np.round(samples.astype(np.float64) * 32768), -32768, 32767) / 32768)
    # tests/sanitation.cpp:204-228: the byte limit and nonfinite samples.
    zeros = np.zeros((4, 2), np.float32)
    with pytest.raises(native.HipError):
        native.wave_write(zeros, native.Limits(pcm_bytes=15))
    assert reference.pcm16_wave(zeros, pcm_bytes=15) is None
    for value in (np.inf, np.nan):
        with pytest.raises(native.HipError, match="nonfinite"):
            native.wave_write(np.array([[value]], np.float32))
        assert reference.pcm16_wave(np.array([[value]], np.float32)) is None


def test_audio_header():
    """The header tsac_hip_audio_encode writes (src/common/audio_analyzer.cpp:78-108):
    joint stereo only for exactly two channels, codebooks 0 = the variant's
    maximum, automatic entropy batch."""
    h = native.audio_header(44100 * 30, 2)
    assert (h.method, h.model_channels, h.groups, h.codebooks, h.frames, h.batch) == (1, 2, 1, 12, 2584, 3)
    h = native.audio_header(44100, 2, separate_channels=True, codebooks=5)
    assert (h.model_channels, h.groups, h.codebooks) == (1, 2, 5)
    h = native.audio_header(1000, 4, method=0)
    assert (h.method, h.model_channels, h.groups, h.codebooks, h.frames) == (0, 1, 4, 9, 2)
    assert native.audio_header(44100 * 120, 1, entropy_batch=7).batch == 7
    for kwargs in ({"codebooks": 13}, {"method": 0, "entropy_batch": 2}):
        with pytest.raises(native.HipError):
            native.audio_header(44100, 2, **kwargs)


def _run(*args, env=None):
    return subprocess.run([str(BINARY), *args], capture_output=True, text=True, timeout=120,
                          env={**os.environ, **(env or {})})


def test_binary_without_gpu_work(tmp_path):
    assert BINARY.exists(), "tsac-hip is built by make -C tsac-metal_amd"
    r = _run("-h")
    assert r.returncode == 1 and "usage: tsac-hip" in r.stdout
    r = _run("c", "in.wav")
    assert r.returncode == 1 and "usage: tsac-hip" in r.stdout
    r = _run("--cuda", "c", "a", "b")
    assert r.returncode == 1 and "tsac-hip: unrecognised option --cuda" in r.stderr
    r = _run("c", str(tmp_path / "absent.wav"), str(tmp_path / "out.tsac"))
    assert r.returncode == 1 and "cannot open input" in r.stderr
    wav = tmp_path / "in.wav"
    wav.write_bytes(native.wave_write(np.zeros((1024, 2), np.float32)))
    r = _run("c", str(wav), str(tmp_path / "out.tsac"), env={"TSAC_HIP_MODELS": str(tmp_path)})
    assert r.returncode == 1 and "cannot open model file" in r.stderr and "tsac_stereo_q8.bin" in r.stderr
    bad = tmp_path / "bad.wav"
    bad.write_bytes(b"RIFF0000WAVX")
    r = _run("c", str(bad), str(tmp_path / "out.tsac"))
    assert r.returncode == 1 and "bad.wav: invalid wav file" in r.stderr
