"""Writes the reference's own DAC analysis, RVQ and synthesis results for the
seeded codec as fixtures.

Runs in the build container only, where oracle/Makefile has compiled the
reference's DacAnalysis, DacSynthesis, RvqEncoder and RvqDecoder
(oracle/_ref/libtsacmodel.so) against the header its own packer generated for
the seeded model files of oracle/seeded_models.py.

Each case is synthetic PCM16 audio (tsac_hip.synthetic.synthetic_audio), taken
as float x/32768 and zero-padded to whole 512-sample frames the way
AudioAnalyzer pads it (src/common/audio_analyzer.cpp:117-138). The recording is
cut into the reference's chunks (audio_chunk, src/common/audio_analyzer.cpp:154-162:
400 central frames, 8 + 9 context frames for analysis, 11 + 11 for synthesis);
every chunk window runs through the reference's DacAnalysis::apply and
RvqEncoder::encode, or RvqDecoder::decode and DacSynthesis::apply, and keeps
its central frames, which is what the reference's analyze_audio /
synthesize_audio do (src/common/audio_pipeline.hpp:37-79). Windows are
evaluated concurrently, one reference model per worker.

Per case, tests/golden/reference_audio/<case>.json holds the shape, the tokens'
SHA-256 and, per synthesis chunk, the SHA-256 of its float PCM bits; the tokens
themselves go to <case>.tokens (uint16, [frame][group][book]).

    python3 tests/golden/make_reference_audio.py [CASE ...]
"""
import concurrent.futures
import hashlib
import json
import pathlib
import sys

ROOT = pathlib.Path(__file__).resolve().parents[2]
for p in (ROOT / "oracle", ROOT / "tsac-metal_amd"):
    sys.path.insert(0, str(p))

import numpy as np  # noqa: E402

OUT = pathlib.Path(__file__).resolve().parent / "reference_audio"
CHUNK = 400
WORKERS = 8

#: name -> (seconds, audio seed, audio channels, model channels, codebooks)
CASES = {
    # The 30 s joint-stereo recording at 12 codebooks (2584 frames).
    "stereo_30s_q12": (30.0, 4, 2, 2, 12),
    # The 10 s joint-stereo recording at 3 codebooks (862 frames).
    "stereo_10s_q3": (10.0, 3, 2, 2, 3),
    # Stereo audio coded as two mono groups (separate channels), 9 codebooks.
    "mono_groups_3s_q9": (3.0, 5, 2, 1, 9),
}


def padded_pcm(seconds, seed, channels, model_channels):
    """float PCM [groups][frames*512][model_channels] and the frame count."""
    from tsac_hip.synthetic import synthetic_audio

    pcm16 = synthetic_audio(seconds, channels=channels, seed=seed)
    samples = pcm16.shape[0]
    frames = (samples + 511) // 512
    groups = channels // model_channels
    out = np.zeros((groups, frames * 512, model_channels), np.float32)
    x = pcm16.astype(np.float32) / np.float32(32768)
    for g in range(groups):
        out[g, :samples, :] = x[:, g * model_channels:(g + 1) * model_channels]
    return out, frames


def chunks(frames, left_context, right_context):
    """(begin, count, left, right) of every chunk (src/common/audio_analyzer.cpp:154-162)."""
    begin = 0
    while begin < frames:
        count = min(CHUNK, frames - begin)
        end = begin + count
        yield begin, count, (begin - left_context if begin > left_context else 0), end + min(right_context,
                                                                                             frames - end)
        begin = end


def run_case(name):
    from oracle import ReferenceComposition

    seconds, seed, channels, model_channels, books = CASES[name]
    composition = ReferenceComposition()
    pcm, frames = padded_pcm(seconds, seed, channels, model_channels)
    groups = pcm.shape[0]
    pool = [composition.dac(model_channels, books) for _ in range(WORKERS)]
    free = list(pool)

    def with_model(work):
        dac = free.pop()
        try:
            return work(dac)
        finally:
            free.append(dac)

    def analyze(group, chunk):
        begin, count, left, right = chunk
        window = pcm[group, left * 512:right * 512]

        def work(dac):
            latent = dac.analysis(window, (right - left) * 512).reshape(right - left, 1024)
            return dac.rvq_encode(latent[begin - left:begin - left + count], count)
        return with_model(work)

    tokens = np.zeros((frames, groups, books), np.uint16)
    with concurrent.futures.ThreadPoolExecutor(WORKERS) as executor:
        jobs = {(g, c): executor.submit(analyze, g, c) for g in range(groups) for c in chunks(frames, 8, 9)}
        for (g, (begin, count, _, _)), job in jobs.items():
            tokens[begin:begin + count, g, :] = job.result().reshape(count, books)

        def synthesize(group, chunk):
            begin, count, left, right = chunk
            selected = np.ascontiguousarray(tokens[left:right, group, :])

            def work(dac):
                latent = dac.rvq_decode(selected, right - left)
                audio = dac.synthesis(latent, right - left).reshape((right - left) * 512, model_channels)
                return audio[(begin - left) * 512:(begin - left + count) * 512]
            return with_model(work)

        jobs = {(g, c): executor.submit(synthesize, g, c) for g in range(groups) for c in chunks(frames, 11, 11)}
        synthesis = [{"group": g, "begin": c[0], "frames": c[1],
                      "sha256": hashlib.sha256(np.ascontiguousarray(job.result()).tobytes()).hexdigest()}
                     for (g, c), job in jobs.items()]
    for dac in pool:
        dac.close()
    OUT.mkdir(exist_ok=True)
    (OUT / f"{name}.tokens").write_bytes(tokens.tobytes())
    case = {"seconds": seconds, "audio_seed": seed, "audio_channels": channels, "model_channels": model_channels,
            "codebooks": books, "frames": frames, "groups": groups, "chunk": CHUNK,
            "pcm": "synthetic_audio(seconds, audio_channels, audio_seed) / 32768, zero-padded to frames * 512",
            "tokens_sha256": hashlib.sha256(tokens.tobytes()).hexdigest(), "synthesis": synthesis}
    (OUT / f"{name}.json").write_text(json.dumps(case, indent=1) + "\n")
    print(name, frames, "frames", flush=True)


if __name__ == "__main__":
    for case_name in sys.argv[1:] or list(CASES):
        run_case(case_name)
