"""Writes the reference's own FBAZ streams for the seeded models as fixtures.

Runs in the build container only, where oracle/Makefile has compiled the
reference's CpuTransformer<scalar::Kernels>, TransformerPredictor and
pack_normal (oracle/_ref/libtsacmodel.so) against the header its own packer
generated for the seeded model files of oracle/seeded_models.py. Each case is
one shape of tests/metal_optimized.cpp (known-token streams :253-259, bounded
lookahead :277-292, resident decode :519-523), a two-group mono case and the
30 s stereo layout (2584 frames in lanes of 862/861/861). Each stream and its
description (shape, model, token rule, length, SHA-256) go to
tests/golden/reference_streams/<case>.{bin,json}; the GPU tests hold the HIP
library's streams and decodes against them byte for byte.

    python3 tests/golden/make_reference_streams.py [CASE ...]
"""
import hashlib
import json
import pathlib
import sys

ROOT = pathlib.Path(__file__).resolve().parents[2]
for p in (ROOT / "oracle", ROOT / "tsac-metal_amd"):
    sys.path.insert(0, str(p))

import numpy as np  # noqa: E402

OUT = pathlib.Path(__file__).resolve().parent / "reference_streams"

AUDIO = pathlib.Path(__file__).resolve().parent / "reference_audio"

#: name -> (model channels, (frames, batch, groups, codebooks), cache_bytes);
#: cases named audio_<case> code the tokens of reference_audio/<case>.tokens
#: (the reference's analysis of that recording) instead of the token rule.
CASES = {
    "known_17_8_16": (2, (17, 8, 16, 12), 0),
    "known_101_3_1": (2, (101, 3, 1, 12), 0),
    "known_51_3_1": (2, (51, 3, 1, 12), 0),
    "known_35_3_2": (2, (35, 3, 2, 12), 0),
    "known_17_1_1": (2, (17, 1, 1, 12), 0),
    "known_3_8_2": (2, (3, 8, 2, 12), 0),
    "rollover_1026_1_1": (2, (1026, 1, 1, 1), 0),
    "bounded_90_3_1": (2, (90, 3, 1, 1), 2300000),
    "decode_197_3_1": (2, (197, 3, 1, 1), 0),
    "decode_197_3_2": (2, (197, 3, 2, 1), 0),
    "decode_3074_3_1": (2, (3074, 3, 1, 1), 0),
    "mono_35_3_2": (1, (35, 3, 2, 9), 0),
    "stereo_2584_3_1": (2, (2584, 3, 1, 12), 0),
    # The 30 s joint-stereo recording, 12 codebooks, entropy batch 3.
    "audio_stereo_30s_q12": (2, (2584, 3, 1, 12), 0),
    # The 10 s joint-stereo recording, 3 codebooks, automatic batch (one lane).
    "audio_stereo_10s_q3": (2, (862, 1, 1, 3), 0),
    # Stereo as two mono groups, 9 codebooks, automatic batch.
    "audio_mono_groups_3s_q9": (1, (259, 1, 2, 9), 0),
}


def tokens(shape, name="") -> np.ndarray:
    """The reference tests' token rule (i*73+19) % 1024 (tests/metal_optimized.cpp:270-273),
    or the analysed recording's tokens for an audio_ case."""
    frames, _, groups, books = shape
    if name.startswith("audio_"):
        t = np.fromfile(AUDIO / f"{name[6:]}.tokens", np.uint16)
        assert t.size == frames * groups * books, name
        return t
    i = np.arange(frames * groups * books, dtype=np.int64)
    return ((i * 73 + 19) % 1024).astype(np.uint16)


def main(names):
    from oracle import ReferenceComposition, header
    import seeded_models

    composition = ReferenceComposition()
    OUT.mkdir(exist_ok=True)
    for name in names:
        channels, shape, cache_bytes = CASES[name]
        with composition.transformer(channels, seeded_models.BOOKS[channels], cache_bytes) as model:
            stream = model.pack_normal(header(*shape, model_channels=channels), tokens(shape, name), threads=8)
        (OUT / f"{name}.bin").write_bytes(stream)
        case = {"channels": channels, "frames": shape[0], "batch": shape[1], "groups": shape[2],
                          "codebooks": shape[3], "cache_bytes": cache_bytes,
                "tokens": f"reference_audio/{name[6:]}.tokens" if name.startswith("audio_") else "(i*73+19)%1024",
                          "bytes": len(stream), "sha256": hashlib.sha256(stream).hexdigest()}
        (OUT / f"{name}.json").write_text(json.dumps(case, indent=1) + "\n")
        print(name, len(stream), flush=True)


if __name__ == "__main__":
    main(sys.argv[1:] or list(CASES))
