"""TEST INFRASTRUCTURE ONLY. Seeded original-format model files for the
reference's own packer.

The reference's composition classes (CpuTransformer, DacAnalysis, DacSynthesis,
RvqEncoder, RvqDecoder) read their weights through TransformerModel and the DAC
model adapters, whose offsets come from the adapter_offsets.hpp that the
reference's packer (src/weights/pack_main.cpp:730-787) writes while it packs
tsac_{mono,stereo}_q8.bin and dac_{mono,stereo}_q8.bin. No trained files exist
offline, so oracle/Makefile writes seeded random-init files in the original
record format with this script, packs them with the packer built from the
reference's sources, and compiles the composition against the generated header.
Tests rebuild the same models from the same seeds for the C oracle.

    python3 seeded_models.py OUTPUT_DIR
"""
import pathlib
import sys

ROOT = pathlib.Path(__file__).resolve().parent.parent
if str(ROOT / "tsac-metal_amd") not in sys.path:
    sys.path.insert(0, str(ROOT / "tsac-metal_amd"))

from tsac_hip import synthetic as syn  # noqa: E402

#: Model channels -> codebooks (src/models/contract.cpp:34-37).
BOOKS = {1: 9, 2: 12}
#: The pack ID the recipe passes to the packer; file names carry it.
PACK_ID = "5eed5eed5eed5eed"


def transformer(channels: int) -> syn.Model:
    """The reference-geometry probability model of one variant."""
    return syn.random_model(syn.Geometry(books=BOOKS[channels], channels=channels), seed=100 + channels)


def dac(channels: int) -> syn.DacModel:
    """The codec (DAC graphs and quantizer) of one variant."""
    return syn.random_dac(channels=channels, books=BOOKS[channels], seed=200 + channels)


def variant(channels: int) -> str:
    return "mono" if channels == 1 else "stereo"


def transformer_file(channels: int) -> bytes:
    return syn.source_file(syn.transformer_source(transformer(channels)))


def dac_file(channels: int) -> bytes:
    return syn.source_file(syn.dac_source(dac(channels)))


def write(directory: pathlib.Path) -> None:
    directory.mkdir(parents=True, exist_ok=True)
    for channels in (1, 2):
        (directory / f"tsac_{variant(channels)}_q8.bin").write_bytes(transformer_file(channels))
        (directory / f"dac_{variant(channels)}_q8.bin").write_bytes(dac_file(channels))


if __name__ == "__main__":
    write(pathlib.Path(sys.argv[1]))
