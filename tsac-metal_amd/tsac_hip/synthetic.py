"""Seeded synthetic models, tokens and audio-shaped inputs in the reference layout.

No trained TSAC weights exist offline, so benchmarks and parity tests run on
random-init weights laid out exactly as the reference's packed Transformer
roles hold them (src/weights/pack_main.cpp:305-391, src/models/types.hpp:44-48):

* projection ``p``: int8 values ``[N][K]`` (input fastest), fp32 block scales
  ``[K/256][N]`` (widened BF16, so every scale is BF16-representable), fp32 bias ``[N]``;
* norms: BF16 gain and bias ``[width]``;
* learned codebook positions (``wpe``): BF16 ``[books][width]``;
* rotary coefficients: BF16 ``[context][head_width]``, interleaved (cos, sin) pairs;
* feedback embeddings: BF16 ``[books][alphabet][latent]``.

Projection and norm indices follow src/models/contract.cpp:88-110,195-211.
"""
from __future__ import annotations

import dataclasses
import math

import numpy as np


@dataclasses.dataclass(frozen=True)
class Geometry:
    """Model shape. The reference fixes width 512, 4x128 heads, FFN 2048,
    12 temporal + 3 codebook layers, context 1024 (src/models/config.hpp:11-16)."""

    width: int = 512
    heads: int = 4
    head_width: int = 128
    ffn: int = 2048
    temporal_layers: int = 12
    codebook_layers: int = 3
    latent: int = 1024
    alphabet: int = 1024
    books: int = 12
    channels: int = 2
    context: int = 1024

    @property
    def attention_scale(self) -> float:
        # 0.0883883461356163f for 128-wide heads (src/common/cpu_transformer.tpp:164).
        return float(np.float32(1.0 / math.sqrt(self.head_width)))

    @property
    def projection_count(self) -> int:
        return 4 * (self.temporal_layers + self.codebook_layers) + 3

    @property
    def norm_count(self) -> int:
        return 2 * (self.temporal_layers + self.codebook_layers) + 2

    def projection_shape(self, index: int) -> tuple[int, int]:
        """(K input, N output) of projection ``index``."""
        stacked = 4 * (self.temporal_layers + self.codebook_layers)
        if index in (stacked, stacked + 1):
            return self.latent, self.width
        if index == stacked + 2:
            return self.width, self.alphabet
        return [
            (self.width, 3 * self.width),
            (self.width, self.width),
            (self.width, self.ffn),
            (self.ffn, self.width),
        ][index % 4]


#: The reference model geometry (stereo variant, 12 codebooks).
REFERENCE = Geometry()
#: The wider geometry named by the throughput configuration: width 1024,
#: FFN 4096, 16 heads of 64, same 12 + 3 layer stacks.
WIDE = Geometry(width=1024, heads=16, head_width=64, ffn=4096)


def bf16_bits(values: np.ndarray) -> np.ndarray:
    """fp32 -> BF16 bit patterns with the reference's integer ties-to-even rule
    (src/common/numeric/bf16.hpp:9-13)."""
    a = np.asarray(values, dtype=np.float32)
    b = np.ascontiguousarray(a).view(np.uint32).astype(np.uint64).reshape(a.shape)
    return ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16)


def bf16_float(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


@dataclasses.dataclass
class Model:
    geometry: Geometry
    projections: list  # [(values int8 [N][K], scales f32 [K/256][N], bias f32 [N])]
    norm_gain: list  # [uint16 [width]]
    norm_bias: list
    positions: np.ndarray  # uint16 [books][width]
    rotations: np.ndarray  # uint16 [context][head_width]
    embeddings: np.ndarray  # uint16 [books][alphabet][latent]


def random_linear(rng: np.random.Generator, k: int, n: int, bias_std: float = 0.02,
                  row_scales: bool = False):
    """int8 U{-127..127}; scales U(0.001, 0.02) rounded to BF16 (one per output
    row replicated over the K/256 blocks when ``row_scales``); fp32 bias."""
    values = rng.integers(-127, 128, size=(n, k), dtype=np.int8)
    if row_scales:
        row = rng.uniform(0.001, 0.02, size=n).astype(np.float32)
        scales = np.broadcast_to(row, (k // 256, n)).copy()
    else:
        scales = rng.uniform(0.001, 0.02, size=(k // 256, n)).astype(np.float32)
    scales = bf16_float(bf16_bits(scales)).reshape(k // 256, n).copy()
    bias = (rng.standard_normal(n) * bias_std).astype(np.float32) if bias_std else np.zeros(
        n, np.float32)
    return values, scales, bias


def rotary_table(geometry: Geometry) -> np.ndarray:
    pairs = geometry.head_width // 2
    position = np.arange(geometry.context, dtype=np.float64)[:, None]
    frequency = 10000.0 ** (-np.arange(pairs, dtype=np.float64) / pairs)
    angle = position * frequency[None, :]
    table = np.empty((geometry.context, geometry.head_width), np.float32)
    table[:, 0::2] = np.cos(angle)
    table[:, 1::2] = np.sin(angle)
    return bf16_bits(table)


def random_model(geometry: Geometry = REFERENCE, seed: int = 1) -> Model:
    rng = np.random.default_rng(seed)
    projections = []
    stacked = 4 * (geometry.temporal_layers + geometry.codebook_layers)
    for p in range(geometry.projection_count):
        k, n = geometry.projection_shape(p)
        # cb_proj tensors carry no bias (src/weights/pack_main.cpp:352-360).
        projections.append(random_linear(rng, k, n, 0.0 if p in (stacked, stacked + 1) else 0.02))
    norm_gain = [bf16_bits(1.0 + 0.1 * rng.standard_normal(geometry.width).astype(np.float32))
                 for _ in range(geometry.norm_count)]
    norm_bias = [bf16_bits(0.1 * rng.standard_normal(geometry.width).astype(np.float32))
                 for _ in range(geometry.norm_count)]
    positions = bf16_bits(0.5 * rng.standard_normal((geometry.books, geometry.width)).astype(
        np.float32))
    embeddings = bf16_bits(rng.standard_normal(
        (geometry.books, geometry.alphabet, geometry.latent)).astype(np.float32))
    return Model(geometry, projections, norm_gain, norm_bias, positions, rotary_table(geometry),
                 embeddings)


def random_tokens(frames: int, groups: int, books: int, seed: int = 7,
                  alphabet: int = 1024) -> np.ndarray:
    """Tokens uniform over the alphabet in the reference's (frame, group, book) order."""
    rng = np.random.default_rng(seed)
    return rng.integers(0, alphabet, size=frames * groups * books, dtype=np.uint16)


def pattern_tokens(count: int) -> np.ndarray:
    """The reference tests' token pattern (i*73+19) % 1024 (tests/metal_optimized.cpp:270-273)."""
    i = np.arange(count, dtype=np.int64)
    return ((i * 73 + 19) % 1024).astype(np.uint16)
