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
import struct

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


# ---------------------------------------------------------------- DAC and RVQ

#: Strides of the four DAC stages (src/common/analysis.tpp, synthesis.tpp).
ANALYSIS_STRIDES = (2, 4, 8, 8)
SYNTHESIS_STRIDES = (8, 8, 4, 2)


def dac_shape(synthesis: bool, channels: int, index: int) -> tuple[int, int, int]:
    """Stored axes (axis 0 fastest) of DAC convolution `index`
    (src/models/contract.cpp:55-84): ordinary [input, kernel, output],
    transposed [output, kernel, input]."""
    if index == 0:
        return (1024, 7, 1536) if synthesis else (channels, 7, 64)
    if index == 29:
        return (96, 7, channels) if synthesis else (1024, 3, 1024)
    stage, within = divmod(index - 1, 7)
    width = (1536 >> stage) if synthesis else (64 << stage)
    stride = (SYNTHESIS_STRIDES if synthesis else ANALYSIS_STRIDES)[stage]
    if synthesis and within == 0:
        return (width // 2, 2 * stride, width)
    if not synthesis and within == 6:
        return (width, 2 * stride, width * 2)
    residual = within - 1 if synthesis else within
    w = width // 2 if synthesis else width
    return (w, 7 if residual % 2 == 0 else 1, w)


def dac_bf8(synthesis: bool, index: int) -> bool:
    """Whether the source stores convolution `index` as BF8 (int8 plus one
    BF16 scale per 32 rows) rather than float32 (src/models/contract.cpp:86-92)."""
    return not ((not synthesis and index == 0) or (synthesis and index >= 22))


def dac_activation_width(synthesis: bool, index: int) -> int:
    """Channels of Snake activation `index` (src/models/contract.cpp:109-116)."""
    if index == 28:
        return 96 if synthesis else 1024
    return ((1536 >> (index // 7)) // (1 if index % 7 == 0 else 2)) if synthesis else (64 << (index // 7))


@dataclasses.dataclass
class DacConvolution:
    """One convolution as the DAC source stores it (src/models/types.hpp:33-37):
    `values` float32 [elements] or int8 [elements] with BF16 `scales`
    [outer][rows/32][align8(cols)] (src/weights/preparation.cpp:31-56), the
    weight-norm gain per stored column (last axis) and the bias per output channel."""
    dims: tuple
    values: np.ndarray
    scales: np.ndarray | None
    gain: np.ndarray
    bias: np.ndarray
    transposed: bool

    @property
    def bf8(self) -> bool:
        return self.scales is not None


@dataclasses.dataclass
class DacModel:
    """DAC analysis and synthesis (30 convolutions and 29 Snake alphas each) and
    the quantizer's source tensors per codebook: codebook [1024][8], in_proj
    v [8][1024] (column per output) / g [8] / bias [8], out_proj v [1024][8] /
    g [1024] / bias [1024]."""
    channels: int
    analysis: list
    analysis_alpha: list
    synthesis: list
    synthesis_alpha: list
    codebook: list
    in_v: list
    in_g: list
    in_bias: list
    out_v: list
    out_g: list
    out_bias: list


def _random_convolution(rng, synthesis, channels, index):
    dims = dac_shape(synthesis, channels, index)
    rows, cols, outer = dims
    count = rows * cols * outer
    transposed = synthesis and 1 <= index <= 28 and (index - 1) % 7 == 0
    out_channels = rows if transposed else outer
    if dac_bf8(synthesis, index):
        values = rng.integers(-127, 128, size=count, dtype=np.int8)
        padded = (cols + 7) // 8 * 8
        scales = bf16_bits(rng.uniform(0.002, 0.02, size=(outer, rows // 32, padded)).astype(np.float32))
    else:
        values = rng.standard_normal(count).astype(np.float32)
        scales = None
    gain = rng.uniform(0.6, 1.2, size=outer).astype(np.float32)
    bias = (0.02 * rng.standard_normal(out_channels)).astype(np.float32)
    return DacConvolution(dims, values, scales, gain, bias, transposed)


def random_dac(channels: int = 2, books: int = 12, seed: int = 1) -> DacModel:
    """Seeded random-init DAC and quantizer in the source layouts. Weight norm
    rescales every column to RMS 1/sqrt(fan_in) times its gain, so signals keep
    a moderate scale through both graphs."""
    rng = np.random.default_rng(seed)
    graphs = {}
    for synthesis in (False, True):
        convs = [_random_convolution(rng, synthesis, channels, i) for i in range(30)]
        if synthesis:
            # Random residual stacks grow the signal about a hundredfold; a small
            # exit gain brings the PCM back to roughly full scale.
            convs[29].gain *= np.float32(0.005)
        alphas = [rng.uniform(0.5, 2.0, size=dac_activation_width(synthesis, i)).astype(np.float32)
                  for i in range(29)]
        graphs[synthesis] = (convs, alphas)
    codebook, in_v, in_g, in_bias, out_v, out_g, out_bias = ([] for _ in range(7))
    for _ in range(books):
        codebook.append(rng.standard_normal((1024, 8)).astype(np.float32))
        in_v.append(rng.standard_normal((8, 1024)).astype(np.float32))
        in_g.append(rng.uniform(0.5, 1.5, size=8).astype(np.float32))
        in_bias.append((0.05 * rng.standard_normal(8)).astype(np.float32))
        out_v.append(rng.standard_normal((1024, 8)).astype(np.float32))
        out_g.append(rng.uniform(0.05, 0.15, size=1024).astype(np.float32))
        out_bias.append((0.01 * rng.standard_normal(1024)).astype(np.float32))
    return DacModel(channels, graphs[False][0], graphs[False][1], graphs[True][0], graphs[True][1],
                    codebook, in_v, in_g, in_bias, out_v, out_g, out_bias)


def synthetic_audio(seconds: float, channels: int = 2, seed: int = 0, rate: int = 44100) -> np.ndarray:
    """PCM16 test signal, interleaved [frames][channels]: three seeded sines per
    channel (80-4000 Hz, random phases, -12 dBFS each) plus independent pink
    noise at -12 dBFS (Voss-McCartney, 16 rows), scaled to int16."""
    rng = np.random.default_rng(seed)
    frames = int(round(seconds * rate))
    t = np.arange(frames) / rate
    amplitude = 10 ** (-12 / 20)
    out = np.zeros((frames, channels), np.float64)
    for c in range(channels):
        for _ in range(3):
            f = rng.uniform(80, 4000)
            out[:, c] += amplitude * np.sin(2 * np.pi * f * t + rng.uniform(0, 2 * np.pi))
        rows = 16
        noise = np.zeros(frames)
        values = rng.uniform(-1, 1, rows)
        total = values.sum()
        updates = rng.uniform(-1, 1, (frames, rows))
        index = np.arange(1, frames + 1)
        trailing = np.minimum(np.log2(index & -index).astype(np.int64), rows - 1)
        for i in range(frames):
            r = trailing[i]
            total += updates[i, r] - values[r]
            values[r] = updates[i, r]
            noise[i] = total
        noise /= np.max(np.abs(noise)) + 1e-12
        out[:, c] += amplitude * noise
    out /= max(1.0, np.max(np.abs(out)) / 0.99)
    return np.clip(np.round(out * 32767), -32768, 32767).astype(np.int16)


# ---------------------------------------------------------------- original model files

#: Storage codes of an original model file's tensor records (src/weights/source_model.hpp:11-17).
F32, BF16, BF8, BF8L = 0, 1, 0x8000B, 0x8000E


@dataclasses.dataclass
class SourceTensor:
    """One record of an original model file: dims axis 0 fastest, payload as stored."""
    name: str
    storage: int
    dims: tuple
    payload: bytes


def _padded(data: bytes, alignment: int) -> bytes:
    return data + bytes(-len(data) % alignment)


def f32_tensor(name: str, dims: tuple, values) -> SourceTensor:
    values = np.ascontiguousarray(values, dtype="<f4").ravel()
    assert values.size == int(np.prod(dims)), name
    return SourceTensor(name, F32, tuple(dims), values.tobytes())


def bf16_tensor(name: str, dims: tuple, bits) -> SourceTensor:
    bits = np.ascontiguousarray(bits, dtype="<u2").ravel()
    assert bits.size == int(np.prod(dims)), name
    return SourceTensor(name, BF16, tuple(dims), bits.tobytes())


def quantized_tensor(name: str, dims: tuple, values, scale_bits, block: int) -> SourceTensor:
    """BF8 (block 32) or BF8L (block 256): int8 values in storage order, then
    BF16 scales [outer][dims[0]/block][align8(dims[1])], each plane padded to
    256 bytes (src/weights/source_model.cpp:18-45,148-160)."""
    values = np.ascontiguousarray(values, dtype=np.int8).ravel()
    rows, cols = dims[0], dims[1]
    outer = int(np.prod(dims)) // rows // cols
    scale_bits = np.ascontiguousarray(scale_bits, dtype="<u2")
    assert values.size == int(np.prod(dims)) and scale_bits.shape == (outer, rows // block, (cols + 7) // 8 * 8), name
    payload = _padded(values.tobytes(), 256) + _padded(scale_bits.tobytes(), 256)
    return SourceTensor(name, BF8 if block == 32 else BF8L, tuple(dims), payload)


def source_file(tensors: list, metadata: bytes = b'{"producer": "tsac_hip.synthetic"}') -> bytes:
    """The record format of tsac_*_q8.bin / dac_*_q8.bin (src/weights/source_model.cpp:99-166):
    u32 0x23f4aefb, u32 metadata length, metadata, then per tensor u32 0x23f4aefa,
    u32 storage, u32 rank, u32 name length, u32 dims[rank], name, payload."""
    out = bytearray(struct.pack("<II", 0x23F4AEFB, len(metadata)) + metadata)
    for t in tensors:
        name = t.name.encode()
        out += struct.pack("<IIII", 0x23F4AEFA, t.storage, len(t.dims), len(name))
        out += struct.pack(f"<{len(t.dims)}I", *t.dims) + name + t.payload
    return bytes(out)


def transformer_source(model: Model) -> list:
    """A reference-geometry Model as the tensors of tsac_*_q8.bin
    (src/weights/source_model.cpp:215-266): BF8L projections [K][N] with
    float32 biases (none for the cb_proj tensors), BF16 norms, codebook
    positions and rotary table. The feedback embeddings are not in this file:
    the packer derives them from the codec's quantizer."""
    g = model.geometry
    assert (g.width, g.heads, g.head_width, g.ffn, g.temporal_layers, g.codebook_layers, g.latent,
            g.context) == (512, 4, 128, 2048, 12, 3, 1024, 1024), "the file format holds the reference geometry"
    tensors = []

    def projection(name: str, index: int, with_bias: bool):
        values, scales, bias = model.projections[index]
        k, n = g.projection_shape(index)
        bits = bf16_bits(scales)
        assert np.array_equal(bf16_float(bits), scales), "block scales must be BF16 values"
        padded = np.zeros((1, k // 256, (n + 7) // 8 * 8), np.uint16)
        padded[0, :, :n] = bits
        tensors.append(quantized_tensor(name, (k, n), values, padded, 256))
        if with_bias:
            tensors.append(f32_tensor(name[:-1] + "b", (n,), bias))

    norm = 0
    for stack, layers, first in (("", g.temporal_layers, 0), ("codebook_decoder.", g.codebook_layers,
                                                                 4 * g.temporal_layers)):
        for layer in range(layers):
            h = f"{stack}h{layer}/"
            for ln in ("ln_1/", "ln_2/"):
                tensors.append(bf16_tensor(h + ln + "g", (g.width,), model.norm_gain[norm]))
                tensors.append(bf16_tensor(h + ln + "b", (g.width,), model.norm_bias[norm]))
                norm += 1
            for op, name in enumerate(("attn/c_attn/w", "attn/c_proj/w", "mlp/c_fc/w", "mlp/c_proj/w")):
                projection(h + name, first + 4 * layer + op, True)
        tensors.append(bf16_tensor(stack + "ln_f/g", (g.width,), model.norm_gain[norm]))
        tensors.append(bf16_tensor(stack + "ln_f/b", (g.width,), model.norm_bias[norm]))
        norm += 1
    stacked = 4 * (g.temporal_layers + g.codebook_layers)
    tensors.append(bf16_tensor("codebook_decoder.wpe", (g.width, g.books), model.positions))
    projection("cb_proj", stacked, False)
    projection("codebook_decoder.cb_proj", stacked + 1, False)
    projection("proj_f/w", stacked + 2, True)
    tensors.append(bf16_tensor("rotary_embed", (g.head_width, g.context), model.rotations))
    return tensors


def dac_graph_names(synthesis: bool) -> tuple[list, list]:
    """Tensor stems of a DAC graph's 30 convolutions and 29 Snake activations in
    graph order (src/weights/pack_main.cpp:580-610)."""
    prefix = "decoder.model." if synthesis else "encoder.block."
    convolutions, activations = [prefix + "0"], []
    for stage in range(4):
        block = f"{prefix}{stage + 1}.block."
        if synthesis:
            activations.append(block + "0")
            convolutions.append(block + "1")
        for unit in range(3):
            residual = f"{block}{unit + (2 if synthesis else 0)}.block."
            activations += [residual + "0", residual + "2"]
            convolutions += [residual + "1", residual + "3"]
        if not synthesis:
            activations.append(block + "3")
            convolutions.append(block + "4")
    activations.append(prefix + "5")
    convolutions.append(prefix + "6")
    return convolutions, activations


def dac_source(dac: DacModel) -> list:
    """A DacModel as the tensors of dac_*_q8.bin: per convolution weight_v (BF8 or
    float32, as stored), weight_g, bias; per activation alpha; per codebook the
    quantizer's codebook, in_proj and out_proj."""
    tensors = []
    for synthesis, convs, alphas in ((False, dac.analysis, dac.analysis_alpha),
                                     (True, dac.synthesis, dac.synthesis_alpha)):
        conv_names, act_names = dac_graph_names(synthesis)
        for name, conv in zip(conv_names, convs):
            if conv.bf8:
                tensors.append(quantized_tensor(name + ".weight_v", conv.dims, conv.values, conv.scales, 32))
            else:
                tensors.append(f32_tensor(name + ".weight_v", conv.dims, conv.values))
            tensors.append(f32_tensor(name + ".weight_g", (1, 1, conv.dims[2]), conv.gain))
            tensors.append(f32_tensor(name + ".bias", (conv.bias.size,), conv.bias))
        for name, alpha in zip(act_names, alphas):
            tensors.append(f32_tensor(name + ".alpha", (alpha.size, 1, 1), alpha))
    for book in range(len(dac.codebook)):
        q = f"quantizer.quantizers.{book}."
        tensors += [f32_tensor(q + "codebook.weight", (8, 1024), dac.codebook[book]),
                    f32_tensor(q + "in_proj.weight_v", (1024, 1, 8), dac.in_v[book]),
                    f32_tensor(q + "in_proj.weight_g", (1, 1, 8), dac.in_g[book]),
                    f32_tensor(q + "in_proj.bias", (8,), dac.in_bias[book]),
                    f32_tensor(q + "out_proj.weight_v", (8, 1, 1024), dac.out_v[book]),
                    f32_tensor(q + "out_proj.weight_g", (1, 1, 1024), dac.out_g[book]),
                    f32_tensor(q + "out_proj.bias", (1024,), dac.out_bias[book])]
    return tensors
