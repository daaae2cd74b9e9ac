"""TEST INFRASTRUCTURE ONLY: ctypes bindings of the CPU oracle (liboracle.so)
and of the compiled reference sources (_ref/libtsacref.so).

Only tests/, ``__graft_entry__.smoke()`` and bench.py's CPU baseline import
this module, and only as the checker or the reported CPU baseline.
"""
from __future__ import annotations

import ctypes as C
import os
import pathlib

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
ORACLE_PATH = HERE / "liboracle.so"
REF_PATH = HERE / "_ref" / "libtsacref.so"

u8p = C.POINTER(C.c_uint8)
u16p = C.POINTER(C.c_uint16)
i8p = C.POINTER(C.c_int8)
f32p = C.POINTER(C.c_float)
sz = C.c_size_t


class Header(C.Structure):
    _fields_ = [("method", C.c_uint8), ("groups", C.c_uint8), ("model_channels", C.c_uint8),
                ("codebooks", C.c_uint8), ("frames", C.c_uint64), ("batch", C.c_uint16)]


class Geometry(C.Structure):
    _fields_ = [(name, C.c_uint32) for name in (
        "width", "heads", "head_width", "ffn", "temporal_layers", "codebook_layers", "latent",
        "alphabet", "books", "channels", "context")] + [("attention_scale", C.c_float)]


class Linear(C.Structure):
    _fields_ = [("values", i8p), ("scales", f32p), ("bias", f32p)]


class ModelDesc(C.Structure):
    _fields_ = [("geometry", Geometry), ("projections", C.POINTER(Linear)),
                ("norm_gain", C.POINTER(u16p)), ("norm_bias", C.POINTER(u16p)),
                ("positions", u16p), ("rotations", u16p), ("embeddings", u16p)]


def ptr(array: np.ndarray, ctype):
    assert array.flags["C_CONTIGUOUS"]
    return array.ctypes.data_as(C.POINTER(ctype))


class OracleError(RuntimeError):
    pass


def _load(path: pathlib.Path):
    if not path.exists():
        raise FileNotFoundError(f"{path} is not built (run `make -C oracle`)")
    return C.CDLL(str(path))


def _declare(lib, prefix: str):
    f = lambda name: getattr(lib, prefix + name)  # noqa: E731
    f("last_error").restype = C.c_char_p
    f("bf16").restype = C.c_uint16
    f("bf16").argtypes = [C.c_float]
    f("exp").restype = C.c_float
    f("exp").argtypes = [C.c_float]
    f("probability_sum").restype = C.c_float
    f("probability_sum").argtypes = [f32p, sz]
    f("conditional_q15").restype = C.c_uint16
    f("conditional_q15").argtypes = [C.c_float, C.c_float]
    f("bf8l").argtypes = [f32p, sz, i8p, u16p]
    f("qlinear").argtypes = [i8p, f32p, f32p, sz, sz, u16p, sz, u16p]
    f("layer_norm").argtypes = [u16p, u16p, u16p, sz, u16p]
    f("gelu").restype = C.c_uint16
    f("gelu").argtypes = [C.c_uint16]
    f("add_bf16").restype = C.c_uint16
    f("add_bf16").argtypes = [C.c_uint16, C.c_uint16]
    f("rotary").argtypes = [u16p, u16p, sz, u16p]
    f("softmax").argtypes = [u16p, sz, u16p]
    f("token_crc32").restype = C.c_uint32
    f("token_crc32").argtypes = [u16p, sz]
    f("exp_batch").argtypes = [f32p, sz, f32p]
    f("bf16_batch").argtypes = [f32p, sz, u16p]


class _Kernels:
    """Kernel-level calls shared by the oracle and the compiled reference."""

    def __init__(self, lib, prefix):
        self.lib, self.prefix = lib, prefix
        _declare(lib, prefix)

    def _f(self, name):
        return getattr(self.lib, self.prefix + name)

    def _check(self, status):
        if status:
            raise OracleError(self._f("last_error")().decode())

    def bf16(self, x: float) -> int:
        return self._f("bf16")(x)

    def exp(self, z: float) -> float:
        return self._f("exp")(z)

    def exp_batch(self, z):
        z = np.ascontiguousarray(z, np.float32)
        out = np.empty_like(z)
        self._f("exp_batch")(ptr(z, C.c_float), z.size, ptr(out, C.c_float))
        return out

    def bf16_batch(self, x):
        x = np.ascontiguousarray(x, np.float32)
        out = np.empty(x.shape, np.uint16)
        self._f("bf16_batch")(ptr(x, C.c_float), x.size, ptr(out, C.c_uint16))
        return out

    def probability_sum(self, values) -> float:
        v = np.ascontiguousarray(values, np.float32)
        return self._f("probability_sum")(ptr(v, C.c_float), v.size)

    def conditional_q15(self, left: float, mass: float) -> int:
        return self._f("conditional_q15")(left, mass)

    def bf8l(self, values):
        v = np.ascontiguousarray(values, np.float32)
        q = np.zeros(v.size, np.int8)
        s = np.zeros(v.size // 256 if v.size % 256 == 0 else 1, np.uint16)
        self._check(self._f("bf8l")(ptr(v, C.c_float), v.size, ptr(q, C.c_int8), ptr(s, C.c_uint16)))
        return q, s

    def qlinear(self, weights, scales, bias, x):
        n, k = weights.shape
        x = np.ascontiguousarray(x, np.uint16).reshape(-1, k)
        y = np.zeros((x.shape[0], n), np.uint16)
        self._check(self._f("qlinear")(
            ptr(np.ascontiguousarray(weights), C.c_int8), ptr(np.ascontiguousarray(scales), C.c_float),
            ptr(np.ascontiguousarray(bias), C.c_float), k, n, ptr(x, C.c_uint16), x.shape[0],
            ptr(y, C.c_uint16)))
        return y

    def layer_norm(self, x, gain, bias):
        x = np.ascontiguousarray(x, np.uint16)
        out = np.zeros_like(x)
        self._check(self._f("layer_norm")(ptr(x, C.c_uint16), ptr(np.ascontiguousarray(gain), C.c_uint16),
                                          ptr(np.ascontiguousarray(bias), C.c_uint16), x.size,
                                          ptr(out, C.c_uint16)))
        return out

    def gelu(self, x: int) -> int:
        return self._f("gelu")(x)

    def add_bf16(self, a: int, b: int) -> int:
        return self._f("add_bf16")(a, b)

    def rotary(self, values, coefficients):
        v = np.ascontiguousarray(values, np.uint16)
        out = np.zeros_like(v)
        self._check(self._f("rotary")(ptr(v, C.c_uint16),
                                      ptr(np.ascontiguousarray(coefficients, np.uint16), C.c_uint16),
                                      v.size, ptr(out, C.c_uint16)))
        return out

    def softmax(self, x):
        x = np.ascontiguousarray(x, np.uint16)
        out = np.zeros_like(x)
        self._check(self._f("softmax")(ptr(x, C.c_uint16), x.size, ptr(out, C.c_uint16)))
        return out

    def token_crc32(self, tokens) -> int:
        t = np.ascontiguousarray(tokens, np.uint16)
        return self._f("token_crc32")(ptr(t, C.c_uint16), t.size)


class OrcConv(C.Structure):
    _fields_ = [(n, sz) for n in ("input", "output", "kernel", "stride", "padding", "dilation")] + \
        [("transposed", C.c_int)]


class OrcDac(C.Structure):
    _fields_ = [("synthesis", C.c_int), ("channels", C.c_uint), ("weights", f32p * 30), ("bias", f32p * 30),
                ("alpha", f32p * 29)]


class OrcRvq(C.Structure):
    _fields_ = [("books", C.c_uint)] + [(n, f32p * 12) for n in (
        "codebook", "search", "input_weights", "input_bias", "output_weights", "output_bias")]


def _f32(a):
    return np.ascontiguousarray(a, np.float32)


class _DspKernels:
    """DAC/RVQ primitives shared by the oracle (orc_) and the compiled reference (ref_)."""

    def _declare_dsp(self):
        f = self._f
        f("conv1d").argtypes = [C.POINTER(OrcConv), f32p, f32p, f32p, sz, sz, f32p] + \
            ([C.c_uint] if self.prefix == "orc_" else [])
        f("snake").argtypes = [f32p, sz, sz, f32p, f32p]
        f("fold_dac_weight_norm").argtypes = [f32p, f32p, sz, sz, f32p]
        f("normalize_search").argtypes = [f32p, f32p]
        f("normalize_search").restype = None
        f("nearest_rvq").argtypes = [f32p, f32p]
        f("nearest_rvq").restype = C.c_uint16
        f("project_codebook").argtypes = [C.c_uint16, f32p, f32p, f32p, f32p]
        f("project_codebook").restype = None

    def conv1d(self, config: OrcConv, w, bias, x, frames, groups=1, threads=4):
        x, w, bias = _f32(x), _f32(w), _f32(bias)
        if config.transposed:
            span = (config.kernel - 1) * config.dilation + 1
            out_frames = (frames - 1) * config.stride + span - 2 * config.padding
        else:
            out_frames = (frames + 2 * config.padding - ((config.kernel - 1) * config.dilation + 1)) // config.stride + 1
        y = np.zeros(out_frames * groups * config.output, np.float32)
        args = [C.byref(config), ptr(w, C.c_float), ptr(bias, C.c_float), ptr(x, C.c_float), frames, groups,
                ptr(y, C.c_float)] + ([threads] if self.prefix == "orc_" else [])
        self._check(self._f("conv1d")(*args))
        return y

    def snake(self, x, channels, alpha):
        x, alpha = _f32(x), _f32(alpha)
        out = np.zeros_like(x)
        self._check(self._f("snake")(ptr(x, C.c_float), x.size, channels, ptr(alpha, C.c_float), ptr(out, C.c_float)))
        return out

    def fold_dac_weight_norm(self, v, g, fan_in):
        v, g = _f32(v), _f32(g)
        out = np.zeros(v.size, np.float32)
        self._check(self._f("fold_dac_weight_norm")(ptr(v, C.c_float), ptr(g, C.c_float), fan_in, g.size,
                                                    ptr(out, C.c_float)))
        return out

    def normalize_search(self, x):
        x = _f32(x)
        out = np.zeros(8, np.float32)
        self._f("normalize_search")(ptr(x, C.c_float), ptr(out, C.c_float))
        return out

    def nearest_rvq(self, x, vectors):
        return int(self._f("nearest_rvq")(ptr(_f32(x), C.c_float), ptr(_f32(vectors), C.c_float)))

    def project_codebook(self, index, codebook, weights, bias):
        out = np.zeros(1024, np.float32)
        self._f("project_codebook")(index, ptr(_f32(codebook), C.c_float), ptr(_f32(weights), C.c_float),
                                    ptr(_f32(bias), C.c_float), ptr(out, C.c_float))
        return out


def model_desc(model):
    """Builds a ModelDesc over the numpy arrays of a tsac_hip.synthetic.Model.
    The returned tuple keeps every array alive while the descriptor is used."""
    g = model.geometry
    geometry = Geometry(g.width, g.heads, g.head_width, g.ffn, g.temporal_layers,
                        g.codebook_layers, g.latent, g.alphabet, g.books, g.channels, g.context,
                        g.attention_scale)
    keep = []
    linears = (Linear * len(model.projections))()
    for i, (values, scales, bias) in enumerate(model.projections):
        values, scales, bias = (np.ascontiguousarray(a) for a in (values, scales, bias))
        keep += [values, scales, bias]
        linears[i] = Linear(ptr(values, C.c_int8), ptr(scales, C.c_float), ptr(bias, C.c_float))
    gains = (u16p * len(model.norm_gain))(*[ptr(np.ascontiguousarray(a), C.c_uint16) for a in model.norm_gain])
    biases = (u16p * len(model.norm_bias))(*[ptr(np.ascontiguousarray(a), C.c_uint16) for a in model.norm_bias])
    keep += [model.norm_gain, model.norm_bias, linears, gains, biases]
    desc = ModelDesc(geometry, linears, gains, biases, ptr(model.positions, C.c_uint16),
                     ptr(model.rotations, C.c_uint16), ptr(model.embeddings, C.c_uint16))
    return desc, keep


def header(frames, batch, groups, codebooks, model_channels=2, method=1) -> Header:
    return Header(method, groups, model_channels, codebooks, frames, batch)


class Oracle(_Kernels, _DspKernels):
    def __init__(self):
        lib = _load(ORACLE_PATH)
        super().__init__(lib, "orc_")
        self._declare_dsp()
        lib.orc_dac_sine_squared.argtypes = [C.c_float]
        lib.orc_dac_sine_squared.restype = C.c_float
        lib.orc_expand_bf8.argtypes = [i8p, u16p, sz, sz, sz, f32p]
        lib.orc_dac_conv_config.argtypes = [C.c_int, C.c_uint, C.c_uint, C.POINTER(OrcConv)]
        lib.orc_dac_apply.argtypes = [C.POINTER(OrcDac), f32p, sz, f32p, C.POINTER(sz), C.c_uint]
        lib.orc_rvq_encode.argtypes = [C.POINTER(OrcRvq), f32p, sz, u16p]
        lib.orc_rvq_decode.argtypes = [C.POINTER(OrcRvq), u16p, sz, f32p]
        lib.orc_analyze_audio.argtypes = [C.POINTER(OrcDac), C.POINTER(OrcRvq), f32p, sz, sz, sz, C.c_uint, u16p]
        lib.orc_synthesize_audio.argtypes = [C.POINTER(OrcDac), C.POINTER(OrcRvq), u16p, sz, sz, sz, C.c_uint, f32p]
        lib.orc_pcm16.argtypes = [C.c_float]
        lib.orc_pcm16.restype = C.c_int16
        lib.orc_attention.argtypes = [u16p, u16p, u16p, sz, sz, sz, C.c_float, C.c_int, u16p]
        lib.orc_gelu_batch.argtypes = [u16p, sz, u16p]
        lib.orc_range_roundtrip_encode.argtypes = [f32p, u16p, sz, sz, u8p, sz, C.POINTER(sz)]
        lib.orc_range_roundtrip_decode.argtypes = [f32p, sz, sz, u8p, sz, u16p]
        lib.orc_parse_header.argtypes = [u8p, sz, C.POINTER(Header), C.POINTER(sz), C.POINTER(sz),
                                         C.POINTER(C.c_uint32)]
        lib.orc_model_create.argtypes = [C.POINTER(ModelDesc), C.POINTER(C.c_void_p)]
        lib.orc_model_destroy.argtypes = [C.c_void_p]
        lib.orc_backend_reset.argtypes = [C.c_void_p, C.POINTER(Header), sz]
        lib.orc_backend_reset_temporal.argtypes = [C.c_void_p, sz]
        lib.orc_backend_temporal_step.argtypes = [C.c_void_p, sz, sz, u16p, sz, C.c_int]
        lib.orc_backend_reset_codebook.argtypes = [C.c_void_p, sz]
        lib.orc_backend_codebook_step.argtypes = [C.c_void_p, sz, sz, u16p, sz, u16p]
        lib.orc_pack_normal.argtypes = [C.c_void_p, C.POINTER(Header), u16p, sz, C.c_uint,
                                        C.POINTER(u8p), C.POINTER(sz)]
        lib.orc_unpack_normal.argtypes = [C.c_void_p, u8p, sz, C.c_uint, C.POINTER(u16p),
                                          C.POINTER(sz)]
        lib.orc_pack_normal_observed.argtypes = [C.c_void_p, C.POINTER(Header), u16p, sz, C.c_uint,
                                                 C.POINTER(u8p), C.POINTER(sz), C.POINTER(C.c_uint32),
                                                 C.POINTER(C.c_uint64)]
        lib.orc_distributions_prefix.argtypes = [C.c_void_p, C.POINTER(Header), u16p, sz, C.c_uint,
                                                 sz, u16p]
        lib.orc_free.argtypes = [C.c_void_p]

    def gelu_batch(self, x):
        x = np.ascontiguousarray(x, np.uint16)
        out = np.empty_like(x)
        self.lib.orc_gelu_batch(ptr(x, C.c_uint16), x.size, ptr(out, C.c_uint16))
        return out

    def attention(self, q, k, v, heads, head_width, scale, prefill=False):
        q, k, v = (np.ascontiguousarray(a, np.uint16) for a in (q, k, v))
        width = heads * head_width
        out = np.zeros(width, np.uint16)
        self._check(self.lib.orc_attention(ptr(q, C.c_uint16), ptr(k, C.c_uint16), ptr(v, C.c_uint16),
                                           k.size // width, heads, head_width, scale, int(prefill),
                                           ptr(out, C.c_uint16)))
        return out

    def range_encode(self, probabilities, symbols):
        p = np.ascontiguousarray(probabilities, np.float32)
        s = np.ascontiguousarray(symbols, np.uint16)
        out = np.zeros(64 + 4 * p.size, np.uint8)
        n = sz()
        self._check(self.lib.orc_range_roundtrip_encode(ptr(p, C.c_float), ptr(s, C.c_uint16), s.size,
                                                        p.shape[-1], ptr(out, C.c_uint8), out.size,
                                                        C.byref(n)))
        return out[:n.value].tobytes()

    def range_decode(self, probabilities, data: bytes):
        p = np.ascontiguousarray(probabilities, np.float32)
        count = p.shape[0]
        b = np.frombuffer(data, np.uint8).copy() if data else np.zeros(1, np.uint8)
        out = np.zeros(count, np.uint16)
        self._check(self.lib.orc_range_roundtrip_decode(ptr(p, C.c_float), count, p.shape[-1],
                                                        ptr(b, C.c_uint8), len(data),
                                                        ptr(out, C.c_uint16)))
        return out

    def parse_header(self, data: bytes):
        b = np.frombuffer(data, np.uint8).copy() if data else np.zeros(1, np.uint8)
        h, off, n, crc = Header(), sz(), sz(), C.c_uint32()
        self._check(self.lib.orc_parse_header(ptr(b, C.c_uint8), len(data), C.byref(h), C.byref(off),
                                              C.byref(n), C.byref(crc)))
        return h, off.value, n.value, crc.value

    def model(self, model) -> "OracleModel":
        return OracleModel(self, model)

    def dac_sine_squared(self, phase: float) -> float:
        return self.lib.orc_dac_sine_squared(phase)

    def dac_conv_config(self, synthesis: bool, channels: int, index: int) -> OrcConv:
        c = OrcConv()
        self._check(self.lib.orc_dac_conv_config(int(synthesis), channels, index, C.byref(c)))
        return c

    def expand_bf8(self, values, scales, dims):
        rows, cols, outer = dims
        values = np.ascontiguousarray(values, np.int8)
        scales = np.ascontiguousarray(scales, np.uint16)
        out = np.zeros(rows * cols * outer, np.float32)
        self._check(self.lib.orc_expand_bf8(ptr(values, C.c_int8), ptr(scales, C.c_uint16), rows, cols, outer,
                                            ptr(out, C.c_float)))
        return out

    def prepare_convolution(self, conv):
        """Convolution::from_weights preparation (src/common/dsp.tpp:117-155):
        expand the source encoding, then fold the DAC weight norm per stored column."""
        rows, cols, outer = conv.dims
        values = self.expand_bf8(conv.values, conv.scales, conv.dims) if conv.bf8 else _f32(conv.values)
        return self.fold_dac_weight_norm(values, conv.gain, rows * cols)

    def dac_model(self, model, books=None) -> "OracleDacModel":
        return OracleDacModel(self, model, books)

    def pcm16(self, x: float) -> int:
        return int(self.lib.orc_pcm16(x))


class OracleModel:
    def __init__(self, oracle: Oracle, model):
        self.oracle, self.lib = oracle, oracle.lib
        self.model = model
        self.desc, self._keep = model_desc(model)
        self.handle = C.c_void_p()
        oracle._check(self.lib.orc_model_create(C.byref(self.desc), C.byref(self.handle)))

    def __del__(self):
        if getattr(self, "handle", None):
            self.lib.orc_model_destroy(self.handle)
            self.handle = None

    def pack_normal(self, h: Header, tokens, threads=1) -> bytes:
        t = np.ascontiguousarray(tokens, np.uint16)
        out, n = u8p(), sz()
        self.oracle._check(self.lib.orc_pack_normal(self.handle, C.byref(h), ptr(t, C.c_uint16), t.size,
                                                    threads, C.byref(out), C.byref(n)))
        data = C.string_at(out, n.value)
        self.lib.orc_free(out)
        return data

    def pack_normal_observed(self, h: Header, tokens, threads=1):
        """pack_normal plus what an EntropyObserver sees: per symbol in stream
        order, after_symbol's bit count and the position (frame, group,
        codebook, lane, step, token_offset)."""
        t = np.ascontiguousarray(tokens, np.uint16)
        out, n = u8p(), sz()
        bits = np.zeros(max(t.size, 1), np.uint32)
        positions = np.zeros((max(t.size, 1), 6), np.uint64)
        self.oracle._check(self.lib.orc_pack_normal_observed(
            self.handle, C.byref(h), ptr(t, C.c_uint16), t.size, threads, C.byref(out), C.byref(n),
            ptr(bits, C.c_uint32), ptr(positions, C.c_uint64)))
        data = C.string_at(out, n.value)
        self.lib.orc_free(out)
        return data, bits[:t.size], positions[:t.size]

    def unpack_normal(self, data: bytes, threads=1) -> np.ndarray:
        b = np.frombuffer(data, np.uint8).copy()
        out, n = u16p(), sz()
        self.oracle._check(self.lib.orc_unpack_normal(self.handle, ptr(b, C.c_uint8), len(data),
                                                      threads, C.byref(out), C.byref(n)))
        tokens = np.ctypeslib.as_array(out, shape=(n.value,)).copy() if n.value else np.zeros(0, np.uint16)
        self.lib.orc_free(out)
        return tokens

    def distributions(self, h: Header, tokens, threads=1, max_symbols=None) -> np.ndarray:
        t = np.ascontiguousarray(tokens, np.uint16)
        out = np.zeros((t.size, self.model.geometry.alphabet), np.uint16)
        limit = C.c_size_t(-1).value if max_symbols is None else max_symbols
        self.oracle._check(self.lib.orc_distributions_prefix(self.handle, C.byref(h), ptr(t, C.c_uint16),
                                                             t.size, threads, limit, ptr(out, C.c_uint16)))
        return out

    # TransformerBackend surface
    def reset(self, h: Header, lanes: int):
        self.oracle._check(self.lib.orc_backend_reset(self.handle, C.byref(h), lanes))

    def reset_temporal(self, lane):
        self.oracle._check(self.lib.orc_backend_reset_temporal(self.handle, lane))

    def temporal_step(self, lane, position, feedback, replay=False):
        f = np.ascontiguousarray(feedback, np.uint16)
        self.oracle._check(self.lib.orc_backend_temporal_step(self.handle, lane, position,
                                                              ptr(f, C.c_uint16), f.size, int(replay)))

    def reset_codebook(self, lane):
        self.oracle._check(self.lib.orc_backend_reset_codebook(self.handle, lane))

    def codebook_step(self, lane, book, prefix):
        p = np.ascontiguousarray(prefix, np.uint16) if len(prefix) else np.zeros(1, np.uint16)
        out = np.zeros(self.model.geometry.alphabet, np.uint16)
        self.oracle._check(self.lib.orc_backend_codebook_step(self.handle, lane, book, ptr(p, C.c_uint16),
                                                              len(prefix), ptr(out, C.c_uint16)))
        return out


class Reference(_Kernels, _DspKernels):
    """The reference's own scalar sources (compiled here from the reference tree)."""

    def __init__(self):
        lib = _load(REF_PATH)
        super().__init__(lib, "ref_")
        self._declare_dsp()
        lib.ref_gelu_table.argtypes = [u16p, sz]
        lib.ref_attention.argtypes = [u16p, u16p, u16p, sz, sz, sz, C.c_float, C.c_int, u16p]
        lib.ref_range_encode.argtypes = [f32p, u16p, sz, sz, u8p, sz, C.POINTER(sz)]
        lib.ref_source_parse.argtypes = [u8p, sz, C.c_uint64, C.c_uint64, C.POINTER(sz)]
        lib.ref_source_dequantize.argtypes = [u8p, sz, C.c_char_p, f32p, sz]
        lib.ref_source_configs.argtypes = [u8p, sz] + [C.POINTER(C.c_uint)] * 3
        lib.ref_pcm16_input.argtypes = [u8p, sz, C.c_uint, f32p, sz, C.POINTER(sz)]
        lib.ref_wave_input.argtypes = [u8p, sz, f32p, sz, C.POINTER(sz), C.POINTER(C.c_uint)]
        lib.ref_pcm16_wave.argtypes = [f32p, sz, C.c_uint, C.c_uint64, u8p, sz, C.POINTER(sz)]
        lib.ref_parse_cli.argtypes = [sz, C.POINTER(C.c_char_p), C.POINTER(C.c_longlong)]

    @staticmethod
    def available() -> bool:
        return REF_PATH.exists()

    # SourceModel (src/weights/source_model.cpp) on an original-format file.
    def source_parse(self, data: bytes, file_bytes: int = 0, metadata_bytes: int = 0):
        """The tensor count, or None when the reference's parser rejects the file."""
        b = np.frombuffer(data, np.uint8).copy() if data else np.zeros(1, np.uint8)
        n = sz()
        status = self.lib.ref_source_parse(ptr(b, C.c_uint8), len(data), file_bytes, metadata_bytes, C.byref(n))
        return None if status else n.value

    def source_dequantize(self, data: bytes, name: str, count: int) -> np.ndarray:
        b = np.frombuffer(data, np.uint8).copy()
        out = np.zeros(max(count, 1), np.float32)
        self._check(self.lib.ref_source_dequantize(ptr(b, C.c_uint8), len(data), name.encode(), ptr(out, C.c_float),
                                                   out.size))
        return out[:count]

    # The command-line codec's audio files and options (src/audio.cpp, src/cli.cpp).
    def pcm16_input(self, data: bytes, channels: int):
        """Float PCM [frames][channels], or None when the reference rejects it."""
        b = np.frombuffer(data, np.uint8).copy() if data else np.zeros(1, np.uint8)
        out = np.zeros(max(1, (len(data) // max(2 * channels, 1) + 512) * max(channels, 1)), np.float32)
        frames = sz()
        if self.lib.ref_pcm16_input(ptr(b, C.c_uint8), len(data), channels, ptr(out, C.c_float), out.size,
                                    C.byref(frames)):
            return None
        return out[:frames.value * channels].reshape(frames.value, channels)

    def wave_input(self, data: bytes):
        b = np.frombuffer(data, np.uint8).copy() if data else np.zeros(1, np.uint8)
        out = np.zeros(len(data) + 512 * 8, np.float32)
        frames, channels = sz(), C.c_uint()
        if self.lib.ref_wave_input(ptr(b, C.c_uint8), len(data), ptr(out, C.c_float), out.size, C.byref(frames),
                                   C.byref(channels)):
            return None
        return out[:frames.value * channels.value].reshape(frames.value, channels.value)

    def pcm16_wave(self, samples, pcm_bytes: int = 0):
        pcm = np.ascontiguousarray(samples, np.float32)
        frames, channels = pcm.shape
        out = np.zeros(44 + 2 * pcm.size, np.uint8)
        n = sz()
        if self.lib.ref_pcm16_wave(ptr(pcm, C.c_float), frames, channels, pcm_bytes, ptr(out, C.c_uint8), out.size,
                                   C.byref(n)):
            return None
        return out[:n.value].tobytes()

    def parse_cli(self, arguments: list):
        """None when the reference rejects the arguments, else its options with
        input/output as the indices of those arguments."""
        encoded = [a.encode() for a in arguments]
        argv = (C.c_char_p * max(len(encoded), 1))(*encoded)
        fields = (C.c_longlong * 12)()
        if self.lib.ref_parse_cli(len(encoded), argv, fields):
            return None
        names = ("command", "threads", "quality", "channels", "batch", "verbose", "fast", "separate", "help",
                 "metal", "input", "output")
        return dict(zip(names, list(fields)))

    def source_configs(self, data: bytes) -> tuple:
        """(channels, codebooks) of dac_config and codebooks of transformer_config,
        each 0 where the reference rejects the file for that role."""
        b = np.frombuffer(data, np.uint8).copy()
        c, d, t = C.c_uint(), C.c_uint(), C.c_uint()
        self._check(self.lib.ref_source_configs(ptr(b, C.c_uint8), len(data), C.byref(c), C.byref(d), C.byref(t)))
        return c.value, d.value, t.value

    def gelu_table(self, values):
        v = np.ascontiguousarray(values, np.uint16).copy()
        self.lib.ref_gelu_table(ptr(v, C.c_uint16), v.size)
        return v

    def attention(self, q, k, v, heads, head_width, scale, prefill=False):
        q, k, v = (np.ascontiguousarray(a, np.uint16) for a in (q, k, v))
        width = heads * head_width
        out = np.zeros(width, np.uint16)
        self._check(self.lib.ref_attention(ptr(q, C.c_uint16), ptr(k, C.c_uint16), ptr(v, C.c_uint16),
                                           k.size // width, heads, head_width, scale, int(prefill),
                                           ptr(out, C.c_uint16)))
        return out

    def range_encode(self, probabilities, symbols):
        p = np.ascontiguousarray(probabilities, np.float32)
        s = np.ascontiguousarray(symbols, np.uint16)
        out = np.zeros(64 + 4 * p.size, np.uint8)
        n = sz()
        self._check(self.lib.ref_range_encode(ptr(p, C.c_float), ptr(s, C.c_uint16), s.size,
                                              p.shape[-1], ptr(out, C.c_uint8), out.size, C.byref(n)))
        return out[:n.value].tobytes()


def host_threads() -> int:
    return len(os.sched_getaffinity(0))


# ---------------------------------------------------------------- DAC and RVQ models


class OracleDacModel:
    """A tsac_hip.synthetic.DacModel prepared the way the reference's runtime
    prepares it (BF8 expansion and DAC weight-norm folding, RVQ search vectors
    and folded projections), bound to the oracle's DAC graphs and quantizer."""

    def __init__(self, oracle: "Oracle", model, books=None):
        self.oracle, self.lib, self.model = oracle, oracle.lib, model
        self.books = books or len(model.codebook)
        self._keep = []
        self.graphs = {}
        for synthesis in (False, True):
            convs = model.synthesis if synthesis else model.analysis
            alphas = model.synthesis_alpha if synthesis else model.analysis_alpha
            desc = OrcDac()
            desc.synthesis = int(synthesis)
            desc.channels = model.channels
            prepared = []
            for i, conv in enumerate(convs):
                w = oracle.prepare_convolution(conv)
                b = _f32(conv.bias)
                prepared.append(w)
                self._keep += [w, b]
                desc.weights[i] = ptr(w, C.c_float)
                desc.bias[i] = ptr(b, C.c_float)
            for i, a in enumerate(alphas):
                a = _f32(a)
                self._keep.append(a)
                desc.alpha[i] = ptr(a, C.c_float)
            self.graphs[synthesis] = (desc, prepared)
        q = OrcRvq()
        q.books = self.books
        self.rvq_tensors = []
        for book in range(self.books):
            codebook = _f32(model.codebook[book])
            search = np.stack([oracle.normalize_search(row) for row in codebook])
            input_weights = oracle.fold_dac_weight_norm(model.in_v[book], model.in_g[book], 1024)
            output_weights = oracle.fold_dac_weight_norm(model.out_v[book], model.out_g[book], 8)
            tensors = (codebook, _f32(search), input_weights, _f32(model.in_bias[book]), output_weights,
                       _f32(model.out_bias[book]))
            self.rvq_tensors.append(tensors)
            self._keep += list(tensors)
            for name, t in zip(("codebook", "search", "input_weights", "input_bias", "output_weights",
                                "output_bias"), tensors):
                getattr(q, name)[book] = ptr(t, C.c_float)
        self.rvq = q

    def apply(self, synthesis: bool, x, frames, threads=8):
        """One DAC graph on one group: analysis PCM [frames][channels] -> latent
        [frames/512][1024]; synthesis latent [frames][1024] -> [frames*512][channels]."""
        desc = self.graphs[synthesis][0]
        x = _f32(x)
        out_frames = frames * 512 if synthesis else frames // 512
        out = np.zeros(out_frames * (self.model.channels if synthesis else 1024), np.float32)
        produced = sz()
        self.oracle._check(self.lib.orc_dac_apply(C.byref(desc), ptr(x, C.c_float), frames, ptr(out, C.c_float),
                                                  C.byref(produced), threads))
        assert produced.value == out_frames
        return out

    def rvq_encode(self, latent, frames):
        latent = _f32(latent)
        tokens = np.zeros(frames * self.books, np.uint16)
        self.oracle._check(self.lib.orc_rvq_encode(C.byref(self.rvq), ptr(latent, C.c_float), frames,
                                                   ptr(tokens, C.c_uint16)))
        return tokens

    def rvq_decode(self, tokens, frames):
        tokens = np.ascontiguousarray(tokens, np.uint16)
        latent = np.zeros(frames * 1024, np.float32)
        self.oracle._check(self.lib.orc_rvq_decode(C.byref(self.rvq), ptr(tokens, C.c_uint16), frames,
                                                   ptr(latent, C.c_float)))
        return latent

    def analyze_audio(self, pcm, frames, groups=1, chunk=400, threads=8):
        """Padded PCM [groups][frames*512][channels] -> tokens [frame][group][book]."""
        pcm = _f32(pcm)
        tokens = np.zeros(frames * groups * self.books, np.uint16)
        self.oracle._check(self.lib.orc_analyze_audio(C.byref(self.graphs[False][0]), C.byref(self.rvq),
                                                      ptr(pcm, C.c_float), frames, groups, chunk, threads,
                                                      ptr(tokens, C.c_uint16)))
        return tokens

    def synthesize_audio(self, tokens, frames, groups=1, chunk=400, threads=8):
        """Tokens -> float PCM [frames*512][groups*channels]."""
        tokens = np.ascontiguousarray(tokens, np.uint16)
        pcm = np.zeros(frames * 512 * groups * self.model.channels, np.float32)
        self.oracle._check(self.lib.orc_synthesize_audio(C.byref(self.graphs[True][0]), C.byref(self.rvq),
                                                         ptr(tokens, C.c_uint16), frames, groups, chunk, threads,
                                                         ptr(pcm, C.c_float)))
        return pcm


# ---------------------------------------------------------------- the reference's composition

COMPOSITION_PATH = HERE / "_ref" / "libtsacmodel.so"
PACKED_PATH = HERE / "_ref" / "gen" / "pack"


class ReferenceComposition:
    """The reference's own CpuTransformer<scalar::Kernels> + TransformerPredictor +
    pack_normal/unpack_normal, DacAnalysis, DacSynthesis, RvqEncoder and
    RvqDecoder (oracle/ref_model.cpp), reading the seeded models of
    seeded_models.py from the files the reference's packer wrote."""

    def __init__(self):
        self.lib = lib = _load(COMPOSITION_PATH)
        lib.refm_last_error.restype = C.c_char_p
        vp, hp, u, cp, szp = C.c_void_p, C.POINTER(Header), C.c_uint, C.c_char_p, C.POINTER(sz)
        lib.refm_transformer_open.argtypes = [cp, u, u, sz, C.POINTER(vp)]
        lib.refm_transformer_close.argtypes = [vp]
        lib.refm_transformer_projection.argtypes = [vp, u, i8p, f32p, f32p, szp, szp]
        lib.refm_transformer_norm.argtypes = [vp, u, u16p, u16p]
        lib.refm_transformer_constants.argtypes = [vp, u16p, u16p, u16p]
        lib.refm_pack_normal.argtypes = [vp, hp, u16p, sz, u, u8p, sz, szp]
        lib.refm_pack_normal_observed.argtypes = [vp, hp, u16p, sz, u8p, sz, szp, C.POINTER(C.c_uint32),
                                                  C.POINTER(C.c_uint64)]
        lib.refm_unpack_normal.argtypes = [vp, u8p, sz, u, u16p, sz, szp]
        lib.refm_distributions.argtypes = [vp, hp, u16p, sz, u, u16p]
        lib.refm_dac_open.argtypes = [cp, u, u, C.POINTER(vp)]
        lib.refm_dac_close.argtypes = [vp]
        lib.refm_dac_analysis.argtypes = [vp, f32p, sz, sz, sz, f32p]
        lib.refm_dac_synthesis.argtypes = [vp, f32p, sz, sz, sz, f32p]
        lib.refm_rvq_encode.argtypes = [vp, hp, f32p, u16p]
        lib.refm_rvq_decode.argtypes = [vp, hp, u16p, f32p]
        lib.refm_dac_convolution.argtypes = [vp, C.c_int, u, u8p, szp, szp, f32p, szp, f32p, szp]
        lib.refm_dac_activation.argtypes = [vp, C.c_int, u, f32p, szp]
        lib.refm_rvq_tensors.argtypes = [vp, u] + [f32p] * 6
        self.directory = str(PACKED_PATH).encode()

    @staticmethod
    def available() -> bool:
        return COMPOSITION_PATH.exists() and (PACKED_PATH / "adapter_offsets.hpp").exists()

    def _check(self, status):
        if status:
            raise OracleError(self.lib.refm_last_error().decode())

    def transformer(self, channels: int, books: int, cache_bytes: int = 0) -> "ReferenceTransformer":
        return ReferenceTransformer(self, channels, books, cache_bytes)

    def dac(self, channels: int, books: int) -> "ReferenceDac":
        return ReferenceDac(self, channels, books)


class _Handle:
    def __init__(self, owner: ReferenceComposition, close):
        self.owner, self.lib, self.handle = owner, owner.lib, C.c_void_p()
        self._close = close

    def close(self):
        if self.handle:
            self._close(self.handle)
            self.handle = C.c_void_p()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class ReferenceTransformer(_Handle):
    def __init__(self, owner, channels, books, cache_bytes):
        super().__init__(owner, owner.lib.refm_transformer_close)
        self.books = books
        owner._check(self.lib.refm_transformer_open(owner.directory, channels, books, sz(cache_bytes),
                                                    C.byref(self.handle)))

    def projection(self, index: int):
        k, n = sz(), sz()
        self.owner._check(self.lib.refm_transformer_projection(self.handle, index, None, None, None,
                                                               C.byref(k), C.byref(n)))
        values = np.zeros((n.value, k.value), np.int8)
        scales = np.zeros((k.value // 256, n.value), np.float32)
        bias = np.zeros(n.value, np.float32)
        self.owner._check(self.lib.refm_transformer_projection(
            self.handle, index, ptr(values, C.c_int8), ptr(scales, C.c_float), ptr(bias, C.c_float),
            C.byref(k), C.byref(n)))
        return values, scales, bias

    def norm(self, index: int):
        gain, bias = np.zeros(512, np.uint16), np.zeros(512, np.uint16)
        self.owner._check(self.lib.refm_transformer_norm(self.handle, index, ptr(gain, C.c_uint16),
                                                         ptr(bias, C.c_uint16)))
        return gain, bias

    def constants(self):
        positions = np.zeros((self.books, 512), np.uint16)
        rotations = np.zeros((1024, 128), np.uint16)
        embeddings = np.zeros((self.books, 1024, 1024), np.uint16)
        self.owner._check(self.lib.refm_transformer_constants(self.handle, ptr(positions, C.c_uint16),
                                                              ptr(rotations, C.c_uint16),
                                                              ptr(embeddings, C.c_uint16)))
        return positions, rotations, embeddings

    def pack_normal(self, h: Header, tokens, threads: int = 1) -> bytes:
        t = np.ascontiguousarray(tokens, np.uint16)
        out = np.zeros(64 + 24 * t.size, np.uint8)  # up to 10 15-bit decisions per symbol
        n = sz()
        self.owner._check(self.lib.refm_pack_normal(self.handle, C.byref(h), ptr(t, C.c_uint16), t.size, threads,
                                                    ptr(out, C.c_uint8), out.size, C.byref(n)))
        return out[:n.value].tobytes()

    def pack_normal_observed(self, h: Header, tokens):
        """pack_normal with an EntropyObserver recording, per symbol in the order it
        sees them, before_symbol's position and after_symbol's bit count."""
        t = np.ascontiguousarray(tokens, np.uint16)
        out = np.zeros(64 + 24 * t.size, np.uint8)
        n = sz()
        bits = np.zeros(max(t.size, 1), np.uint32)
        positions = np.zeros((max(t.size, 1), 6), np.uint64)
        self.owner._check(self.lib.refm_pack_normal_observed(
            self.handle, C.byref(h), ptr(t, C.c_uint16), t.size, ptr(out, C.c_uint8), out.size, C.byref(n),
            ptr(bits, C.c_uint32), ptr(positions, C.c_uint64)))
        return out[:n.value].tobytes(), bits[:t.size], positions[:t.size]

    def unpack_normal(self, data: bytes, capacity: int, threads: int = 1) -> np.ndarray:
        b = np.frombuffer(data, np.uint8).copy()
        out = np.zeros(max(capacity, 1), np.uint16)
        n = sz()
        self.owner._check(self.lib.refm_unpack_normal(self.handle, ptr(b, C.c_uint8), len(data), threads,
                                                      ptr(out, C.c_uint16), out.size, C.byref(n)))
        return out[:n.value]

    def distributions(self, h: Header, tokens, threads: int = 1) -> np.ndarray:
        t = np.ascontiguousarray(tokens, np.uint16)
        out = np.zeros((t.size, 1024), np.uint16)
        self.owner._check(self.lib.refm_distributions(self.handle, C.byref(h), ptr(t, C.c_uint16), t.size,
                                                      threads, ptr(out, C.c_uint16)))
        return out


class ReferenceDac(_Handle):
    def __init__(self, owner, channels, books):
        super().__init__(owner, owner.lib.refm_dac_close)
        self.channels, self.books = channels, books
        owner._check(self.lib.refm_dac_open(owner.directory, channels, books, C.byref(self.handle)))

    def analysis(self, pcm, samples: int, groups: int = 1, chunk: int = 0) -> np.ndarray:
        """PCM [groups][samples][channels] -> latent [groups][samples/512][1024]."""
        x = _f32(pcm)
        assert x.size == groups * samples * self.channels
        out = np.zeros(groups * (samples // 512) * 1024, np.float32)
        self.owner._check(self.lib.refm_dac_analysis(self.handle, ptr(x, C.c_float), samples, groups, chunk,
                                                     ptr(out, C.c_float)))
        return out

    def synthesis(self, latent, frames: int, groups: int = 1, chunk: int = 0) -> np.ndarray:
        """Latent [groups][frames][1024] -> PCM [groups][frames*512][channels]."""
        x = _f32(latent)
        assert x.size == groups * frames * 1024
        out = np.zeros(groups * frames * 512 * self.channels, np.float32)
        self.owner._check(self.lib.refm_dac_synthesis(self.handle, ptr(x, C.c_float), frames, groups, chunk,
                                                      ptr(out, C.c_float)))
        return out

    def rvq_encode(self, latent, frames: int, groups: int = 1) -> np.ndarray:
        """Latent [groups][frames][1024] -> tokens [frame][group][book]."""
        x = _f32(latent)
        h = header(frames, 1, groups, self.books, model_channels=self.channels)
        out = np.zeros(frames * groups * self.books, np.uint16)
        self.owner._check(self.lib.refm_rvq_encode(self.handle, C.byref(h), ptr(x, C.c_float),
                                                   ptr(out, C.c_uint16)))
        return out

    def rvq_decode(self, tokens, frames: int, groups: int = 1) -> np.ndarray:
        """Tokens [frame][group][book] -> latent [groups][frames][1024]."""
        t = np.ascontiguousarray(tokens, np.uint16)
        h = header(frames, 1, groups, self.books, model_channels=self.channels)
        out = np.zeros(groups * frames * 1024, np.float32)
        self.owner._check(self.lib.refm_rvq_decode(self.handle, C.byref(h), ptr(t, C.c_uint16),
                                                   ptr(out, C.c_float)))
        return out

    def convolution(self, synthesis: bool, index: int):
        """(payload bytes, data-plane bytes, gains, biases) as the DAC model adapter reads them."""
        pb, dp, ng, nb = sz(), sz(), sz(), sz()
        args = (self.handle, int(synthesis), index)
        self.owner._check(self.lib.refm_dac_convolution(*args, None, C.byref(pb), C.byref(dp), None,
                                                        C.byref(ng), None, C.byref(nb)))
        payload = np.zeros(pb.value, np.uint8)
        gains, biases = np.zeros(ng.value, np.float32), np.zeros(nb.value, np.float32)
        self.owner._check(self.lib.refm_dac_convolution(*args, ptr(payload, C.c_uint8), C.byref(pb), C.byref(dp),
                                                        ptr(gains, C.c_float), C.byref(ng),
                                                        ptr(biases, C.c_float), C.byref(nb)))
        return payload, dp.value, gains, biases

    def activation(self, synthesis: bool, index: int) -> np.ndarray:
        n = sz()
        self.owner._check(self.lib.refm_dac_activation(self.handle, int(synthesis), index, None, C.byref(n)))
        out = np.zeros(n.value, np.float32)
        self.owner._check(self.lib.refm_dac_activation(self.handle, int(synthesis), index, ptr(out, C.c_float),
                                                       C.byref(n)))
        return out

    def rvq_tensors(self, book: int):
        """codebook [1024][8], search [1024][8], input projection [1024 in][8 out]
        (input-major), input bias [8], output projection [8][1024], output bias [1024]."""
        arrays = (np.zeros((1024, 8), np.float32), np.zeros((1024, 8), np.float32), np.zeros((1024, 8), np.float32),
                  np.zeros(8, np.float32), np.zeros((8, 1024), np.float32), np.zeros(1024, np.float32))
        self.owner._check(self.lib.refm_rvq_tensors(self.handle, book, *(ptr(a, C.c_float) for a in arrays)))
        return arrays
