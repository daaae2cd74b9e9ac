"""ctypes bindings of libtsac_hip.so (include/tsac_hip.h).

The library is the product: every call here runs the hand-written gfx950
kernels. Loading fails loudly when the library has not been built; there is no
fallback path.
"""
from __future__ import annotations

import ctypes as C
import pathlib

import numpy as np

PACKAGE = pathlib.Path(__file__).resolve().parent.parent
LIBRARY = PACKAGE / "libtsac_hip.so"

u8p = C.POINTER(C.c_uint8)
u16p = C.POINTER(C.c_uint16)
i8p = C.POINTER(C.c_int8)
f32p = C.POINTER(C.c_float)
i32p = C.POINTER(C.c_int)
sz = C.c_size_t
vp = C.c_void_p

#: Exported entry points declared by include/tsac_hip.h.
EXPORTS = (
    "tsac_hip_last_error", "tsac_hip_model_create", "tsac_hip_model_destroy",
    "tsac_hip_session_create", "tsac_hip_session_destroy", "tsac_hip_session_clear",
    "tsac_hip_encode", "tsac_hip_decode", "tsac_hip_free", "tsac_hip_distributions",
    "tsac_hip_session_timing", "tsac_hip_linear_create", "tsac_hip_linear_destroy",
    "tsac_hip_linear_apply", "tsac_hip_linear_apply_quantized", "tsac_hip_bf8l",
    "tsac_hip_layer_norm", "tsac_hip_softmax", "tsac_hip_gelu", "tsac_hip_rotary", "tsac_hip_add",
    "tsac_hip_attention", "tsac_hip_attention_causal", "tsac_hip_bf8l_tiles", "tsac_hip_tile_rows",
    "tsac_hip_probe_read", "tsac_hip_probe_mfma", "tsac_hip_encode_observed", "tsac_hip_decode_observed",
    "tsac_hip_linear_apply_static", "tsac_hip_dac_create", "tsac_hip_dac_destroy", "tsac_hip_prepare_rvq",
    "tsac_hip_dac_analyze", "tsac_hip_dac_synthesize", "tsac_hip_audio_encode", "tsac_hip_audio_decode",
    "tsac_hip_dac_apply", "tsac_hip_source_load", "tsac_hip_source_parse", "tsac_hip_source_destroy",
    "tsac_hip_source_tensor_count", "tsac_hip_source_tensor_info", "tsac_hip_source_metadata",
    "tsac_hip_source_dequantize", "tsac_hip_source_dac_config", "tsac_hip_source_transformer_config",
    "tsac_hip_prepare_transformer", "tsac_hip_prepared_transformer_destroy", "tsac_hip_prepare_dac",
    "tsac_hip_prepared_dac_destroy", "tsac_hip_model_create_from_source", "tsac_hip_dac_create_from_source",
    "tsac_hip_pcm16_read", "tsac_hip_wave_read", "tsac_hip_wave_write", "tsac_hip_audio_header",
    "tsac_hip_parse_header", "tsac_hip_cli_parse", "tsac_hip_cli_help",
)

PATH_AUTO, PATH_GEMV, PATH_GEMM, PATH_GEMM_TILES, PATH_SMALL = 0, 1, 2, 3, 4
PASS_ENCODE, PASS_DECODE = 0, 1


class HipError(RuntimeError):
    pass


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


class Limits(C.Structure):
    _fields_ = [(name, C.c_uint64) for name in (
        "file_bytes", "symbols", "pcm_bytes", "cache_bytes", "tensor_elements")]


class Header(C.Structure):
    _fields_ = [("method", C.c_uint8), ("groups", C.c_uint8), ("model_channels", C.c_uint8),
                ("codebooks", C.c_uint8), ("frames", C.c_uint64), ("batch", C.c_uint16)]


class Position(C.Structure):
    _fields_ = [(name, C.c_uint64) for name in ("frame", "group", "codebook", "lane", "step", "token_offset")]


BEFORE_SYMBOL = C.CFUNCTYPE(C.c_int, vp, C.POINTER(Position))
AFTER_SYMBOL = C.CFUNCTYPE(C.c_int, vp, C.POINTER(Position), C.c_uint64)


class Observer(C.Structure):
    _fields_ = [("context", vp), ("before_symbol", BEFORE_SYMBOL), ("after_symbol", AFTER_SYMBOL)]


class DacConvolution(C.Structure):
    _fields_ = [("dims", C.c_uint32 * 3), ("values", f32p), ("quantized", i8p), ("scales", u16p), ("gain", f32p),
                ("bias", f32p)]


class RvqBook(C.Structure):
    _fields_ = [(n, f32p) for n in ("codebook", "search", "input_weights", "input_bias", "output_weights",
                                    "output_bias")]


class DacDesc(C.Structure):
    _fields_ = [("channels", C.c_uint32), ("books", C.c_uint32), ("analysis", DacConvolution * 30),
                ("analysis_alpha", f32p * 29), ("synthesis", DacConvolution * 30), ("synthesis_alpha", f32p * 29),
                ("rvq", RvqBook * 12)]


class SourceLimits(C.Structure):
    _fields_ = [(name, C.c_uint64) for name in (
        "file_bytes", "tensor_elements", "tensors", "metadata_bytes", "name_bytes")]


class SourceTensorInfo(C.Structure):
    _fields_ = [("name", C.c_char_p), ("storage", C.c_uint32), ("rank", C.c_uint32), ("dims", C.c_uint64 * 8),
                ("elements", C.c_uint64)]


class CliOptions(C.Structure):
    _fields_ = [("command", C.c_char), ("input", C.c_char_p), ("output", C.c_char_p), ("threads", C.c_int32),
                ("quality", C.c_int32), ("channels", C.c_int32), ("batch", C.c_int32), ("verbose", C.c_uint32),
                ("fast", C.c_uint8), ("separate", C.c_uint8), ("help", C.c_uint8), ("metal", C.c_uint8)]


class EncodeOptions(C.Structure):
    _fields_ = [("method", C.c_uint8), ("codebooks", C.c_uint8), ("separate_channels", C.c_uint8),
                ("entropy_batch", C.c_uint16)]


def header(frames, batch, groups, codebooks, model_channels=2, method=1) -> Header:
    return Header(method, groups, model_channels, codebooks, frames, batch)


_lib = None


def library() -> C.CDLL:
    """Loads libtsac_hip.so once; raises if it is missing."""
    global _lib
    if _lib is None:
        if not LIBRARY.exists():
            raise HipError(f"{LIBRARY} is not built: run `make -C {PACKAGE}` "
                           "(or __graft_entry__.build())")
        lib = C.CDLL(str(LIBRARY))
        lib.tsac_hip_last_error.restype = C.c_char_p
        lib.tsac_hip_model_create.argtypes = [C.POINTER(ModelDesc), C.POINTER(Limits), C.POINTER(vp)]
        lib.tsac_hip_model_destroy.argtypes = [vp]
        lib.tsac_hip_session_create.argtypes = [vp, C.POINTER(vp)]
        lib.tsac_hip_session_destroy.argtypes = [vp]
        lib.tsac_hip_session_clear.argtypes = [vp]
        lib.tsac_hip_encode.argtypes = [vp, C.POINTER(Header), u16p, sz, C.POINTER(u8p), C.POINTER(sz)]
        lib.tsac_hip_decode.argtypes = [vp, u8p, sz, C.POINTER(u16p), C.POINTER(sz)]
        lib.tsac_hip_free.argtypes = [vp]
        lib.tsac_hip_dac_create.argtypes = [C.POINTER(DacDesc), C.POINTER(Limits), C.POINTER(vp)]
        lib.tsac_hip_dac_destroy.argtypes = [vp]
        lib.tsac_hip_prepare_rvq.argtypes = [f32p] * 8
        lib.tsac_hip_dac_analyze.argtypes = [vp, vp, f32p, sz, sz, C.c_uint32, u16p]
        lib.tsac_hip_dac_synthesize.argtypes = [vp, vp, u16p, sz, sz, C.c_uint32, f32p]
        lib.tsac_hip_dac_apply.argtypes = [vp, vp, C.c_int, f32p, sz, f32p]
        lib.tsac_hip_audio_encode.argtypes = [vp, vp, f32p, sz, C.c_uint32, C.POINTER(EncodeOptions),
                                              C.POINTER(Observer), C.POINTER(u8p), C.POINTER(sz)]
        lib.tsac_hip_audio_decode.argtypes = [vp, vp, u8p, sz, C.POINTER(Observer), C.POINTER(f32p), C.POINTER(sz),
                                              C.POINTER(C.c_uint32)]
        lib.tsac_hip_encode_observed.argtypes = [vp, C.POINTER(Header), u16p, sz, C.POINTER(Observer),
                                                 C.POINTER(u8p), C.POINTER(sz)]
        lib.tsac_hip_decode_observed.argtypes = [vp, u8p, sz, C.POINTER(Observer), C.POINTER(u16p),
                                                 C.POINTER(sz)]
        lib.tsac_hip_distributions.argtypes = [vp, C.POINTER(Header), u16p, sz, C.c_int, u16p]
        lib.tsac_hip_session_timing.argtypes = [vp, C.POINTER(C.c_double), sz]
        lib.tsac_hip_linear_create.argtypes = [C.POINTER(Linear), sz, sz, C.POINTER(vp)]
        lib.tsac_hip_linear_destroy.argtypes = [vp]
        lib.tsac_hip_linear_apply.argtypes = [vp, vp, sz, vp, C.c_int, vp]
        lib.tsac_hip_linear_apply_static.argtypes = [vp, vp, sz, vp, C.c_int, vp]
        lib.tsac_hip_linear_apply_quantized.argtypes = [vp, vp, vp, sz, vp, vp, C.c_int, vp]
        lib.tsac_hip_bf8l.argtypes = [vp, sz, sz, vp, vp, vp]
        lib.tsac_hip_bf8l_tiles.argtypes = [vp, sz, sz, vp, vp, vp]
        lib.tsac_hip_tile_rows.argtypes = [sz]
        lib.tsac_hip_tile_rows.restype = sz
        lib.tsac_hip_layer_norm.argtypes = [vp, sz, sz, vp, vp, vp, vp]
        lib.tsac_hip_softmax.argtypes = [vp, sz, sz, vp, vp]
        lib.tsac_hip_gelu.argtypes = [vp, sz, vp, vp]
        lib.tsac_hip_rotary.argtypes = [vp, vp, sz, vp, vp]
        lib.tsac_hip_add.argtypes = [vp, vp, sz, sz, sz, vp, vp]
        lib.tsac_hip_attention.argtypes = [vp, vp, vp, sz, sz, sz, sz, sz, C.c_float, C.c_int, vp, vp]
        lib.tsac_hip_attention_causal.argtypes = [vp, sz, sz, vp, vp, vp, sz, sz, vp, C.c_float, vp, vp]
        lib.tsac_hip_probe_read.argtypes = [vp, sz, vp]
        lib.tsac_hip_probe_mfma.argtypes = [sz, C.c_int, C.POINTER(C.c_double), vp]
        lib.tsac_hip_source_load.argtypes = [C.c_char_p, C.POINTER(SourceLimits), C.POINTER(vp)]
        lib.tsac_hip_source_parse.argtypes = [u8p, sz, C.POINTER(SourceLimits), C.POINTER(vp)]
        lib.tsac_hip_source_destroy.argtypes = [vp]
        lib.tsac_hip_source_tensor_count.argtypes = [vp, C.POINTER(sz)]
        lib.tsac_hip_source_tensor_info.argtypes = [vp, sz, C.POINTER(SourceTensorInfo)]
        lib.tsac_hip_source_metadata.argtypes = [vp, C.POINTER(C.c_char_p), C.POINTER(sz)]
        lib.tsac_hip_source_dequantize.argtypes = [vp, C.c_char_p, f32p, sz]
        lib.tsac_hip_source_dac_config.argtypes = [vp, C.POINTER(C.c_uint32), C.POINTER(C.c_uint32)]
        lib.tsac_hip_source_transformer_config.argtypes = [vp, C.POINTER(C.c_uint32)]
        lib.tsac_hip_prepare_transformer.argtypes = [vp, vp, C.POINTER(vp), C.POINTER(ModelDesc)]
        lib.tsac_hip_prepared_transformer_destroy.argtypes = [vp]
        lib.tsac_hip_prepare_dac.argtypes = [vp, C.POINTER(vp), C.POINTER(DacDesc)]
        lib.tsac_hip_prepared_dac_destroy.argtypes = [vp]
        lib.tsac_hip_model_create_from_source.argtypes = [vp, vp, C.POINTER(Limits), C.POINTER(vp)]
        lib.tsac_hip_dac_create_from_source.argtypes = [vp, C.POINTER(Limits), C.POINTER(vp)]
        lib.tsac_hip_pcm16_read.argtypes = [u8p, sz, C.c_uint32, C.POINTER(Limits), C.POINTER(f32p), C.POINTER(sz)]
        lib.tsac_hip_wave_read.argtypes = [u8p, sz, C.POINTER(Limits), C.POINTER(f32p), C.POINTER(sz),
                                           C.POINTER(C.c_uint32)]
        lib.tsac_hip_wave_write.argtypes = [f32p, sz, C.c_uint32, C.POINTER(Limits), C.POINTER(u8p), C.POINTER(sz)]
        lib.tsac_hip_audio_header.argtypes = [sz, C.c_uint32, C.POINTER(EncodeOptions), C.POINTER(Limits),
                                              C.POINTER(Header)]
        lib.tsac_hip_parse_header.argtypes = [u8p, sz, C.POINTER(Limits), C.POINTER(Header)]
        lib.tsac_hip_cli_parse.argtypes = [sz, C.POINTER(C.c_char_p), C.POINTER(CliOptions)]
        lib.tsac_hip_cli_help.restype = C.c_char_p
        _lib = lib
    return _lib


def check(status: int) -> None:
    if status:
        raise HipError(library().tsac_hip_last_error().decode())


def _ptr(array: np.ndarray, ctype):
    assert array.flags["C_CONTIGUOUS"]
    return array.ctypes.data_as(C.POINTER(ctype))


def model_desc(model):
    """ModelDesc over a tsac_hip.synthetic.Model; returns (desc, keepalive)."""
    g = model.geometry
    geometry = Geometry(g.width, g.heads, g.head_width, g.ffn, g.temporal_layers, g.codebook_layers,
                        g.latent, g.alphabet, g.books, g.channels, g.context, g.attention_scale)
    keep = []
    linears = (Linear * len(model.projections))()
    for i, (values, scales, bias) in enumerate(model.projections):
        values, scales, bias = (np.ascontiguousarray(a) for a in (values, scales, bias))
        keep += [values, scales, bias]
        linears[i] = Linear(_ptr(values, C.c_int8), _ptr(scales, C.c_float), _ptr(bias, C.c_float))
    gains = [np.ascontiguousarray(a) for a in model.norm_gain]
    biases = [np.ascontiguousarray(a) for a in model.norm_bias]
    gain_ptrs = (u16p * len(gains))(*[_ptr(a, C.c_uint16) for a in gains])
    bias_ptrs = (u16p * len(biases))(*[_ptr(a, C.c_uint16) for a in biases])
    arrays = [np.ascontiguousarray(model.positions), np.ascontiguousarray(model.rotations),
              np.ascontiguousarray(model.embeddings)]
    keep += [linears, gains, biases, gain_ptrs, bias_ptrs, arrays]
    desc = ModelDesc(geometry, linears, gain_ptrs, bias_ptrs, _ptr(arrays[0], C.c_uint16),
                     _ptr(arrays[1], C.c_uint16), _ptr(arrays[2], C.c_uint16))
    return desc, keep


def _release(owner, destroy: str):
    """Destroys owner.handle once. The destroy entry point is resolved while the
    handle is created (owner._library), so a finaliser that runs during interpreter
    shutdown, after this module's globals are cleared, still reaches it."""
    handle = getattr(owner, "handle", None)
    lib = getattr(owner, "_library", None)
    if handle and lib is not None:
        getattr(lib, destroy)(handle)
    owner.handle = None


class SourceFile:
    """An original model file (tsac_*_q8.bin or dac_*_q8.bin) parsed by the
    library (tsac_hip_source_parse/load: SourceModel, src/weights/source_model.hpp)."""

    def __init__(self, data: bytes | None = None, path: str | None = None, limits: SourceLimits | None = None):
        lib = library()
        handle = vp()
        if path is not None:
            check(lib.tsac_hip_source_load(str(path).encode(), C.byref(limits) if limits else None,
                                           C.byref(handle)))
        else:
            b = np.frombuffer(data, np.uint8).copy() if data else np.zeros(1, np.uint8)
            check(lib.tsac_hip_source_parse(_ptr(b, C.c_uint8), len(data), C.byref(limits) if limits else None,
                                            C.byref(handle)))
        self.handle, self._library = handle, lib

    def __del__(self, release=_release):  # bound now: module globals are cleared at shutdown
        release(self, "tsac_hip_source_destroy")

    def close(self):
        _release(self, "tsac_hip_source_destroy")

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def tensors(self) -> list:
        """[(name, storage, dims (axis 0 fastest), elements)] in file order."""
        n = sz()
        check(library().tsac_hip_source_tensor_count(self.handle, C.byref(n)))
        out = []
        for i in range(n.value):
            info = SourceTensorInfo()
            check(library().tsac_hip_source_tensor_info(self.handle, i, C.byref(info)))
            out.append((info.name.decode(), info.storage, tuple(info.dims[:info.rank]), info.elements))
        return out

    def metadata(self) -> bytes:
        p, n = C.c_char_p(), sz()
        check(library().tsac_hip_source_metadata(self.handle, C.byref(p), C.byref(n)))
        return C.string_at(p, n.value)

    def dequantize(self, name: str) -> np.ndarray:
        elements = {t[0]: t[3] for t in self.tensors()}.get(name, 0)
        out = np.zeros(max(elements, 1), np.float32)
        check(library().tsac_hip_source_dequantize(self.handle, name.encode(), _ptr(out, C.c_float), out.size))
        return out[:elements]

    def dac_config(self) -> tuple:
        channels, books = C.c_uint32(), C.c_uint32()
        check(library().tsac_hip_source_dac_config(self.handle, C.byref(channels), C.byref(books)))
        return channels.value, books.value

    def transformer_books(self) -> int:
        books = C.c_uint32()
        check(library().tsac_hip_source_transformer_config(self.handle, C.byref(books)))
        return books.value


def _bytes_arg(data: bytes):
    return np.frombuffer(data, np.uint8).copy() if data else np.zeros(1, np.uint8)


def pcm16_read(data: bytes, channels: int, limits: Limits | None = None) -> np.ndarray:
    """tsac_hip_pcm16_read: float PCM [frames][channels], padded to 512 frames."""
    b, out, frames = _bytes_arg(data), f32p(), sz()
    check(library().tsac_hip_pcm16_read(_ptr(b, C.c_uint8), len(data), channels, C.byref(limits) if limits else None,
                                        C.byref(out), C.byref(frames)))
    pcm = np.ctypeslib.as_array(out, shape=(frames.value * channels,)).copy() if frames.value else np.zeros(0, np.float32)
    library().tsac_hip_free(out)
    return pcm.reshape(frames.value, channels)


def wave_read(data: bytes, limits: Limits | None = None) -> np.ndarray:
    """tsac_hip_wave_read: float PCM [frames][channels] of a 44100 Hz 16-bit WAVE file."""
    b, out, frames, channels = _bytes_arg(data), f32p(), sz(), C.c_uint32()
    check(library().tsac_hip_wave_read(_ptr(b, C.c_uint8), len(data), C.byref(limits) if limits else None,
                                       C.byref(out), C.byref(frames), C.byref(channels)))
    count = frames.value * channels.value
    pcm = np.ctypeslib.as_array(out, shape=(count,)).copy() if count else np.zeros(0, np.float32)
    library().tsac_hip_free(out)
    return pcm.reshape(frames.value, channels.value)


def wave_write(samples: np.ndarray, limits: Limits | None = None) -> bytes:
    """tsac_hip_wave_write of float PCM [frames][channels]."""
    pcm = np.ascontiguousarray(samples, np.float32)
    frames, channels = pcm.shape
    out, n = u8p(), sz()
    check(library().tsac_hip_wave_write(_ptr(pcm, C.c_float) if pcm.size else None, frames, channels,
                                        C.byref(limits) if limits else None, C.byref(out), C.byref(n)))
    data = C.string_at(out, n.value)
    library().tsac_hip_free(out)
    return data


def audio_header(frames: int, channels: int, method=1, codebooks=0, separate_channels=False, entropy_batch=0,
                 limits: Limits | None = None) -> Header:
    options = EncodeOptions(method, codebooks, int(separate_channels), entropy_batch)
    h = Header()
    check(library().tsac_hip_audio_header(frames, channels, C.byref(options), C.byref(limits) if limits else None,
                                          C.byref(h)))
    return h


def parse_header(stream: bytes, limits: Limits | None = None) -> Header:
    b, h = _bytes_arg(stream), Header()
    check(library().tsac_hip_parse_header(_ptr(b, C.c_uint8), len(stream), C.byref(limits) if limits else None,
                                          C.byref(h)))
    return h


def cli_parse(arguments: list) -> dict:
    """tsac_hip_cli_parse of the arguments after the program name."""
    encoded = [a.encode() for a in arguments]
    argv = (C.c_char_p * max(len(encoded), 1))(*encoded)
    o = CliOptions()
    check(library().tsac_hip_cli_parse(len(encoded), argv, C.byref(o)))
    return {"command": o.command.decode() if o.command != b"\0" else "", "input": o.input and o.input.decode(),
            "output": o.output and o.output.decode(), "threads": o.threads, "quality": o.quality,
            "channels": o.channels, "batch": o.batch, "verbose": o.verbose, "fast": bool(o.fast),
            "separate": bool(o.separate), "help": bool(o.help), "metal": bool(o.metal)}


def cli_help() -> str:
    return library().tsac_hip_cli_help().decode()


def prepare_transformer(transformer: SourceFile, dac: SourceFile):
    """The packer's preparation of a probability model (tsac_hip_prepare_transformer),
    copied out as a tsac_hip.synthetic.Model."""
    from .synthetic import Geometry as GeometryShape, Model

    prepared, desc = vp(), ModelDesc()
    check(library().tsac_hip_prepare_transformer(transformer.handle, dac.handle, C.byref(prepared),
                                                 C.byref(desc)))
    try:
        g = desc.geometry
        geometry = GeometryShape(g.width, g.heads, g.head_width, g.ffn, g.temporal_layers, g.codebook_layers,
                                 g.latent, g.alphabet, g.books, g.channels, g.context)
        projections = []
        for i in range(geometry.projection_count):
            k, n = geometry.projection_shape(i)
            linear = desc.projections[i]
            projections.append((np.ctypeslib.as_array(linear.values, shape=(n, k)).copy(),
                                np.ctypeslib.as_array(linear.scales, shape=(k // 256, n)).copy(),
                                np.ctypeslib.as_array(linear.bias, shape=(n,)).copy()))
        gains = [np.ctypeslib.as_array(desc.norm_gain[i], shape=(g.width,)).copy() for i in range(geometry.norm_count)]
        biases = [np.ctypeslib.as_array(desc.norm_bias[i], shape=(g.width,)).copy() for i in range(geometry.norm_count)]
        positions = np.ctypeslib.as_array(desc.positions, shape=(g.books, g.width)).copy()
        rotations = np.ctypeslib.as_array(desc.rotations, shape=(g.context, g.head_width)).copy()
        embeddings = np.ctypeslib.as_array(desc.embeddings, shape=(g.books, g.alphabet, g.latent)).copy()
        return Model(geometry, projections, gains, biases, positions, rotations, embeddings)
    finally:
        library().tsac_hip_prepared_transformer_destroy(prepared)


def prepare_dac(dac: SourceFile) -> dict:
    """The packer's preparation of a codec (tsac_hip_prepare_dac), copied out:
    {"channels", "books", "analysis"/"synthesis": [(dims, values or (int8, BF16 scales), gain, bias)],
    "analysis_alpha"/"synthesis_alpha": [alpha], "rvq": [(codebook, search, input_weights,
    input_bias, output_weights, output_bias)]}."""
    prepared, desc = vp(), DacDesc()
    check(library().tsac_hip_prepare_dac(dac.handle, C.byref(prepared), C.byref(desc)))
    try:
        out = {"channels": desc.channels, "books": desc.books}
        for graph in ("analysis", "synthesis"):
            convs = []
            for c in getattr(desc, graph):
                dims = tuple(c.dims)
                count = dims[0] * dims[1] * dims[2]
                outer = dims[2]
                channels_out = dims[0] if (graph == "synthesis" and len(convs) in range(1, 29) and
                                           (len(convs) - 1) % 7 == 0) else dims[2]
                if c.quantized:
                    padded = (dims[1] + 7) // 8 * 8
                    values = (np.ctypeslib.as_array(c.quantized, shape=(count,)).copy(),
                              np.ctypeslib.as_array(c.scales, shape=(outer, dims[0] // 32, padded)).copy())
                else:
                    values = np.ctypeslib.as_array(c.values, shape=(count,)).copy()
                convs.append((dims, values, np.ctypeslib.as_array(c.gain, shape=(outer,)).copy(),
                              np.ctypeslib.as_array(c.bias, shape=(channels_out,)).copy()))
            out[graph] = convs
        from .synthetic import dac_activation_width

        for graph, synthesis in (("analysis", False), ("synthesis", True)):
            out[graph + "_alpha"] = [np.ctypeslib.as_array(getattr(desc, graph + "_alpha")[i],
                                                           shape=(dac_activation_width(synthesis, i),)).copy()
                                     for i in range(29)]
        shapes = (8192, 8192, 8192, 8, 8192, 1024)
        out["rvq"] = [tuple(np.ctypeslib.as_array(getattr(desc.rvq[b], name), shape=(n,)).copy()
                            for name, n in zip(("codebook", "search", "input_weights", "input_bias",
                                                "output_weights", "output_bias"), shapes))
                      for b in range(desc.books)]
        return out
    finally:
        library().tsac_hip_prepared_dac_destroy(prepared)


class HipModel:
    """Immutable device model (MetalTransformer::from_model, src/metal/transformer.hpp:16)."""

    def __init__(self, model, limits: Limits | None = None):
        self.geometry = model.geometry
        lib = library()
        desc, keep = model_desc(model)
        handle = vp()
        check(lib.tsac_hip_model_create(C.byref(desc), C.byref(limits) if limits else None,
                                        C.byref(handle)))
        self.handle, self._library = handle, lib
        del keep

    @classmethod
    def from_source(cls, transformer: SourceFile, dac: SourceFile, limits: Limits | None = None) -> "HipModel":
        """tsac_hip_model_create_from_source: the original files straight to the device."""
        from .synthetic import Geometry as GeometryShape

        lib = library()
        handle = vp()
        check(lib.tsac_hip_model_create_from_source(transformer.handle, dac.handle,
                                                    C.byref(limits) if limits else None, C.byref(handle)))
        self = cls.__new__(cls)
        channels, books = dac.dac_config()
        self.geometry = GeometryShape(books=books, channels=channels)
        self.handle, self._library = handle, lib
        return self

    def __del__(self, release=_release):  # bound now: module globals are cleared at shutdown
        release(self, "tsac_hip_model_destroy")

    def close(self):
        """Destroys the device model now (every session of it must be closed
        first); later calls are no-ops."""
        _release(self, "tsac_hip_model_destroy")

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def session(self) -> "HipSession":
        return HipSession(self)


class HipSession:
    """Mutable session (MetalTransformer::new_session / encode / decode)."""

    def __init__(self, model: HipModel):
        self.model = model
        handle = vp()
        check(library().tsac_hip_session_create(model.handle, C.byref(handle)))
        self.handle, self._library = handle, library()

    def __del__(self, release=_release):  # bound now: module globals are cleared at shutdown
        release(self, "tsac_hip_session_destroy")

    def close(self):
        """Destroys the session (its stream, caches and scratch) now; later
        calls are no-ops."""
        _release(self, "tsac_hip_session_destroy")

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def clear(self):
        check(library().tsac_hip_session_clear(self.handle))

    def encode(self, h: Header, tokens) -> bytes:
        t = np.ascontiguousarray(tokens, np.uint16)
        out, n = u8p(), sz()
        check(library().tsac_hip_encode(self.handle, C.byref(h), _ptr(t, C.c_uint16), t.size,
                                        C.byref(out), C.byref(n)))
        data = C.string_at(out, n.value)
        library().tsac_hip_free(out)
        return data

    def decode(self, data: bytes) -> np.ndarray:
        b = np.frombuffer(data, np.uint8).copy() if data else np.zeros(1, np.uint8)
        out, n = u16p(), sz()
        check(library().tsac_hip_decode(self.handle, _ptr(b, C.c_uint8), len(data), C.byref(out),
                                        C.byref(n)))
        tokens = np.ctypeslib.as_array(out, shape=(n.value,)).copy() if n.value else np.zeros(0, np.uint16)
        library().tsac_hip_free(out)
        return tokens

    @staticmethod
    def _observer(before, after):
        """C observer over Python callables before(position) and
        after(position, bits), each given a Position; a callable returning a
        true value stops the call."""
        b = BEFORE_SYMBOL(lambda _, p: int(bool(before(p.contents)))) if before else BEFORE_SYMBOL()
        a = AFTER_SYMBOL(lambda _, p, bits: int(bool(after(p.contents, bits)))) if after else AFTER_SYMBOL()
        return Observer(None, b, a), (b, a)

    def encode_observed(self, h: Header, tokens, before=None, after=None) -> bytes:
        t = np.ascontiguousarray(tokens, np.uint16)
        out, n = u8p(), sz()
        observer, keep = self._observer(before, after)
        check(library().tsac_hip_encode_observed(self.handle, C.byref(h), _ptr(t, C.c_uint16), t.size,
                                                 C.byref(observer), C.byref(out), C.byref(n)))
        data = C.string_at(out, n.value)
        library().tsac_hip_free(out)
        del keep
        return data

    def decode_observed(self, data: bytes, before=None, after=None) -> np.ndarray:
        b = np.frombuffer(data, np.uint8).copy() if data else np.zeros(1, np.uint8)
        out, n = u16p(), sz()
        observer, keep = self._observer(before, after)
        check(library().tsac_hip_decode_observed(self.handle, _ptr(b, C.c_uint8), len(data), C.byref(observer),
                                                 C.byref(out), C.byref(n)))
        tokens = np.ctypeslib.as_array(out, shape=(n.value,)).copy() if n.value else np.zeros(0, np.uint16)
        library().tsac_hip_free(out)
        del keep
        return tokens

    def distributions(self, h: Header, tokens, mode: int = PASS_ENCODE) -> np.ndarray:
        t = np.ascontiguousarray(tokens, np.uint16)
        out = np.zeros((t.size, self.model.geometry.alphabet), np.uint16)
        check(library().tsac_hip_distributions(self.handle, C.byref(h), _ptr(t, C.c_uint16), t.size,
                                               mode, _ptr(out, C.c_uint16)))
        return out

    #: How the frame steps of the last decode-side call were launched (timing()["frame_launch"]).
    FRAME_LAUNCH = {-1: None, 0: "cooperative", 1: "plain (TSAC_HIP_FRAME_LAUNCH=plain)",
                    2: "plain (cooperative-launch resources held by another process)"}

    def timing(self):
        t = (C.c_double * 8)()
        check(library().tsac_hip_session_timing(self.handle, t, 8))
        return {"model": t[0], "range_coding": t[1], "total": t[2], "input_upload": t[3], "steps_gpu": t[4],
                "steps": int(t[5]), "frame_launch": self.FRAME_LAUNCH[int(t[6])], "stepwise": bool(t[7])}


def prepare_rvq(codebook, in_v, in_g, out_v, out_g):
    """The packer's quantizer preparation (tsac_hip_prepare_rvq): (search,
    input_weights, output_weights) for one codebook."""
    a = [np.ascontiguousarray(x, np.float32) for x in (codebook, in_v, in_g, out_v, out_g)]
    out = [np.zeros(8192, np.float32) for _ in range(3)]
    check(library().tsac_hip_prepare_rvq(*[_ptr(x, C.c_float) for x in a + out]))
    return out


class HipDac:
    """The DAC codec's device model (tsac_hip_dac_create) from a
    tsac_hip.synthetic.DacModel: convolutions in their source encoding, Snake
    alphas, and the quantizer prepared as the packer prepares it."""

    @classmethod
    def from_source(cls, dac: SourceFile, limits: Limits | None = None) -> "HipDac":
        """tsac_hip_dac_create_from_source: an original codec file straight to the device."""
        lib = library()
        handle = vp()
        check(lib.tsac_hip_dac_create_from_source(dac.handle, C.byref(limits) if limits else None, C.byref(handle)))
        self = cls.__new__(cls)
        self.channels, self.books = dac.dac_config()
        self.handle, self._library = handle, lib
        return self

    def __init__(self, model, limits: Limits | None = None):
        self.channels, self.books = model.channels, len(model.codebook)
        desc = DacDesc()
        desc.channels, desc.books = model.channels, self.books
        keep = []
        for name, convs, alphas in (("analysis", model.analysis, model.analysis_alpha),
                                    ("synthesis", model.synthesis, model.synthesis_alpha)):
            for i, conv in enumerate(convs):
                d = getattr(desc, name)[i]
                d.dims = (C.c_uint32 * 3)(*conv.dims)
                gain, bias = np.ascontiguousarray(conv.gain, np.float32), np.ascontiguousarray(conv.bias, np.float32)
                keep += [gain, bias]
                d.gain, d.bias = _ptr(gain, C.c_float), _ptr(bias, C.c_float)
                if conv.bf8:
                    q, sc = np.ascontiguousarray(conv.values, np.int8), np.ascontiguousarray(conv.scales, np.uint16)
                    keep += [q, sc]
                    d.quantized, d.scales = _ptr(q, C.c_int8), _ptr(sc, C.c_uint16)
                else:
                    v = np.ascontiguousarray(conv.values, np.float32)
                    keep.append(v)
                    d.values = _ptr(v, C.c_float)
            for i, a in enumerate(alphas):
                a = np.ascontiguousarray(a, np.float32)
                keep.append(a)
                getattr(desc, name + "_alpha")[i] = _ptr(a, C.c_float)
        for b in range(self.books):
            search, input_weights, output_weights = prepare_rvq(model.codebook[b], model.in_v[b], model.in_g[b],
                                                                model.out_v[b], model.out_g[b])
            parts = [np.ascontiguousarray(model.codebook[b], np.float32), search, input_weights,
                     np.ascontiguousarray(model.in_bias[b], np.float32), output_weights,
                     np.ascontiguousarray(model.out_bias[b], np.float32)]
            keep += parts
            desc.rvq[b] = RvqBook(*[_ptr(x, C.c_float) for x in parts])
        handle = vp()
        check(library().tsac_hip_dac_create(C.byref(desc), C.byref(limits) if limits else None, C.byref(handle)))
        self.handle, self._library = handle, library()
        del keep

    def __del__(self, release=_release):  # bound now: module globals are cleared at shutdown
        release(self, "tsac_hip_dac_destroy")

    def close(self):
        _release(self, "tsac_hip_dac_destroy")

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def analyze(self, session: "HipSession", pcm, frames, groups=1, codebooks=None) -> np.ndarray:
        """Padded interleaved PCM [frames*512][groups*channels] -> tokens [frame][group][book]."""
        books = codebooks or self.books
        pcm = np.ascontiguousarray(pcm, np.float32)
        tokens = np.zeros(frames * groups * books, np.uint16)
        check(library().tsac_hip_dac_analyze(session.handle, self.handle, _ptr(pcm, C.c_float), frames, groups, books,
                                             _ptr(tokens, C.c_uint16)))
        return tokens

    def apply(self, session: "HipSession", synthesis: bool, x, frames) -> np.ndarray:
        """DacAnalysis/DacSynthesis::apply on one window (reference Signal layout)."""
        x = np.ascontiguousarray(x, np.float32)
        count = frames * 512 * self.channels if synthesis else frames // 512 * 1024
        out = np.zeros(count, np.float32)
        check(library().tsac_hip_dac_apply(session.handle, self.handle, int(synthesis), _ptr(x, C.c_float), frames,
                                           _ptr(out, C.c_float)))
        return out

    def synthesize(self, session: "HipSession", tokens, frames, groups=1, codebooks=None) -> np.ndarray:
        books = codebooks or self.books
        tokens = np.ascontiguousarray(tokens, np.uint16)
        pcm = np.zeros(frames * 512 * groups * self.channels, np.float32)
        check(library().tsac_hip_dac_synthesize(session.handle, self.handle, _ptr(tokens, C.c_uint16), frames,
                                                groups, books, _ptr(pcm, C.c_float)))
        return pcm

    def encode(self, session: "HipSession", samples, channels, method=1, codebooks=0, separate_channels=False,
               entropy_batch=0, before=None, after=None) -> bytes:
        """AudioAnalyzer::encode of interleaved float PCM [frames][channels]."""
        samples = np.ascontiguousarray(samples, np.float32)
        options = EncodeOptions(method, codebooks, int(separate_channels), entropy_batch)
        observer, keep = HipSession._observer(before, after)
        out, n = u8p(), sz()
        check(library().tsac_hip_audio_encode(session.handle, self.handle, _ptr(samples, C.c_float),
                                              samples.size // channels, channels, C.byref(options), C.byref(observer),
                                              C.byref(out), C.byref(n)))
        data = C.string_at(out, n.value)
        library().tsac_hip_free(out)
        del keep
        return data

    def decode(self, session: "HipSession", data: bytes, before=None, after=None):
        """AudioAnalyzer::decode: (interleaved float PCM [frames][channels], channels)."""
        b = np.frombuffer(data, np.uint8).copy() if data else np.zeros(1, np.uint8)
        observer, keep = HipSession._observer(before, after)
        out, frames, channels = f32p(), sz(), C.c_uint32()
        check(library().tsac_hip_audio_decode(session.handle, self.handle, _ptr(b, C.c_uint8), len(data),
                                              C.byref(observer), C.byref(out), C.byref(frames), C.byref(channels)))
        count = frames.value * channels.value
        pcm = np.ctypeslib.as_array(out, shape=(count,)).copy() if count else np.zeros(0, np.float32)
        library().tsac_hip_free(out)
        del keep
        return pcm.reshape(frames.value, channels.value), channels.value


# ---------------------------------------------------------------- operators on torch tensors

def _stream(stream=None):
    import torch

    s = stream if stream is not None else torch.cuda.current_stream()
    return vp(s.cuda_stream)


def _dp(tensor):
    assert tensor.is_cuda and tensor.is_contiguous()
    return vp(tensor.data_ptr())


class DeviceLinear:
    """PackedLinear on the GPU (src/common/packed_linear.tpp:216-302)."""

    def __init__(self, values: np.ndarray, scales: np.ndarray, bias: np.ndarray):
        n, k = values.shape
        self.K, self.N = k, n
        values = np.ascontiguousarray(values, np.int8)
        scales = np.ascontiguousarray(scales, np.float32)
        bias = np.ascontiguousarray(bias, np.float32)
        desc = Linear(_ptr(values, C.c_int8), _ptr(scales, C.c_float), _ptr(bias, C.c_float))
        handle = vp()
        check(library().tsac_hip_linear_create(C.byref(desc), k, n, C.byref(handle)))
        self.handle, self._library = handle, library()

    def __del__(self, release=_release):  # bound now: module globals are cleared at shutdown
        release(self, "tsac_hip_linear_destroy")

    def apply(self, x, y, path=PATH_AUTO, stream=None):
        """x: int16/uint16 cuda tensor [M][K] of BF16 bits -> y [M][N]."""
        m = x.numel() // self.K
        check(library().tsac_hip_linear_apply(self.handle, _dp(x), m, _dp(y), path, _stream(stream)))

    def apply_static(self, x, y, path=PATH_AUTO, stream=None):
        """apply() with the BF8L buffer in the library's fixed device array (no allocation)."""
        m = x.numel() // self.K
        check(library().tsac_hip_linear_apply_static(self.handle, _dp(x), m, _dp(y), path, _stream(stream)))

    def apply_quantized(self, q, scales, m, y, residual=None, path=PATH_AUTO, stream=None):
        check(library().tsac_hip_linear_apply_quantized(
            self.handle, _dp(q), _dp(scales), m, _dp(y), _dp(residual) if residual is not None else None,
            path, _stream(stream)))


def bf8l(x, rows, k, q, scales, stream=None):
    check(library().tsac_hip_bf8l(_dp(x), rows, k, _dp(q), _dp(scales), _stream(stream)))


def bf8l_tiles(x, rows, k, q, scales, stream=None):
    """BF8L into MFMA operand tiles: q holds tile_rows(rows)*k bytes, scales
    tile_rows(rows)*k/256 floats (transposed)."""
    check(library().tsac_hip_bf8l_tiles(_dp(x), rows, k, _dp(q), _dp(scales), _stream(stream)))


def tile_rows(rows):
    return int(library().tsac_hip_tile_rows(rows))


def layer_norm(x, rows, width, gain, bias, out, stream=None):
    check(library().tsac_hip_layer_norm(_dp(x), rows, width, _dp(gain), _dp(bias), _dp(out),
                                        _stream(stream)))


def softmax(x, rows, width, out, stream=None):
    check(library().tsac_hip_softmax(_dp(x), rows, width, _dp(out), _stream(stream)))


def gelu(x, out, stream=None):
    check(library().tsac_hip_gelu(_dp(x), x.numel(), _dp(out), _stream(stream)))


def rotary(x, coefficients, out, stream=None):
    check(library().tsac_hip_rotary(_dp(x), _dp(coefficients), x.numel(), _dp(out), _stream(stream)))


def add(a, b, rows, width, period, out, stream=None):
    check(library().tsac_hip_add(_dp(a), _dp(b), rows, width, period, _dp(out), _stream(stream)))


def attention(query, keys, values, sequence_stride, sequences, time, heads, head_width, scale,
              prefill, out, stream=None):
    check(library().tsac_hip_attention(_dp(query), _dp(keys), _dp(values), sequence_stride, sequences,
                                       time, heads, head_width, scale, int(prefill), _dp(out),
                                       _stream(stream)))


def attention_causal(qkv, heads, head_width, start, length, replay, sequences, max_length, rotations,
                     scale, out, stream=None):
    check(library().tsac_hip_attention_causal(
        _dp(qkv), heads, head_width, _dp(start), _dp(length), _dp(replay), sequences, max_length,
        _dp(rotations) if rotations is not None else None, scale, _dp(out), _stream(stream)))


def probe_read(data, stream=None):
    """One streaming read pass over a contiguous cuda tensor (size a multiple of 64 KiB)."""
    check(library().tsac_hip_probe_read(_dp(data), data.numel() * data.element_size(), _stream(stream)))


def probe_mfma(workgroups: int, iterations: int, stream=None) -> float:
    """Launches the int8 MFMA loop; returns the operations that launch performs."""
    ops = C.c_double()
    check(library().tsac_hip_probe_mfma(workgroups, iterations, C.byref(ops), _stream(stream)))
    return ops.value
