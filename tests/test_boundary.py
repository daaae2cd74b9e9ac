"""The drop-in boundary without a GPU: the C-ABI library loads, exports every
function include/tsac_hip.h declares, and reports argument errors as a status
plus a message (no exception crosses the ABI)."""
import ctypes
import pathlib
import re
import shutil
import subprocess

import numpy as np
import pytest

ROOT = pathlib.Path(__file__).resolve().parent.parent


def declared_functions():
    text = (ROOT / "include" / "tsac_hip.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(tsac_hip_\w+)\s*\(", text)))


def test_header_declares_the_operator_surface():
    names = declared_functions()
    for required in ("tsac_hip_model_create", "tsac_hip_session_create", "tsac_hip_encode",
                     "tsac_hip_decode", "tsac_hip_linear_apply", "tsac_hip_attention"):
        assert required in names


def test_library_exports_every_declared_symbol():
    from tsac_hip import native

    lib = native.library()
    for name in declared_functions():
        assert hasattr(lib, name), name
    assert set(native.EXPORTS) == set(declared_functions())


def test_errors_cross_the_abi_as_status_codes():
    from tsac_hip import native

    lib = native.library()
    handle = ctypes.c_void_p()
    assert lib.tsac_hip_model_create(None, None, ctypes.byref(handle)) != 0
    assert b"missing" in lib.tsac_hip_last_error()
    assert lib.tsac_hip_session_create(None, ctypes.byref(handle)) != 0


def test_model_validation_runs_before_any_device_work():
    """An invalid geometry is rejected by the host checks (no GPU needed)."""
    from tsac_hip import native
    from tsac_hip.synthetic import Geometry, random_model

    model = random_model(Geometry(width=256, heads=2, head_width=128, ffn=256, temporal_layers=1,
                                  codebook_layers=1, latent=256), seed=1)
    model.geometry = Geometry(width=256, heads=3, head_width=128, ffn=256, temporal_layers=1,
                              codebook_layers=1, latent=256)
    with pytest.raises(native.HipError, match="heads"):
        native.HipModel(model)


def test_synthetic_model_layout():
    from tsac_hip.synthetic import REFERENCE, random_model

    model = random_model(REFERENCE, seed=1)
    assert len(model.projections) == 63 and len(model.norm_gain) == 32
    values, scales, bias = model.projections[0]
    assert values.shape == (1536, 512) and scales.shape == (2, 1536) and bias.shape == (1536,)
    assert model.projections[60][0].shape == (512, 1024) and not model.projections[60][2].any()
    assert model.embeddings.shape == (12, 1024, 1024)
    # Block scales are BF16-representable, as the packed format stores them.
    assert not (scales.view(np.uint32) & 0xFFFF).any()


REFERENCE_TREE = pathlib.Path("/root/reference")


@pytest.mark.parametrize("compiler", [["g++", "-std=c++2b"], ["/opt/rocm/llvm/bin/clang++", "-std=c++23"]],
                         ids=["g++", "clang++"])
def test_reference_side_adapter_compiles(compiler):
    """tsac-metal_amd/integration/hip_transformer.cpp (HipTransformer, the
    MetalTransformer drop-in) type-checks against the reference's own headers
    and include/tsac_hip.h, so a change to either side that breaks it fails here."""
    if not (REFERENCE_TREE / "src" / "format" / "entropy.hpp").exists():
        pytest.skip("reference tree not present")
    if shutil.which(compiler[0]) is None:
        pytest.skip(f"{compiler[0]} not installed")
    source = ROOT / "tsac-metal_amd" / "integration" / "hip_transformer.cpp"
    run = subprocess.run(compiler + ["-fsyntax-only", "-Wall", "-Wextra", "-Werror", f"-I{ROOT / 'include'}",
                                     f"-I{REFERENCE_TREE / 'src'}", f"-I{REFERENCE_TREE / 'include'}", str(source)],
                         capture_output=True, text=True)
    assert run.returncode == 0, run.stderr
