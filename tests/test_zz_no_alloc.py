"""tsac_hip_linear_apply_static (no device allocation; BF8L buffer in the
library's fixed per-device array) against tsac_hip_linear_apply, bit for bit,
through the C ABI: two calls in a row on each path, the second with a smaller
input, the largest input the buffer holds, and the errors it must raise."""
import numpy as np
import pytest

from tsac_hip.synthetic import bf16_bits, random_linear

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch():
    import torch

    assert torch.cuda.is_available(), "GPU tests need a visible MI355X"
    return torch


@pytest.fixture(scope="module")
def native():
    from tsac_hip import native

    native.library()
    return native


def _rows(torch, rng, m, k):
    x = bf16_bits(rng.standard_normal((m, k)).astype(np.float32))
    return torch.from_numpy(x.view(np.int16)).cuda()


@pytest.mark.parametrize("k,n,path,sizes", [
    (1024, 4096, "gemv", (8, 3)),
    (2048, 512, "gemm", (1000, 130)),
    (1024, 1024, "auto", (4096, 5)),
    (512, 1536, "auto", (300, 64)),
])
def test_static_matches_allocating_entry_point(torch, native, k, n, path, sizes):
    rng = np.random.default_rng(k + n)
    linear = native.DeviceLinear(*random_linear(rng, k, n))
    code = {"gemv": native.PATH_GEMV, "gemm": native.PATH_GEMM, "auto": native.PATH_AUTO}[path]
    for m in sizes:
        x = _rows(torch, rng, m, k)
        expected = torch.empty((m, n), dtype=torch.int16, device="cuda")
        got = torch.full((m, n), -1, dtype=torch.int16, device="cuda")
        linear.apply(x, expected, path=code)
        linear.apply_static(x, got, path=code)
        torch.cuda.synchronize()
        assert torch.equal(got, expected), (path, m)


def test_static_largest_input_and_limits(torch, native):
    rng = np.random.default_rng(5)
    k, n = 2048, 512
    linear = native.DeviceLinear(*random_linear(rng, k, n))
    x = _rows(torch, rng, 8192, k)  # 8192 x 2048 = the whole 16 MiB buffer
    expected = torch.empty((8192, n), dtype=torch.int16, device="cuda")
    got = torch.empty_like(expected)
    linear.apply(x, expected)
    linear.apply_static(x, got)
    torch.cuda.synchronize()
    assert torch.equal(got, expected)
    bigger = _rows(torch, rng, 8193, k)  # pads to 8320 rows: over the buffer
    with pytest.raises(native.HipError, match="static buffer"):
        linear.apply_static(bigger, torch.empty((8193, n), dtype=torch.int16, device="cuda"))
    # A non-finite activation is an error; the next call starts from cleared error words.
    small = _rows(torch, rng, 3, k)
    poisoned = small.clone()
    poisoned[1, 7] = 0x7F80
    out = torch.empty((3, n), dtype=torch.int16, device="cuda")
    with pytest.raises(native.HipError, match="finite"):
        linear.apply_static(poisoned, out)
    linear.apply(small, expected[:3])
    linear.apply_static(small, out)
    torch.cuda.synchronize()
    assert torch.equal(out, expected[:3])
