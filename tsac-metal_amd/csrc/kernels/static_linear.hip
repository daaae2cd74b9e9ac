// Allocation-free qlinear: PackedLinear::apply_into on BF16 rows with the BF8L
// buffer in a fixed device array instead of stream-ordered scratch, for callers
// that cannot allocate device memory.
//
// Every call on a device shares that device's copy of the array and leaves its
// contents behind: the error words are cleared by a kernel at the start of each
// call, and calls that overlap on one device race on the buffer.
#include "kernels.hpp"

#include <mutex>

namespace
{
// Quantised activations (int8, rows or MFMA operand tiles), then their fp32
// block scales (one per 256 values), then the two error words.
constexpr std::size_t static_values_bytes = std::size_t{16} << 20;
constexpr std::size_t static_scales_bytes = static_values_bytes / 64;
constexpr std::size_t static_scratch_bytes = static_values_bytes + static_scales_bytes + 256;
} // namespace

// The buffer itself (16.25 MiB per device, held until the process ends). Host
// code never uses this name as an address: it takes each device's address from
// hipGetSymbolAddress (static_scratch below).
static __device__ __align__(256) uint8_t scratch[static_scratch_bytes];

namespace tsac_hip
{
namespace
{
__global__ void clear_words(uint32_t* words, int count)
{
    if (int(threadIdx.x) < count)
    {
        words[threadIdx.x] = 0u;
    }
}

constexpr int max_devices = 64;
std::mutex setup;
uint8_t* addresses[max_devices] = {};

// This device's copy of `scratch`, looked up once per device with the device current.
uint8_t* static_scratch()
{
    int device = 0;
    check_hip(hipGetDevice(&device), "hipGetDevice");
    require(device >= 0 && device < max_devices, "static qlinear: device index out of range");
    std::lock_guard<std::mutex> lock(setup);
    if (!addresses[device])
    {
        void* address = nullptr;
        check_hip(hipGetSymbolAddress(&address, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
        require(address != nullptr, "static qlinear: no device address for the scratch buffer");
        addresses[device] = static_cast<uint8_t*>(address);
    }
    return addresses[device];
}
} // namespace

std::size_t static_linear_max_bytes()
{
    return static_values_bytes;
}

void linear_apply_static(const DeviceLinear& w, const uint16_t* x, std::size_t M, uint16_t* y, LinearPath path,
                         hipStream_t stream)
{
    const std::size_t K = w.K;
    const bool tiles = path == LinearPath::gemm || (path == LinearPath::automatic && M > small_gemm_max_rows() &&
                                                    !small_gemm_chosen(M, w.N, K));
    const Layout layout = tiles ? Layout::tiles : Layout::rows;
    const std::size_t rows = tiles ? tile_padded_rows(M) : M;
    require(K % 256 == 0 && rows * K <= static_values_bytes,
            "static qlinear: activations exceed the 16 MiB static buffer (padded rows x K)");
    uint8_t* base = static_scratch();
    auto* q = reinterpret_cast<int8_t*>(base);
    auto* scales = reinterpret_cast<float*>(base + static_values_bytes);
    auto* error = reinterpret_cast<uint32_t*>(base + static_values_bytes + static_scales_bytes);
    clear_words<<<1, 64, 0, stream>>>(error, 2);
    check_hip(hipGetLastError(), "clear error words");
    quantize_rows(x, M, K, Prologue::none, nullptr, nullptr, q, scales, nullptr, error, stream, layout);
    linear(w, q, scales, M, y, nullptr, path, stream, layout);
    uint32_t flags[2] = {0u, 0u};
    check_hip(hipMemcpyAsync(flags, error, sizeof flags, hipMemcpyDeviceToHost, stream), "read error words");
    check_hip(hipStreamSynchronize(stream), "hipStreamSynchronize");
    require(!flags[0], "BF8L activations must be finite");
}
} // namespace tsac_hip
