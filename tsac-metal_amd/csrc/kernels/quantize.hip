// BF8L activation quantisation with optional LayerNorm or GELU prologue.
//
// One 64-lane wavefront owns one row of K BF16 values; lane l holds the V = K/64
// consecutive values [l*V, l*V+V). That placement makes the cross-lane
// adjacent-pair tree (strides 1, 2, 4, ...) identical to the reference's pair
// tree over the whole row, and puts each 256-value BF8L block on 256/V aligned
// neighbouring lanes.
#include "kernels.hpp"
#include "row_ops.hpp"

namespace tsac_hip
{
namespace
{
constexpr int rows_per_block = 4;

template <int V, Prologue prologue>
__global__ __launch_bounds__(256) void quantize_kernel(const uint16_t* __restrict__ x, int rows,
                                                       const uint16_t* __restrict__ gain,
                                                       const uint16_t* __restrict__ bias,
                                                       int8_t* __restrict__ q,
                                                       float* __restrict__ scales,
                                                       uint16_t* __restrict__ normalized,
                                                       uint32_t* __restrict__ error,
                                                       std::size_t padded_rows)
{
    constexpr int K = 64 * V;
    const int lane = threadIdx.x % wave;
    const int row = blockIdx.x * rows_per_block + threadIdx.x / wave;
    if (row >= rows)
    {
        return;
    }
    uint16_t v[V];
    load_row<V>(x + size_t(row) * K + lane * V, v);
    if constexpr (prologue == Prologue::layer_norm)
    {
        layer_norm_lane<V>(v, gain, bias, lane);
        if (normalized)
        {
            store_row<V>(normalized + size_t(row) * K + lane * V, v);
        }
    }
    else if constexpr (prologue == Prologue::gelu)
    {
#pragma unroll
        for (int i = 0; i < V; ++i)
        {
            v[i] = gelu_bf16(v[i]);
        }
    }
    if (padded_rows)
    {
        bf8l_tiles<V>(v, lane, std::size_t(row), q, scales, padded_rows, error);
    }
    else
    {
        bf8l_lane<V>(v, lane, q + size_t(row) * K, scales + size_t(row) * (K / 256), error);
    }
}

// BF8L of row-major rows without a prologue: one row per workgroup of Waves
// waves (the row layout of bf8l_spread, which the decode frame step's
// projections use).
template <int Vw, int Waves>
__global__ __launch_bounds__(Waves * 64) void bf8l_rows_kernel(const uint16_t* __restrict__ x,
                                                               int8_t* __restrict__ q,
                                                               float* __restrict__ scales,
                                                               uint32_t* __restrict__ error)
{
    constexpr int K = Waves * wave * Vw;
    __shared__ uint32_t exchange[Waves];
    const int warp = __builtin_amdgcn_readfirstlane(int(threadIdx.x / wave));
    uint16_t v[Vw];
    load_row<Vw>(x + std::size_t(blockIdx.x) * K + threadIdx.x * Vw, v);
    bf8l_spread<Vw, Waves>(v, warp, q + std::size_t(blockIdx.x) * K, scales + std::size_t(blockIdx.x) * (K / 256),
                           error, exchange);
}

template <int Vw, int Waves>
void launch_bf8l_rows(const uint16_t* x, std::size_t rows, int8_t* q, float* scales, uint32_t* error,
                      hipStream_t stream)
{
    bf8l_rows_kernel<Vw, Waves><<<unsigned(rows), Waves * 64, 0, stream>>>(x, q, scales, error);
}

template <int V>
void launch_quantize(const uint16_t* x, std::size_t rows, Prologue prologue, const uint16_t* gain,
                     const uint16_t* bias, int8_t* q, float* scales, uint16_t* normalized,
                     uint32_t* error, std::size_t padded_rows, hipStream_t stream)
{
    const dim3 grid(unsigned((rows + rows_per_block - 1) / rows_per_block)), block(256);
    switch (prologue)
    {
    case Prologue::none:
        quantize_kernel<V, Prologue::none><<<grid, block, 0, stream>>>(
            x, int(rows), gain, bias, q, scales, normalized, error, padded_rows);
        break;
    case Prologue::layer_norm:
        quantize_kernel<V, Prologue::layer_norm><<<grid, block, 0, stream>>>(
            x, int(rows), gain, bias, q, scales, normalized, error, padded_rows);
        break;
    case Prologue::gelu:
        quantize_kernel<V, Prologue::gelu><<<grid, block, 0, stream>>>(
            x, int(rows), gain, bias, q, scales, normalized, error, padded_rows);
        break;
    }
}
} // namespace

std::size_t tile_padded_rows(std::size_t rows)
{
    return (rows + gemm_tile_rows - 1) / gemm_tile_rows * gemm_tile_rows;
}

void quantize_rows(const uint16_t* x, std::size_t rows, std::size_t K, Prologue prologue,
                   const uint16_t* gain, const uint16_t* bias, int8_t* q, float* scales,
                   uint16_t* normalized, uint32_t* error, hipStream_t stream, Layout layout)
{
    require(rows < (std::size_t(1) << 31), "too many rows");
    require(prologue != Prologue::layer_norm || (gain && bias), "layer norm needs gain and bias");
    if (rows == 0)
    {
        return;
    }
    const std::size_t padded = layout == Layout::tiles ? tile_padded_rows(rows) : 0;
    if (prologue == Prologue::none && layout == Layout::rows)
    {
        switch (K)
        {
        case 256:
            launch_bf8l_rows<1, 4>(x, rows, q, scales, error, stream);
            break;
        case 512:
            launch_bf8l_rows<1, 8>(x, rows, q, scales, error, stream);
            break;
        case 1024:
            launch_bf8l_rows<2, 8>(x, rows, q, scales, error, stream);
            break;
        case 2048:
            launch_bf8l_rows<4, 8>(x, rows, q, scales, error, stream);
            break;
        case 4096:
            launch_bf8l_rows<8, 8>(x, rows, q, scales, error, stream);
            break;
        default:
            throw Error("quantize: K must be one of 256, 512, 1024, 2048, 4096");
        }
        check_hip(hipGetLastError(), "bf8l launch");
        return;
    }
    switch (K)
    {
    case 256:
        launch_quantize<4>(x, rows, prologue, gain, bias, q, scales, normalized, error, padded, stream);
        break;
    case 512:
        launch_quantize<8>(x, rows, prologue, gain, bias, q, scales, normalized, error, padded, stream);
        break;
    case 1024:
        launch_quantize<16>(x, rows, prologue, gain, bias, q, scales, normalized, error, padded, stream);
        break;
    case 2048:
        launch_quantize<32>(x, rows, prologue, gain, bias, q, scales, normalized, error, padded, stream);
        break;
    case 4096:
        launch_quantize<64>(x, rows, prologue, gain, bias, q, scales, normalized, error, padded, stream);
        break;
    default:
        throw Error("quantize: K must be one of 256, 512, 1024, 2048, 4096");
    }
    check_hip(hipGetLastError(), "quantize launch");
}
} // namespace tsac_hip
