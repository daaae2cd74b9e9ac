// Row-wise LayerNorm (one row per workgroup, spread over its waves) and
// softmax (one wavefront per row), BF16 residual adds, GELU and rotary helpers.
#include "kernels.hpp"
#include "row_ops.hpp"

namespace tsac_hip
{
namespace
{
constexpr int rows_per_block = 4;

// One row per workgroup of Waves waves (the row layout of layer_norm_spread,
// which the decode frame step's projections use).
template <int Vw, int Waves>
__global__ __launch_bounds__(Waves * 64) void layer_norm_kernel(const uint16_t* x,
                                                                const uint16_t* __restrict__ gain,
                                                                const uint16_t* __restrict__ bias,
                                                                uint16_t* out)
{
    constexpr int width = Waves * wave * Vw;
    __shared__ float exchange[2 * Waves];
    const int warp = __builtin_amdgcn_readfirstlane(int(threadIdx.x / wave));
    const std::size_t at = std::size_t(blockIdx.x) * width + threadIdx.x * Vw;
    uint16_t v[Vw], g[Vw], b[Vw];
    load_row<Vw>(x + at, v);
    load_row<Vw>(gain + threadIdx.x * Vw, g);
    load_row<Vw>(bias + threadIdx.x * Vw, b);
    layer_norm_spread<Vw, Waves>(v, g, b, warp, exchange);
    store_row<Vw>(out + at, v);
}

// src/common/probability.cpp:96-122
template <int V>
__global__ __launch_bounds__(256) void softmax_kernel(const uint16_t* x, int rows, uint16_t* out,
                                                      uint32_t* error)
{
    constexpr int width = wave * V;
    const int lane = threadIdx.x % wave;
    const int row = blockIdx.x * rows_per_block + threadIdx.x / wave;
    if (row >= rows)
    {
        return;
    }
    uint16_t v[V];
    load_row<V>(x + std::size_t(row) * width + lane * V, v);
    float maximum = -__builtin_inff();
    bool finite = true;
#pragma unroll
    for (int i = 0; i < V; ++i)
    {
        const float value = bf16_to_float(v[i]);
        finite = finite && is_finite(value);
        maximum = maximum < value ? value : maximum;
    }
    if (!finite)
    {
        error[0] = error_nonfinite;
    }
    maximum = group_max<wave>(maximum);
    float e[V], leaves[V];
#pragma unroll
    for (int i = 0; i < V; ++i)
    {
        const float shifted = bf16_to_float(v[i]) - maximum;
        e[i] = original_exp(shifted);
        leaves[i] = e[i];
    }
    const float total = row_sum<V>(leaves);
    const float reciprocal = 1.0f / total;
#pragma unroll
    for (int i = 0; i < V; ++i)
    {
        v[i] = float_to_bf16(e[i] * reciprocal);
    }
    store_row<V>(out + std::size_t(row) * width + lane * V, v);
}

__global__ void add_kernel(const uint16_t* a, const uint16_t* b, std::size_t count,
                           std::size_t width, std::size_t period, uint16_t* out)
{
    for (std::size_t i = blockIdx.x * std::size_t(blockDim.x) + threadIdx.x; i < count;
         i += std::size_t(gridDim.x) * blockDim.x)
    {
        const std::size_t row = i / width, column = i % width;
        const uint16_t right = b[(row % period) * width + column];
        out[i] = float_to_bf16(bf16_to_float(a[i]) + bf16_to_float(right));
    }
}

__global__ void gelu_kernel(const uint16_t* x, std::size_t count, uint16_t* out)
{
    for (std::size_t i = blockIdx.x * std::size_t(blockDim.x) + threadIdx.x; i < count;
         i += std::size_t(gridDim.x) * blockDim.x)
    {
        out[i] = gelu_bf16(x[i]);
    }
}

// src/common/probability.cpp:24-43 over (real, imaginary) pairs.
__global__ void rotary_kernel(const uint16_t* x, const uint16_t* c, std::size_t pairs,
                              uint16_t* out)
{
    for (std::size_t i = blockIdx.x * std::size_t(blockDim.x) + threadIdx.x; i < pairs;
         i += std::size_t(gridDim.x) * blockDim.x)
    {
        const float re = bf16_to_float(x[2 * i]), im = bf16_to_float(x[2 * i + 1]);
        const float cosine = bf16_to_float(c[2 * i]), sine = bf16_to_float(c[2 * i + 1]);
        const float im_sine = im * sine;
        const float re_sine = re * sine;
        out[2 * i] = float_to_bf16(__builtin_fmaf(re, cosine, -im_sine));
        out[2 * i + 1] = float_to_bf16(__builtin_fmaf(im, cosine, re_sine));
    }
}

unsigned grid_for(std::size_t count)
{
    const std::size_t blocks = (count + 255) / 256;
    return unsigned(blocks < 8192 ? (blocks ? blocks : 1) : 8192);
}
} // namespace

void layer_norm_rows(const uint16_t* x, std::size_t rows, std::size_t width, const uint16_t* gain,
                     const uint16_t* bias, uint16_t* out, hipStream_t stream)
{
    if (!rows)
    {
        return;
    }
    require(rows < (std::size_t(1) << 31), "too many rows");
    const dim3 grid(static_cast<unsigned>(rows));
    switch (width)
    {
    case 256:
        layer_norm_kernel<1, 4><<<grid, 256, 0, stream>>>(x, gain, bias, out);
        break;
    case 512:
        layer_norm_kernel<1, 8><<<grid, 512, 0, stream>>>(x, gain, bias, out);
        break;
    case 1024:
        layer_norm_kernel<2, 8><<<grid, 512, 0, stream>>>(x, gain, bias, out);
        break;
    case 2048:
        layer_norm_kernel<4, 8><<<grid, 512, 0, stream>>>(x, gain, bias, out);
        break;
    default:
        throw Error("layer norm: width must be one of 256, 512, 1024, 2048");
    }
    check_hip(hipGetLastError(), "layer norm launch");
}

void softmax_rows(const uint16_t* x, std::size_t rows, std::size_t width, uint16_t* out,
                  uint32_t* error, hipStream_t stream)
{
    if (!rows)
    {
        return;
    }
    require(rows < (std::size_t(1) << 31), "too many rows");
    const dim3 grid(unsigned((rows + rows_per_block - 1) / rows_per_block));
    switch (width)
    {
    case 256:
        softmax_kernel<4><<<grid, 256, 0, stream>>>(x, int(rows), out, error);
        break;
    case 512:
        softmax_kernel<8><<<grid, 256, 0, stream>>>(x, int(rows), out, error);
        break;
    case 1024:
        softmax_kernel<16><<<grid, 256, 0, stream>>>(x, int(rows), out, error);
        break;
    case 2048:
        softmax_kernel<32><<<grid, 256, 0, stream>>>(x, int(rows), out, error);
        break;
    default:
        throw Error("softmax: width must be one of 256, 512, 1024, 2048");
    }
    check_hip(hipGetLastError(), "softmax launch");
}

void add_rows(const uint16_t* a, const uint16_t* b, std::size_t rows, std::size_t width,
              std::size_t b_period, uint16_t* out, hipStream_t stream)
{
    require(width > 0 && b_period > 0, "add: empty shape");
    const std::size_t count = rows * width;
    if (!count)
    {
        return;
    }
    add_kernel<<<grid_for(count), 256, 0, stream>>>(a, b, count, width, b_period, out);
    check_hip(hipGetLastError(), "add launch");
}

void gelu_values(const uint16_t* x, std::size_t count, uint16_t* out, hipStream_t stream)
{
    if (!count)
    {
        return;
    }
    gelu_kernel<<<grid_for(count), 256, 0, stream>>>(x, count, out);
    check_hip(hipGetLastError(), "gelu launch");
}

void rotary_values(const uint16_t* x, const uint16_t* coefficients, std::size_t count,
                   uint16_t* out, hipStream_t stream)
{
    require(count % 2 == 0, "rotary pair shape mismatch");
    if (!count)
    {
        return;
    }
    rotary_kernel<<<grid_for(count / 2), 256, 0, stream>>>(x, coefficients, count / 2, out);
    check_hip(hipGetLastError(), "rotary launch");
}
} // namespace tsac_hip
