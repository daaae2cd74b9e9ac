// W8A8 quantised linear: y = bf16(sum_b fma(dot_b, w_scale[b][n] * a_scale[m][b]) + bias[n]).
//
// The int8 dot of each 256-value block is exact in int32 (|dot| <= 256*128*128
// < 2^24), so any summation order inside a block gives the same integer; only
// the fp32 chain over blocks has a fixed order (ascending b, one fma each), as
// in src/scalar/packed_linear.cpp:16-27. Both paths below compute the exact
// block dots and then run that same chain, so GEMV and GEMM agree bit for bit
// with each other and with the reference.
//
//  * GEMV (decode, M <= 8 columns): one wavefront streams a group of weight rows
//    as contiguous 1 KiB loads, v_dot4 against activations staged in LDS, exact
//    16-lane integer reductions, then the ordered chain.
//  * GEMM (encode, large M): 128x128 tiles per 256-thread workgroup, int8 MFMA
//    32x32x32 into int32 accumulators per 256-wide K block, LDS-staged operand
//    tiles, and the per-block fp32 fma epilogue into a second accumulator set.
#include "device_numeric.hpp"
#include "kernels.hpp"

namespace tsac_hip
{
namespace
{
// ------------------------------------------------------------------ epilogue

__device__ __forceinline__ uint16_t finish(float sum, float bias, const uint16_t* residual,
                                           std::size_t index)
{
    const uint16_t y = float_to_bf16(sum + bias);
    if (residual)
    {
        return float_to_bf16(bf16_to_float(residual[index]) + bf16_to_float(y));
    }
    return y;
}

// ------------------------------------------------------------------ GEMV

constexpr int gemv_waves = 4;
constexpr int gemv_unroll = 4;
constexpr int gemv_max_columns = 8;

__device__ __forceinline__ int dot16(uint4 w, uint4 a, int acc)
{
    acc = __builtin_amdgcn_sdot4(int(w.x), int(a.x), acc, false);
    acc = __builtin_amdgcn_sdot4(int(w.y), int(a.y), acc, false);
    acc = __builtin_amdgcn_sdot4(int(w.z), int(a.z), acc, false);
    acc = __builtin_amdgcn_sdot4(int(w.w), int(a.w), acc, false);
    return acc;
}

// K: input width. G = rows per wave group (1 KiB of weights for K <= 1024).
// J = 16-byte segments per lane per group. M = activation columns.
template <int K, int M>
__global__ __launch_bounds__(gemv_waves * wave) void gemv_kernel(
    const int8_t* __restrict__ weights, const float* __restrict__ weight_scales,
    const float* __restrict__ bias, int N, const int8_t* __restrict__ q,
    const float* __restrict__ activation_scales, uint16_t* y, const uint16_t* residual)
{
    constexpr int G = K >= 1024 ? 1 : 1024 / K;
    constexpr int J = G * K / 1024;
    constexpr int blocks = K / 256;
    constexpr int segments_per_row = K / 16;
    __shared__ uint4 staged[M * K / 16];
    for (int i = threadIdx.x; i < M * K / 16; i += blockDim.x)
    {
        staged[i] = reinterpret_cast<const uint4*>(q)[i];
    }
    __syncthreads();

    const int lane = threadIdx.x % wave;
    const int groups = N / G;
    const int total_waves = gridDim.x * gemv_waves;
    for (int first = blockIdx.x * gemv_waves + threadIdx.x / wave; first < groups;
         first += total_waves * gemv_unroll)
    {
        // Issue every weight load of this iteration before any arithmetic.
        uint4 w[gemv_unroll][J];
#pragma unroll
        for (int u = 0; u < gemv_unroll; ++u)
        {
            const int group = first + u * total_waves;
            const int g = group < groups ? group : groups - 1;
#pragma unroll
            for (int j = 0; j < J; ++j)
            {
                w[u][j] = reinterpret_cast<const uint4*>(weights + std::size_t(g) * G * K +
                                                         j * 1024)[lane];
            }
        }
#pragma unroll
        for (int u = 0; u < gemv_unroll; ++u)
        {
            const int group = first + u * total_waves;
            if (group >= groups)
            {
                break;
            }
            int dots[J][M];
#pragma unroll
            for (int j = 0; j < J; ++j)
            {
                const int segment = j * wave + lane;
                const int k16 = segment % segments_per_row;
#pragma unroll
                for (int m = 0; m < M; ++m)
                {
                    dots[j][m] = group_isum<16>(dot16(w[u][j], staged[m * segments_per_row + k16], 0));
                }
            }
            // Ordered per-block chain; every lane computes it, lane r*M+m stores.
            uint16_t out = 0;
#pragma unroll
            for (int r = 0; r < G; ++r)
            {
                const int n = group * G + r;
#pragma unroll
                for (int m = 0; m < M; ++m)
                {
                    float sum = 0.0f;
#pragma unroll
                    for (int b = 0; b < blocks; ++b)
                    {
                        const int segment = r * segments_per_row + 16 * b;
                        const int dot = __shfl(dots[segment / wave][m], segment % wave, wave);
                        const float scale = weight_scales[b * N + n] * activation_scales[m * blocks + b];
                        sum = __builtin_fmaf(float(dot), scale, sum);
                    }
                    if (lane == r * M + m)
                    {
                        out = finish(sum, bias[n], residual, std::size_t(m) * N + n);
                    }
                }
            }
            if (lane < G * M)
            {
                const int r = lane / M, m = lane % M;
                y[std::size_t(m) * N + group * G + r] = out;
            }
        }
    }
}

template <int K>
void launch_gemv_k(const DeviceLinear& w, const int8_t* q, const float* scales, std::size_t M,
                   uint16_t* y, const uint16_t* residual, hipStream_t stream)
{
    constexpr int G = K >= 1024 ? 1 : 1024 / K;
    const std::size_t groups = w.N / G;
    const std::size_t wanted = (groups + gemv_waves - 1) / gemv_waves;
    const unsigned grid = unsigned(wanted < 2048 ? wanted : 2048);
    const int N = int(w.N);
#define TSAC_GEMV(MM)                                                                              \
    case MM:                                                                                       \
        gemv_kernel<K, MM><<<grid, gemv_waves * wave, 0, stream>>>(w.values, w.scales, w.bias, N,  \
                                                                   q, scales, y, residual);       \
        break;
    switch (M)
    {
        TSAC_GEMV(1)
        TSAC_GEMV(2)
        TSAC_GEMV(3)
        TSAC_GEMV(4)
        TSAC_GEMV(5)
        TSAC_GEMV(6)
        TSAC_GEMV(7)
        TSAC_GEMV(8)
    default:
        throw Error("gemv: column count out of range");
    }
#undef TSAC_GEMV
}

void launch_gemv(const DeviceLinear& w, const int8_t* q, const float* scales, std::size_t M,
                 uint16_t* y, const uint16_t* residual, hipStream_t stream)
{
    switch (w.K)
    {
    case 256:
        launch_gemv_k<256>(w, q, scales, M, y, residual, stream);
        break;
    case 512:
        launch_gemv_k<512>(w, q, scales, M, y, residual, stream);
        break;
    case 1024:
        launch_gemv_k<1024>(w, q, scales, M, y, residual, stream);
        break;
    case 2048:
        launch_gemv_k<2048>(w, q, scales, M, y, residual, stream);
        break;
    case 4096:
        launch_gemv_k<4096>(w, q, scales, M, y, residual, stream);
        break;
    default:
        throw Error("gemv: K must be one of 256, 512, 1024, 2048, 4096");
    }
}

// ------------------------------------------------------------------ GEMM (MFMA)

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

constexpr int tile_m = 128, tile_n = 128, stage_k = 128, lds_stride = stage_k + 16;

__global__ __launch_bounds__(256) void gemm_kernel(
    const int8_t* __restrict__ weights, const float* __restrict__ weight_scales,
    const float* __restrict__ bias, int N, int K, const int8_t* __restrict__ q,
    const float* __restrict__ activation_scales, int M, uint16_t* y, const uint16_t* residual)
{
    __shared__ __attribute__((aligned(16))) int8_t a_tile[tile_m * lds_stride];
    __shared__ __attribute__((aligned(16))) int8_t b_tile[tile_n * lds_stride];
    __shared__ float a_scale[tile_m];
    __shared__ float w_scale[tile_n];

    const int tid = threadIdx.x, lane = tid % wave, warp = tid / wave;
    const int wm = warp / 2, wn = warp % 2;
    const int n0 = blockIdx.x * tile_n, m0 = blockIdx.y * tile_m;
    const int blocks = K / 256;

    v16i acc[2][2];
    float sum[2][2][16];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
        {
#pragma unroll
            for (int r = 0; r < 16; ++r)
            {
                acc[i][j][r] = 0;
                sum[i][j][r] = 0.0f;
            }
        }

    for (int k0 = 0; k0 < K; k0 += stage_k)
    {
        // Global -> registers: 128 rows x 128 bytes per operand, 4 x 16 B per thread.
        uint4 ra[4], rb[4];
#pragma unroll
        for (int it = 0; it < 4; ++it)
        {
            const int index = it * 256 + tid, row = index / 8, chunk = index % 8;
            const int m = m0 + row;
            ra[it] = m < M ? *reinterpret_cast<const uint4*>(q + std::size_t(m) * K + k0 + chunk * 16)
                           : make_uint4(0, 0, 0, 0);
            const int n = n0 + row;
            rb[it] = n < N ? *reinterpret_cast<const uint4*>(weights + std::size_t(n) * K + k0 +
                                                            chunk * 16)
                           : make_uint4(0, 0, 0, 0);
        }
        const int block = k0 / 256;
        const bool block_start = k0 % 256 == 0;
        float scale_value = 0.0f;
        if (block_start)
        {
            if (tid < tile_m)
            {
                const int m = m0 + tid;
                scale_value = m < M ? activation_scales[std::size_t(m) * blocks + block] : 0.0f;
            }
            else
            {
                const int n = n0 + tid - tile_m;
                scale_value = n < N ? weight_scales[std::size_t(block) * N + n] : 0.0f;
            }
        }
        __syncthreads();
#pragma unroll
        for (int it = 0; it < 4; ++it)
        {
            const int index = it * 256 + tid, row = index / 8, chunk = index % 8;
            *reinterpret_cast<uint4*>(a_tile + row * lds_stride + chunk * 16) = ra[it];
            *reinterpret_cast<uint4*>(b_tile + row * lds_stride + chunk * 16) = rb[it];
        }
        if (block_start)
        {
            if (tid < tile_m)
            {
                a_scale[tid] = scale_value;
            }
            else
            {
                w_scale[tid - tile_m] = scale_value;
            }
        }
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < stage_k; kk += 32)
        {
            v4i a[2], b[2];
            const int koff = kk + (lane / 32) * 16;
#pragma unroll
            for (int i = 0; i < 2; ++i)
            {
                a[i] = *reinterpret_cast<const v4i*>(a_tile + (wm * 64 + i * 32 + lane % 32) *
                                                                  lds_stride + koff);
                b[i] = *reinterpret_cast<const v4i*>(b_tile + (wn * 64 + i * 32 + lane % 32) *
                                                                  lds_stride + koff);
            }
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                {
                    acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[i], b[j], acc[i][j], 0, 0, 0);
                }
        }
        if ((k0 + stage_k) % 256 == 0)
        {
            // Block epilogue: one fp32 fma per output in ascending block order.
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                {
                    const float ws = w_scale[wn * 64 + j * 32 + lane % 32];
#pragma unroll
                    for (int r = 0; r < 16; ++r)
                    {
                        const int row = wm * 64 + i * 32 + 8 * (r / 4) + 4 * (lane / 32) + r % 4;
                        const float scale = ws * a_scale[row];
                        sum[i][j][r] = __builtin_fmaf(float(acc[i][j][r]), scale, sum[i][j][r]);
                        acc[i][j][r] = 0;
                    }
                }
        }
    }
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
        {
            const int n = n0 + wn * 64 + j * 32 + lane % 32;
            if (n >= N)
            {
                continue;
            }
            const float b = bias[n];
#pragma unroll
            for (int r = 0; r < 16; ++r)
            {
                const int m = m0 + wm * 64 + i * 32 + 8 * (r / 4) + 4 * (lane / 32) + r % 4;
                if (m < M)
                {
                    const std::size_t index = std::size_t(m) * N + n;
                    y[index] = finish(sum[i][j][r], b, residual, index);
                }
            }
        }
}

void launch_gemm(const DeviceLinear& w, const int8_t* q, const float* scales, std::size_t M,
                 uint16_t* y, const uint16_t* residual, hipStream_t stream)
{
    require(M < (std::size_t(1) << 30), "gemm: too many rows");
    const dim3 grid(unsigned((w.N + tile_n - 1) / tile_n), unsigned((M + tile_m - 1) / tile_m));
    gemm_kernel<<<grid, 256, 0, stream>>>(w.values, w.scales, w.bias, int(w.N), int(w.K), q, scales,
                                          int(M), y, residual);
}
} // namespace

std::size_t gemv_max_rows()
{
    return gemv_max_columns;
}

void linear(const DeviceLinear& w, const int8_t* q, const float* scales, std::size_t M,
            uint16_t* y, const uint16_t* residual, LinearPath path, hipStream_t stream)
{
    require(w.K >= 256 && w.K % 256 == 0 && w.K <= 4096, "linear: K must be a multiple of 256 <= 4096");
    require(w.N > 0 && w.N % 16 == 0 && w.N < (std::size_t(1) << 30), "linear: N must be a multiple of 16");
    if (M == 0)
    {
        return;
    }
    if (path == LinearPath::automatic)
    {
        path = M <= gemv_max_columns ? LinearPath::gemv : LinearPath::gemm;
    }
    if (path == LinearPath::gemv)
    {
        require(M <= gemv_max_columns, "gemv: at most 8 columns");
        const std::size_t G = w.K >= 1024 ? 1 : 1024 / w.K;
        require(w.N % G == 0, "gemv: N must be a multiple of the row group");
        launch_gemv(w, q, scales, M, y, residual, stream);
    }
    else
    {
        launch_gemm(w, q, scales, M, y, residual, stream);
    }
    check_hip(hipGetLastError(), "linear launch");
}
} // namespace tsac_hip
