// W8A8 quantised linear: y = bf16(sum_b fma(dot_b, w_scale[b][n] * a_scale[m][b]) + bias[n]).
//
// The int8 dot of each 256-value block is exact in int32 (|dot| <= 256*128*128
// < 2^24), so any summation order inside a block gives the same integer; only
// the fp32 chain over blocks has a fixed order (ascending b, one fma each), as
// in src/scalar/packed_linear.cpp:16-27. Both paths below compute the exact
// block dots and then run that same chain, so GEMV and GEMM agree bit for bit
// with each other and with the reference.
//
// Weights live in HBM in "row tiles", laid out once at load time: 64 output rows
// x one 256-value block form a 16 KiB tile stored as [segment 0..15][row 0..63]
// [16 bytes], tiles ordered [N/64][K/256]. A wavefront load of one segment is
// then 1 KiB contiguous with lane l holding row l.
//
//  * GEMV (decode, M <= 8 columns): one workgroup per 64-row tile, one
//    wavefront per block; every lane accumulates its row's whole block dot with
//    v_dot4 against wave-uniform activations (no cross-lane reduction), then the
//    ordered chain runs per (row, column) from LDS.
//  * GEMM (encode, large M): 128x128 output tiles per 256-thread workgroup,
//    int8 MFMA 32x32x32 into int32 accumulators per 256-wide K block, LDS-staged
//    operand tiles, and the per-block fp32 fma epilogue into a second
//    accumulator set.
#include "device_numeric.hpp"
#include "kernels.hpp"

#include <cstring>

namespace tsac_hip
{
namespace
{
constexpr int tile_rows = 64;
constexpr int segments = 16; // 16-byte segments per 256-value block

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

// Byte offset of segment `s` of block `b` in row tile `t` (row 0 of the tile).
__device__ __forceinline__ std::size_t tile_offset(int t, int b, int s, int blocks)
{
    return ((std::size_t(t) * blocks + b) * segments + s) * (tile_rows * 16);
}

// ------------------------------------------------------------------ GEMV

constexpr int gemv_waves = 4;
constexpr int gemv_max_columns = 8;

template <int M>
__global__ __launch_bounds__(gemv_waves * wave) void gemv_kernel(
    const int8_t* __restrict__ weights, const float* __restrict__ weight_scales,
    const float* __restrict__ bias, int N, int K, const int8_t* __restrict__ q,
    const float* __restrict__ activation_scales, uint16_t* y, const uint16_t* residual)
{
    extern __shared__ int block_dots[]; // [blocks][M][64]
    const int blocks = K / 256;
    const int tile = blockIdx.x;
    const int lane = threadIdx.x % wave;
    const int warp = __builtin_amdgcn_readfirstlane(threadIdx.x / wave);
    for (int b = warp; b < blocks; b += gemv_waves)
    {
        uint4 w[segments];
        const int8_t* base = weights + tile_offset(tile, b, 0, blocks) + lane * 16;
#pragma unroll
        for (int s = 0; s < segments; ++s)
        {
            w[s] = *reinterpret_cast<const uint4*>(base + s * tile_rows * 16);
        }
        int dot[M];
#pragma unroll
        for (int m = 0; m < M; ++m)
        {
            dot[m] = 0;
            const uint4* a = reinterpret_cast<const uint4*>(q + std::size_t(m) * K + b * 256);
#pragma unroll
            for (int s = 0; s < segments; ++s)
            {
                const uint4 x = a[s];
                dot[m] = __builtin_amdgcn_sdot4(int(w[s].x), int(x.x), dot[m], false);
                dot[m] = __builtin_amdgcn_sdot4(int(w[s].y), int(x.y), dot[m], false);
                dot[m] = __builtin_amdgcn_sdot4(int(w[s].z), int(x.z), dot[m], false);
                dot[m] = __builtin_amdgcn_sdot4(int(w[s].w), int(x.w), dot[m], false);
            }
            block_dots[(b * M + m) * tile_rows + lane] = dot[m];
        }
    }
    __syncthreads();
    // Ordered chain per (row, column): ascending blocks, one fma each.
    for (int pair = threadIdx.x; pair < M * tile_rows; pair += blockDim.x)
    {
        const int m = pair / tile_rows, row = pair % tile_rows;
        const int n = tile * tile_rows + row;
        float sum = 0.0f;
        for (int b = 0; b < blocks; ++b)
        {
            const float scale = weight_scales[std::size_t(b) * N + n] * activation_scales[m * blocks + b];
            sum = __builtin_fmaf(float(block_dots[(b * M + m) * tile_rows + row]), scale, sum);
        }
        const std::size_t index = std::size_t(m) * N + n;
        y[index] = finish(sum, bias[n], residual, index);
    }
}

void launch_gemv(const DeviceLinear& w, const int8_t* q, const float* scales, std::size_t M,
                 uint16_t* y, const uint16_t* residual, hipStream_t stream)
{
    const unsigned grid = unsigned(w.N / tile_rows);
    const std::size_t lds = (w.K / 256) * M * tile_rows * sizeof(int);
    const int N = int(w.N), K = int(w.K);
#define TSAC_GEMV(MM)                                                                              \
    case MM:                                                                                       \
        gemv_kernel<MM><<<grid, gemv_waves * wave, lds, stream>>>(w.values, w.scales, w.bias, N, K, \
                                                                  q, scales, y, residual);        \
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
    const int row_tiles = N / tile_rows;

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
        const int block = k0 / 256, first_segment = (k0 % 256) / 16;
        // Global -> registers: 128 rows x 128 bytes per operand, 4 x 16 B per thread.
        uint4 ra[4], rb[4];
#pragma unroll
        for (int it = 0; it < 4; ++it)
        {
            const int index = it * 256 + tid, row = index / 8, chunk = index % 8;
            const int m = m0 + row;
            ra[it] = m < M ? *reinterpret_cast<const uint4*>(q + std::size_t(m) * K + k0 + chunk * 16)
                           : make_uint4(0, 0, 0, 0);
            // Weights: 2 row tiles x 8 segments, each a contiguous 1 KiB.
            const int c = index / 64, t = n0 / tile_rows + c / 8;
            rb[it] = t < row_tiles
                         ? *reinterpret_cast<const uint4*>(
                               weights + tile_offset(t, block, first_segment + c % 8, blocks) + (index % 64) * 16)
                         : make_uint4(0, 0, 0, 0);
        }
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
            const int c = index / 64;
            *reinterpret_cast<uint4*>(b_tile + ((c / 8) * tile_rows + index % 64) * lds_stride + (c % 8) * 16) =
                rb[it];
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

void tile_weights(const int8_t* canonical, std::size_t K, std::size_t N, int8_t* tiled)
{
    require(K % 256 == 0 && N % tile_rows == 0, "weights: K must be a multiple of 256, N of 64");
    const std::size_t blocks = K / 256;
    for (std::size_t n = 0; n < N; ++n)
    {
        const std::size_t t = n / tile_rows, lane = n % tile_rows;
        for (std::size_t b = 0; b < blocks; ++b)
        {
            for (std::size_t s = 0; s < segments; ++s)
            {
                std::memcpy(tiled + ((t * blocks + b) * segments + s) * tile_rows * 16 + lane * 16,
                            canonical + n * K + b * 256 + s * 16, 16);
            }
        }
    }
}

void linear(const DeviceLinear& w, const int8_t* q, const float* scales, std::size_t M,
            uint16_t* y, const uint16_t* residual, LinearPath path, hipStream_t stream)
{
    require(w.K >= 256 && w.K % 256 == 0 && w.K <= 4096, "linear: K must be a multiple of 256 <= 4096");
    require(w.N > 0 && w.N % tile_rows == 0 && w.N < (std::size_t(1) << 30),
            "linear: N must be a multiple of 64");
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
        launch_gemv(w, q, scales, M, y, residual, stream);
    }
    else
    {
        launch_gemm(w, q, scales, M, y, residual, stream);
    }
    check_hip(hipGetLastError(), "linear launch");
}
} // namespace tsac_hip
