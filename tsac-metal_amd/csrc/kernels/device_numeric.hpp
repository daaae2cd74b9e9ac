// Device-side arithmetic shared by every probability-model kernel.
//
// Each helper is one IEEE binary32 operation with round-to-nearest-even (the
// library is compiled with -ffp-contract=off and IEEE fp32 denormals), so a
// kernel that calls them in the reference's order reproduces the reference's
// bits. Flush-to-zero happens only where the reference flushes explicitly.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#pragma clang fp contract(off)

namespace tsac_hip
{
constexpr int wave = 64;

__device__ __forceinline__ float bf16_to_float(uint16_t h)
{
    return __uint_as_float(uint32_t(h) << 16);
}

// Integer ties-to-even without NaN canonicalisation (src/common/numeric/bf16.hpp:9-13).
__device__ __forceinline__ uint16_t float_to_bf16(float x)
{
    const uint32_t b = __float_as_uint(x);
    return uint16_t((b + 0x7fffu + ((b >> 16) & 1u)) >> 16);
}

__device__ __forceinline__ float round_bf16(float x)
{
    return bf16_to_float(float_to_bf16(x));
}

// Zero exponent -> signed zero (src/common/numeric/float_math.hpp:33-37).
__device__ __forceinline__ float flush(float x)
{
    const uint32_t b = __float_as_uint(x);
    return (b & 0x7f800000u) == 0 ? __uint_as_float(b & 0x80000000u) : x;
}

__device__ __forceinline__ float ftz_add(float x, float y)
{
    return flush(flush(x) + flush(y));
}

__device__ __forceinline__ float ftz_multiply(float x, float y)
{
    return flush(flush(x) * flush(y));
}

__device__ __forceinline__ float ftz_divide(float x, float y)
{
    return flush(flush(x) / flush(y));
}

__device__ __forceinline__ bool is_finite(float x)
{
    return (__float_as_uint(x) & 0x7f800000u) != 0x7f800000u;
}

// The reference's polynomial exponential (src/common/numeric/probability.hpp:14-33).
__device__ __forceinline__ float original_exp(float z)
{
    z = 87.0f < z ? 87.0f : z;
    z = -88.0f > z ? -88.0f : z;
    const float exponent = z * 0x1.715476p+0f;
    const int32_t n = is_finite(exponent) ? int32_t(__builtin_rintf(exponent)) : int32_t(0x80000000u);
    z = __builtin_fmaf(float(n), -0x1.630000p-1f, z);
    z = __builtin_fmaf(float(n), 0x1.bd0106p-13f, z);
    float p = __builtin_fmaf(0x1.a01a02p-13f, z, 0x1.6c16c2p-10f);
    p = __builtin_fmaf(p, z, 0x1.111112p-7f);
    p = __builtin_fmaf(p, z, 0x1.555556p-5f);
    p = __builtin_fmaf(p, z, 0x1.555556p-3f);
    const float square = z * z;
    p = __builtin_fmaf(p, z, 0.5f);
    z = __builtin_fmaf(p, square, z);
    const float plus_one = z + 1.0f;
    return __uint_as_float(__float_as_uint(plus_one) + (uint32_t(n) << 23));
}

// tanh-GELU with the reference's rounding boundaries (src/common/probability.cpp:45-63).
__device__ __forceinline__ uint16_t gelu_bf16(uint16_t bits)
{
    const float x = bf16_to_float(bits);
    const float cubic = 0x1.2444f2p-5f * x;
    float z = __builtin_fmaf(cubic, x, 0x1.988454p-1f);
    z = z * x;
    const float half = x * 0.5f;
    z = z * -2.0f;
    const float e = original_exp(z);
    const float denominator = e + 1.0f;
    const float sigmoid = 2.0f / denominator;
    const float t = sigmoid - 1.0f;
    const float plus = t + 1.0f;
    return float_to_bf16(half * plus);
}

// ---- cross-lane helpers (64-wide wavefronts) -----------------------------------

__device__ __forceinline__ float lane_xor(float v, int mask)
{
    return __shfl_xor(v, mask, wave);
}

__device__ __forceinline__ int lane_xor(int v, int mask)
{
    return __shfl_xor(v, mask, wave);
}

// Balanced adjacent-pair FTZ tree across `lanes` consecutive lanes (power of two).
// Lane pairs at strides 1, 2, 4, ... combine neighbouring subtrees, so with each
// lane holding the tree of its own consecutive leaves the result is the
// reference's pair tree over all leaves (src/format/categorical.cpp:17-30).
// Every lane of the group receives the sum.
template <int lanes> __device__ __forceinline__ float tree_sum(float v)
{
#pragma unroll
    for (int stride = 1; stride < lanes; stride *= 2)
    {
        v = ftz_add(v, lane_xor(v, stride));
    }
    return v;
}

template <int lanes> __device__ __forceinline__ float group_max(float v)
{
#pragma unroll
    for (int stride = 1; stride < lanes; stride *= 2)
    {
        const float o = lane_xor(v, stride);
        v = v < o ? o : v;
    }
    return v;
}

template <int lanes> __device__ __forceinline__ int group_isum(int v)
{
#pragma unroll
    for (int stride = 1; stride < lanes; stride *= 2)
    {
        v += lane_xor(v, stride);
    }
    return v;
}

// Pair tree over `count` consecutive registers (count a power of two).
template <int count> __device__ __forceinline__ float register_tree(float (&v)[count])
{
#pragma unroll
    for (int width = count; width > 1; width /= 2)
    {
#pragma unroll
        for (int i = 0; i < width / 2; ++i)
        {
            v[i] = ftz_add(v[2 * i], v[2 * i + 1]);
        }
    }
    return v[0];
}
} // namespace tsac_hip
