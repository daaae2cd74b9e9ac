// Device helpers shared by the decode-side kernels: row-tile addressing, the
// rotary pair rotation, conditional_q15 and the categorical subtree masses.
#pragma once

#include "device_numeric.hpp"
#include "row_ops.hpp"

#include <cstddef>

namespace tsac_hip
{
namespace step
{
constexpr int tile_rows = 64;
constexpr int segments = 16;
constexpr int max_columns = 8;

__device__ __forceinline__ std::size_t tile_offset(int t, int b, int s, int blocks)
{
    return ((std::size_t(t) * blocks + b) * segments + s) * (tile_rows * 16);
}

__device__ __forceinline__ void rotate(float& re, float& im, const uint16_t* c)
{
    const float cosine = bf16_to_float(c[0]), sine = bf16_to_float(c[1]);
    const float im_sine = im * sine;
    const float re_sine = re * sine;
    const float r = __builtin_fmaf(re, cosine, -im_sine);
    const float i = __builtin_fmaf(im, cosine, re_sine);
    re = bf16_to_float(float_to_bf16(r));
    im = bf16_to_float(float_to_bf16(i));
}

// conditional_q15 (src/format/categorical.cpp:76-89).
__device__ __forceinline__ uint16_t q15(float left, float mass)
{
    const float value = ftz_divide(ftz_multiply(left, 32768.0f), mass);
    if (!is_finite(value) || value >= 0x1p63f || value < -0x1p63f)
    {
        return 1;
    }
    const long long integer = static_cast<long long>(__builtin_rintf(value));
    const int low = int(uint32_t(uint64_t(integer)));
    return uint16_t(low < 1 ? 1 : (low > 32767 ? 32767 : low));
}

// Heap-ordered subtree masses of one 1024-symbol row held 16 per lane, into
// nodes[1..1023] (shared memory).
__device__ __forceinline__ bool build_masses(const float (&leaf)[16], int lane, float* nodes)
{
    bool valid = true;
#pragma unroll
    for (int i = 0; i < 16; ++i)
    {
        valid = valid && is_finite(leaf[i]) && leaf[i] >= 0.0f;
    }
    float level[8];
#pragma unroll
    for (int i = 0; i < 8; ++i)
    {
        level[i] = ftz_add(leaf[2 * i], leaf[2 * i + 1]);
        nodes[512 + lane * 8 + i] = level[i];
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
    {
        level[i] = ftz_add(level[2 * i], level[2 * i + 1]);
        nodes[256 + lane * 4 + i] = level[i];
    }
#pragma unroll
    for (int i = 0; i < 2; ++i)
    {
        level[i] = ftz_add(level[2 * i], level[2 * i + 1]);
        nodes[128 + lane * 2 + i] = level[i];
    }
    float v = ftz_add(level[0], level[1]);
    nodes[64 + lane] = v;
    // Level l spans 32 << l leaves (2 << l lanes); one lane per node stores it.
    const auto store = [&](int l) {
        const int size = 32 << l;
        if ((lane * 16) % size == 0)
        {
            nodes[1024 / size + lane * 16 / size] = v;
        }
    };
    v = butterfly_ftz_add<1>(v);
    store(0);
    v = butterfly_ftz_add<2>(v);
    store(1);
    v = butterfly_ftz_add<4>(v);
    store(2);
    v = butterfly_ftz_add<8>(v);
    store(3);
    v = butterfly_ftz_add<16>(v);
    store(4);
    v = butterfly_ftz_add<32>(v);
    store(5);
    return __all(valid);
}

} // namespace step
} // namespace tsac_hip
