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
// Zeros map to themselves, so only subnormals (class mask 0x90) change.
__device__ __forceinline__ float flush(float x)
{
    return __builtin_amdgcn_classf(x, 0x90) ? __uint_as_float(__float_as_uint(x) & 0x80000000u) : x;
}

__device__ __forceinline__ float ftz_add(float x, float y)
{
    return flush(flush(x) + flush(y));
}

// ftz_add for operands that are already flushed (flush is idempotent).
__device__ __forceinline__ float flushed_add(float x, float y)
{
    return flush(x + y);
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
// Every helper here must be called by a whole wave (all 64 lanes active).

// The value of lane (this lane ^ 1), through DPP rather than LDS.
__device__ __forceinline__ uint32_t lane_swap1(uint32_t v)
{
    return uint32_t(__builtin_amdgcn_mov_dpp(int(v), 0xb1, 0xf, 0xf, false)); // quad_perm:[1,0,3,2]
}

// One level of a butterfly: returns combine(a, b) where {a, b} are this lane's
// value and that of lane (this lane ^ stride), in either order, so `combine`
// must be commutative. Precondition: every aligned group of `stride` lanes
// holds one value, as at each level of a butterfly started from stride 1.
// Then any lane of the neighbouring group is as good as lane ^ stride, which
// lets the mirror DPP patterns stand in for xor 4 and 8 inside a row of 16
// lanes, and gfx950's permlane swaps exchange rows (16) and half-waves (32).
// No level passes through LDS.
template <int stride, class Combine> __device__ __forceinline__ uint32_t butterfly(uint32_t v, Combine combine)
{
    static_assert(stride >= 1 && stride <= 32 && (stride & (stride - 1)) == 0, "power of two below 64");
    const int x = int(v);
    if constexpr (stride == 1)
    {
        return combine(v, lane_swap1(v));
    }
    else if constexpr (stride == 2)
    {
        return combine(v, uint32_t(__builtin_amdgcn_mov_dpp(x, 0x4e, 0xf, 0xf, false))); // quad_perm:[2,3,0,1]
    }
    else if constexpr (stride == 4)
    {
        return combine(v, uint32_t(__builtin_amdgcn_mov_dpp(x, 0x141, 0xf, 0xf, false))); // row_half_mirror
    }
    else if constexpr (stride == 8)
    {
        return combine(v, uint32_t(__builtin_amdgcn_mov_dpp(x, 0x140, 0xf, 0xf, false))); // row_mirror
    }
    else if constexpr (stride == 16)
    {
        // Rows (r0, r1, r2, r3) in both operands -> (r0, r0, r2, r2) and (r1, r1, r3, r3).
        const auto p = __builtin_amdgcn_permlane16_swap(x, x, false, false);
        return combine(uint32_t(p[0]), uint32_t(p[1]));
    }
    else
    {
        // Halves (h0, h1) in both operands -> (h0, h0) and (h1, h1).
        const auto p = __builtin_amdgcn_permlane32_swap(x, x, false, false);
        return combine(uint32_t(p[0]), uint32_t(p[1]));
    }
}

// One butterfly level of FTZ sums; v must already be flushed (as every
// ftz_add result is).
template <int stride> __device__ __forceinline__ float butterfly_ftz_add(float v)
{
    return __uint_as_float(butterfly<stride>(__float_as_uint(v), [](uint32_t a, uint32_t b) {
        return __float_as_uint(flushed_add(__uint_as_float(a), __uint_as_float(b)));
    }));
}

template <int stride> __device__ __forceinline__ float butterfly_add(float v)
{
    return __uint_as_float(butterfly<stride>(__float_as_uint(v), [](uint32_t a, uint32_t b) {
        return __float_as_uint(__uint_as_float(a) + __uint_as_float(b));
    }));
}

// Balanced adjacent-pair tree across `lanes` consecutive lanes (power of two).
// Lane pairs at strides 1, 2, 4, ... combine neighbouring subtrees, so with each
// lane holding the tree of its own consecutive leaves the result is the
// reference's pair tree over all leaves (src/format/categorical.cpp:17-30).
// IEEE addition is commutative, so the order inside a pair is immaterial.
// Every lane of the group receives the sum. Ftz selects FTZ additions; plain
// additions are for operands whose sums provably never meet a subnormal.
template <int lanes, bool Ftz, int stride> __device__ __forceinline__ float tree_levels(float v)
{
    if constexpr (stride >= lanes)
    {
        return v;
    }
    else if constexpr (Ftz)
    {
        return tree_levels<lanes, Ftz, 2 * stride>(butterfly_ftz_add<stride>(v));
    }
    else
    {
        return tree_levels<lanes, Ftz, 2 * stride>(butterfly_add<stride>(v));
    }
}

// Two independent pair trees, level by level, so that their dependency
// chains interleave.
template <int lanes, bool Ftz, int stride = 1> __device__ __forceinline__ void tree_levels2(float& a, float& b)
{
    if constexpr (stride < lanes)
    {
        if constexpr (Ftz)
        {
            a = butterfly_ftz_add<stride>(a);
            b = butterfly_ftz_add<stride>(b);
        }
        else
        {
            a = butterfly_add<stride>(a);
            b = butterfly_add<stride>(b);
        }
        tree_levels2<lanes, Ftz, 2 * stride>(a, b);
    }
}

template <int lanes> __device__ __forceinline__ float tree_sum(float v)
{
    return tree_levels<lanes, true, 1>(flush(v));
}

template <int lanes> __device__ __forceinline__ float plain_tree_sum(float v)
{
    return tree_levels<lanes, false, 1>(v);
}

// The lane's value, or -inf where DPP control Ctrl gives it no source lane
// (or its row or bank is masked out).
template <int Ctrl, int RowMask = 0xf, int BankMask = 0xf> __device__ __forceinline__ float dpp_or_minus_inf(float v)
{
    return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(-__builtin_inff()), __float_as_int(v), Ctrl,
                                                      RowMask, BankMask, false));
}

// Inclusive scan of the running maximum over the wave's lanes with the merge
// recurrence's own update (an earlier value stays unless it is smaller), on
// DPP row shifts and row broadcasts: within each row of 16 lanes by shifts of
// 1, 2, 4 and 8, then lane 15 into rows 1 and 3, then lane 31 into rows 2 and
// 3. Associative for values without NaN.
__device__ __forceinline__ float running_max_scan(float x)
{
    const auto keep = [](float earlier, float later) { return earlier < later ? later : earlier; };
    x = keep(dpp_or_minus_inf<0x111>(x), x);
    x = keep(dpp_or_minus_inf<0x112>(x), x);
    x = keep(dpp_or_minus_inf<0x114>(x), x);
    x = keep(dpp_or_minus_inf<0x118>(x), x);
    x = keep(dpp_or_minus_inf<0x142, 0xa>(x), x);
    x = keep(dpp_or_minus_inf<0x143, 0xc>(x), x);
    return x;
}

// The previous lane's value (wave shift right by one); lane 0 gets `first`.
__device__ __forceinline__ float previous_lane(float v, float first)
{
    return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(first), __float_as_int(v), 0x138, 0xf, 0xf, false));
}

// Largest value across the group. For values that compare equal but differ in
// bits (+0 and -0) a lane may receive either.
template <int lanes, int stride = 1> __device__ __forceinline__ float group_max(float v)
{
    if constexpr (stride >= lanes)
    {
        return v;
    }
    else
    {
        const uint32_t m = butterfly<stride>(__float_as_uint(v), [](uint32_t a, uint32_t b) {
            return __uint_as_float(a) < __uint_as_float(b) ? b : a;
        });
        return group_max<lanes, 2 * stride>(__uint_as_float(m));
    }
}

template <int lanes, int stride = 1> __device__ __forceinline__ int group_isum(int v)
{
    if constexpr (stride >= lanes)
    {
        return v;
    }
    else
    {
        const uint32_t s = butterfly<stride>(uint32_t(v), [](uint32_t a, uint32_t b) { return a + b; });
        return group_isum<lanes, 2 * stride>(int(s));
    }
}

// Pair tree over `count` consecutive registers (count a power of two), FTZ or
// plain as for tree_levels. The FTZ tree's result is flushed.
template <int count, bool Ftz = true> __device__ __forceinline__ float register_tree(float (&v)[count])
{
    if constexpr (Ftz)
    {
#pragma unroll
        for (int i = 0; i < count; ++i)
        {
            v[i] = flush(v[i]);
        }
    }
#pragma unroll
    for (int width = count; width > 1; width /= 2)
    {
#pragma unroll
        for (int i = 0; i < width / 2; ++i)
        {
            v[i] = Ftz ? flushed_add(v[2 * i], v[2 * i + 1]) : v[2 * i] + v[2 * i + 1];
        }
    }
    return v[0];
}

// Unsigned maximum across `lanes` consecutive lanes (power of two).
template <int lanes, int stride = 1> __device__ __forceinline__ uint32_t group_umax(uint32_t v)
{
    if constexpr (stride >= lanes)
    {
        return v;
    }
    else
    {
        return group_umax<lanes, 2 * stride>(butterfly<stride>(v, [](uint32_t a, uint32_t b) { return a < b ? b : a; }));
    }
}
} // namespace tsac_hip
