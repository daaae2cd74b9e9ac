// Row helpers for kernels where one 64-lane wavefront owns one row and lane l
// holds the V consecutive BF16 values [l*V, l*V+V).
#pragma once

#include "device_numeric.hpp"

namespace tsac_hip
{
__device__ __forceinline__ void wait_shared_memory()
{
    __builtin_amdgcn_s_waitcnt(0xc07f); // lgkmcnt(0)
}

// Workgroup barrier for hand-offs between a workgroup's waves through LDS.
// __syncthreads() would also wait for the wave's outstanding global loads and
// stores (s_waitcnt vmcnt(0)), such as weight prefetches and words just
// published; waiting for the wave's LDS accesses (lgkmcnt(0)) is all an LDS
// hand-off needs. The empty asm statements keep the compiler from moving
// memory accesses across it.
__device__ __forceinline__ void lds_barrier()
{
    asm volatile("" ::: "memory");
    wait_shared_memory();
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

template <int V> __device__ __forceinline__ void load_row(const uint16_t* p, uint16_t (&v)[V])
{
    if constexpr (V == 1)
    {
        v[0] = p[0];
    }
    else if constexpr (V == 2)
    {
        const uint32_t u = *reinterpret_cast<const uint32_t*>(p);
        v[0] = u & 0xffff, v[1] = u >> 16;
    }
    else if constexpr (V == 4)
    {
        const uint2 u = *reinterpret_cast<const uint2*>(p);
        v[0] = u.x & 0xffff, v[1] = u.x >> 16, v[2] = u.y & 0xffff, v[3] = u.y >> 16;
    }
    else
    {
#pragma unroll
        for (int c = 0; c < V / 8; ++c)
        {
            const uint4 u = reinterpret_cast<const uint4*>(p)[c];
            const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
            for (int i = 0; i < 4; ++i)
            {
                v[8 * c + 2 * i] = w[i] & 0xffff;
                v[8 * c + 2 * i + 1] = w[i] >> 16;
            }
        }
    }
}

template <int V> __device__ __forceinline__ void store_row(uint16_t* p, const uint16_t (&v)[V])
{
    if constexpr (V == 1)
    {
        p[0] = v[0];
    }
    else if constexpr (V == 2)
    {
        *reinterpret_cast<uint32_t*>(p) = v[0] | (uint32_t(v[1]) << 16);
    }
    else if constexpr (V == 4)
    {
        *reinterpret_cast<uint2*>(p) =
            make_uint2(v[0] | (uint32_t(v[1]) << 16), v[2] | (uint32_t(v[3]) << 16));
    }
    else
    {
#pragma unroll
        for (int c = 0; c < V / 8; ++c)
        {
            uint32_t w[4];
#pragma unroll
            for (int i = 0; i < 4; ++i)
            {
                w[i] = v[8 * c + 2 * i] | (uint32_t(v[8 * c + 2 * i + 1]) << 16);
            }
            reinterpret_cast<uint4*>(p)[c] = make_uint4(w[0], w[1], w[2], w[3]);
        }
    }
}

// The reference's probability_sum over a full row of 64*V leaves (V >= 2):
// the balanced pair tree equals its 64-block binary-carry merge, which ends
// with add(+0, S) (src/format/categorical.cpp:44-74).
template <int V> __device__ __forceinline__ float row_sum(float (&v)[V])
{
    static_assert(V >= 2, "rows of 64 or fewer values use the single-block tree");
    return flushed_add(0.0f, tree_sum<wave>(register_tree(v)));
}

// row_sum with plain additions, for leaves whose sums never meet a subnormal
// (see sums_stay_normal); then every flush of the FTZ tree is an identity and
// the two trees agree bit for bit.
template <int V> __device__ __forceinline__ float plain_row_sum(float (&v)[V])
{
    return 0.0f + plain_tree_sum<wave>(register_tree<V, false>(v));
}

// True (for the whole wave) when every value of the row is zero or at least
// 2^-56 in magnitude (BF16 magnitude bits 0 or >= 0x2380). Such a value is a
// multiple of 2^-63 and its square, exact in fp32, a multiple of 2^-126. Sums
// of multiples of 2^-k stay multiples of 2^-k after fp32 rounding, so every
// partial sum of values or of squares is zero or at least 2^-126: no leaf and
// no partial sum is subnormal, and FTZ and plain pair trees agree.
template <int V> __device__ __forceinline__ bool sums_stay_normal(const uint16_t (&v)[V])
{
    bool tiny = false;
#pragma unroll
    for (int i = 0; i < V; ++i)
    {
        tiny = tiny || (uint32_t(v[i]) & 0x7fffu) - 1u < 0x237fu;
    }
    return !__any(tiny);
}

// Largest magnitude of this lane's values as BF16 bits: on non-negative BF16
// patterns integer order is numeric order, and patterns from 0x7f80 up are
// not finite.
template <int V> __device__ __forceinline__ uint32_t bf8l_lane_top(const uint16_t (&v)[V])
{
    uint32_t top = 0;
#pragma unroll
    for (int i = 0; i < V; ++i)
    {
        const uint32_t magnitude = uint32_t(v[i]) & 0x7fffu;
        top = top < magnitude ? magnitude : top;
    }
    return top;
}

template <int V>
__device__ __forceinline__ uint16_t bf8l_with_top(const uint16_t (&v)[V], uint32_t top,
                                                  uint32_t (&packed)[(V + 3) / 4], uint32_t* error);

// BF8L quantisation of one row held V-per-lane (src/scalar/probability.cpp:20-38):
// packs this lane's V int8 values four to a word and returns the BF16 scale of
// its 256-value block. Sets error[0] when a value is not finite.
template <int V>
__device__ __forceinline__ uint16_t bf8l_pack(const uint16_t (&v)[V], uint32_t (&packed)[(V + 3) / 4],
                                              uint32_t* error)
{
    return bf8l_with_top<V>(v, group_umax<256 / V>(bf8l_lane_top<V>(v)), packed, error);
}

// The block's scale from its largest magnitude `top`, and this lane's values
// quantised with it.
template <int V>
__device__ __forceinline__ uint16_t bf8l_with_top(const uint16_t (&v)[V], uint32_t top,
                                                  uint32_t (&packed)[(V + 3) / 4], uint32_t* error)
{
    if (top >= 0x7f80u)
    {
        error[0] = 1u;
    }
    // The reference takes the largest flushed magnitude, which is the flushed
    // largest magnitude.
    const float maximum = top < 0x80u ? 0.0f : bf16_to_float(uint16_t(top));
    // ftz_divide(maximum, 127): a subnormal quotient would be flushed to +0,
    // and +0 and every subnormal alike are raised to the 1e-35 floor.
    float s = maximum / 127.0f;
    s = s < 1e-35f ? 1e-35f : s;
    const uint16_t scale = float_to_bf16(s);
    // 1e-35 <= scale <= 2^128/127: operand and quotient are normal, so the
    // flushes of ftz_divide(1, scale) are identities.
    const float reciprocal = 1.0f / bf16_to_float(scale);
#pragma unroll
    for (int i = 0; i < (V + 3) / 4; ++i)
    {
        packed[i] = 0;
    }
#pragma unroll
    for (int i = 0; i < V; ++i)
    {
        // rint(ftz_multiply(value, reciprocal)): with reciprocal <= 2^117 a
        // subnormal value gives a product below 2^-9 and a subnormal product
        // is below 2^-126, so with or without the flushes these round to a
        // signed zero and store 0.
        float r = __builtin_rintf(bf16_to_float(v[i]) * reciprocal);
        r = __builtin_fminf(__builtin_fmaxf(r, -128.0f), 127.0f);
        packed[i / 4] |= (uint32_t(int(r)) & 0xffu) << (8 * (i % 4));
    }
    return scale;
}

// BF8L of one row into row-major storage: q_row/s_row are the row's int8
// values [K] and block scales [K/256] (fp32, widened BF16).
template <int V>
__device__ __forceinline__ void bf8l_lane(const uint16_t (&v)[V], int lane, int8_t* q_row,
                                          float* s_row, uint32_t* error)
{
    constexpr int lanes_per_block = 256 / V;
    uint32_t packed[(V + 3) / 4];
    const uint16_t scale = bf8l_pack<V>(v, packed, error);
    int8_t* q = q_row + lane * V;
    if constexpr (V == 4)
    {
        *reinterpret_cast<uint32_t*>(q) = packed[0];
    }
    else
    {
#pragma unroll
        for (int c = 0; c < V / 8; ++c)
        {
            *reinterpret_cast<uint2*>(q + 8 * c) = make_uint2(packed[2 * c], packed[2 * c + 1]);
        }
    }
    if (lane % lanes_per_block == 0)
    {
        s_row[lane / lanes_per_block] = bf16_to_float(scale);
    }
}

// BF8L of row `row` into MFMA operand tiles. Byte k of row m lives at
//   ((m/32)*(K/32) + k/32)*1024 + ((m%32) + 32*((k/16)%2))*16 + k%16,
// so each block of 32 rows x 32 bytes is 1 KiB in the lane order of the int8
// MFMA's 16-byte operand (lane = row + 32*half). Block scales are stored
// transposed, scales[b*padded_rows + m], so a run of rows is contiguous.
template <int V>
__device__ __forceinline__ void bf8l_tiles(const uint16_t (&v)[V], int lane, std::size_t row,
                                           int8_t* q, float* scales, std::size_t padded_rows,
                                           uint32_t* error)
{
    constexpr int K = 64 * V, lanes_per_block = 256 / V;
    uint32_t packed[(V + 3) / 4];
    const uint16_t scale = bf8l_pack<V>(v, packed, error);
    int8_t* base = q + (row / 32) * (K / 32) * 1024 + (row % 32) * 16;
    const auto at = [&](int k) { return base + (k / 32) * 1024 + ((k / 16) % 2) * 512 + k % 16; };
    if constexpr (V == 4)
    {
        *reinterpret_cast<uint32_t*>(at(lane * V)) = packed[0];
    }
    else
    {
#pragma unroll
        for (int c = 0; c < V / 8; ++c)
        {
            *reinterpret_cast<uint2*>(at(lane * V + 8 * c)) = make_uint2(packed[2 * c], packed[2 * c + 1]);
        }
    }
    if (lane % lanes_per_block == 0)
    {
        scales[std::size_t(lane / lanes_per_block) * padded_rows + row] = bf16_to_float(scale);
    }
}

// LayerNorm of one row (src/common/probability.cpp:138-169), in place, with
// this lane's gain and bias values already loaded.
template <int V>
__device__ __forceinline__ void layer_norm_values(uint16_t (&v)[V], const uint16_t (&g)[V],
                                                  const uint16_t (&b)[V])
{
    float values[V], squares[V], x[V];
#pragma unroll
    for (int i = 0; i < V; ++i)
    {
        x[i] = bf16_to_float(v[i]);
        values[i] = x[i];
        squares[i] = x[i] * x[i];
    }
    constexpr int width = wave * V;
    float sum, sum_squares;
    if (sums_stay_normal<V>(v))
    {
        sum = plain_row_sum<V>(values);
        sum_squares = plain_row_sum<V>(squares);
    }
    else
    {
        sum = row_sum<V>(values);
        sum_squares = row_sum<V>(squares);
    }
    const float reciprocal = 1.0f / float(width);
    const float mean = sum * reciprocal;
    float variance = __builtin_fmaf(sum_squares, reciprocal, 0.0f);
    variance = __builtin_fmaf(mean, -mean, variance);
    variance += 1e-5f;
    const float inverse = 1.0f / __builtin_sqrtf(variance);
    const float offset = -mean * inverse;
#pragma unroll
    for (int i = 0; i < V; ++i)
    {
        const float normalized = __builtin_fmaf(x[i], inverse, offset);
        v[i] = float_to_bf16(__builtin_fmaf(normalized, bf16_to_float(g[i]), bf16_to_float(b[i])));
    }
}

// LayerNorm of one row (src/common/probability.cpp:138-169), in place.
template <int V>
__device__ __forceinline__ void layer_norm_lane(uint16_t (&v)[V], const uint16_t* gain,
                                                const uint16_t* bias, int lane)
{
    uint16_t g[V], b[V];
    load_row<V>(gain + lane * V, g);
    load_row<V>(bias + lane * V, b);
    layer_norm_values<V>(v, g, b);
}

// ---- rows spread over a workgroup ----------------------------------------------
// A row of K = Waves*64*Vw values held by the Waves wavefronts of a workgroup:
// wave w holds the 64*Vw consecutive values from w*64*Vw, and lane l of it the
// Vw consecutive values from (w*64 + l)*Vw. Leaves are in row order, so each
// wave's in-lane and cross-lane trees are the reference's pair tree over its
// part of the row, and the waves' results join as the tree's top levels. Every
// wave of the workgroup calls these helpers (they contain barriers).

// FTZ pair tree over `count` (a power of two) flushed values.
template <int count> __device__ __forceinline__ float flushed_tree(float (&t)[count])
{
#pragma unroll
    for (int width = count; width > 1; width /= 2)
    {
#pragma unroll
        for (int i = 0; i < width / 2; ++i)
        {
            t[i] = flushed_add(t[2 * i], t[2 * i + 1]);
        }
    }
    return t[0];
}

// LayerNorm of a spread row, in place; `exchange` is 2*Waves floats of LDS.
// A wave whose values are all zero or at least 2^-56 in magnitude sums its part
// with plain additions: every partial sum inside its subtree is then zero or at
// least 2^-126 (sums_stay_normal), so the FTZ tree's flushes are identities
// there. The waves' sums always join with FTZ additions, as the reference's
// tree does, whatever the other waves' parts hold.
template <int Vw, int Waves>
__device__ __forceinline__ void layer_norm_spread(uint16_t (&v)[Vw], const uint16_t (&g)[Vw], const uint16_t (&b)[Vw],
                                                  int warp, float* exchange)
{
    float values[Vw], squares[Vw], x[Vw];
#pragma unroll
    for (int i = 0; i < Vw; ++i)
    {
        x[i] = bf16_to_float(v[i]);
        values[i] = x[i];
        squares[i] = x[i] * x[i];
    }
    float sum, sum_squares;
    if (sums_stay_normal<Vw>(v))
    {
        sum = register_tree<Vw, false>(values);
        sum_squares = register_tree<Vw, false>(squares);
        tree_levels2<wave, false>(sum, sum_squares);
    }
    else
    {
        sum = flush(register_tree<Vw>(values));
        sum_squares = flush(register_tree<Vw>(squares));
        tree_levels2<wave, true>(sum, sum_squares);
    }
    if constexpr (Waves > 1)
    {
        if (threadIdx.x % wave == 0)
        {
            exchange[warp] = sum;
            exchange[Waves + warp] = sum_squares;
        }
        lds_barrier();
        float sums[Waves], square_sums[Waves];
#pragma unroll
        for (int w = 0; w < Waves; ++w)
        {
            sums[w] = exchange[w];
            square_sums[w] = exchange[Waves + w];
        }
        sum = flushed_tree<Waves>(sums);
        sum_squares = flushed_tree<Waves>(square_sums);
    }
    // The row's probability_sum ends with add(+0, S) (src/format/categorical.cpp:44-74).
    sum = flushed_add(0.0f, sum);
    sum_squares = flushed_add(0.0f, sum_squares);
    constexpr int width = Waves * wave * Vw;
    const float reciprocal = 1.0f / float(width);
    const float mean = sum * reciprocal;
    float variance = __builtin_fmaf(sum_squares, reciprocal, 0.0f);
    variance = __builtin_fmaf(mean, -mean, variance);
    variance += 1e-5f;
    const float inverse = 1.0f / __builtin_sqrtf(variance);
    const float offset = -mean * inverse;
#pragma unroll
    for (int i = 0; i < Vw; ++i)
    {
        const float normalized = __builtin_fmaf(x[i], inverse, offset);
        v[i] = float_to_bf16(__builtin_fmaf(normalized, bf16_to_float(g[i]), bf16_to_float(b[i])));
    }
}

// BF8L of a spread row into row-major storage (q_row [K], s_row [K/256]);
// `exchange` is Waves words of LDS, used when a 256-value block spans waves.
template <int Vw, int Waves>
__device__ __forceinline__ void bf8l_spread(const uint16_t (&v)[Vw], int warp, int8_t* q_row, float* s_row,
                                            uint32_t* error, uint32_t* exchange)
{
    constexpr int block_lanes = 256 / Vw; // lanes holding one 256-value block
    const int lane = threadIdx.x % wave, position = warp * wave + lane;
    uint32_t top = bf8l_lane_top<Vw>(v);
    if constexpr (block_lanes <= wave)
    {
        top = group_umax<block_lanes>(top);
    }
    else
    {
        constexpr int block_waves = block_lanes / wave;
        top = group_umax<wave>(top);
        if (lane == 0)
        {
            exchange[warp] = top;
        }
        lds_barrier();
        const int first = warp / block_waves * block_waves;
        top = 0;
#pragma unroll
        for (int i = 0; i < block_waves; ++i)
        {
            const uint32_t t = exchange[first + i];
            top = top < t ? t : top;
        }
    }
    uint32_t packed[(Vw + 3) / 4];
    const uint16_t scale = bf8l_with_top<Vw>(v, top, packed, error);
    int8_t* q = q_row + position * Vw;
    if constexpr (Vw == 1)
    {
        *q = int8_t(packed[0] & 0xffu);
    }
    else if constexpr (Vw == 2)
    {
        *reinterpret_cast<uint16_t*>(q) = uint16_t(packed[0] & 0xffffu);
    }
    else if constexpr (Vw == 4)
    {
        *reinterpret_cast<uint32_t*>(q) = packed[0];
    }
    else
    {
#pragma unroll
        for (int c = 0; c < Vw / 8; ++c)
        {
            *reinterpret_cast<uint2*>(q + 8 * c) = make_uint2(packed[2 * c], packed[2 * c + 1]);
        }
    }
    if (position % block_lanes == 0)
    {
        s_row[position / block_lanes] = bf16_to_float(scale);
    }
}
} // namespace tsac_hip
