// Causal multi-head attention with the reference's exact arithmetic
// (src/scalar/attention.cpp:12-131):
//   * scores: one serial fma chain over the head coordinates (ascending), times scale;
//   * keys in 64-position blocks: block max, original_exp(score - max), pair-tree
//     block sum, per-coordinate serial fma value sums (BF16-rounded when the
//     query's history exceeds 64 positions or during replay);
//   * blocks merged in ascending order with the online-softmax recurrence.
// Matrix cores would reorder those sums, so everything runs on the VALU.
//
// Decode (one query per sequence): one workgroup per (sequence, head) computes
// the block partials into LDS and merges them in order; histories beyond what
// its LDS holds use one wavefront per (sequence, head, block) and a second
// launch for the merge.
// Prefill (encode, all queries known): one workgroup per (sequence, head,
// 64-query tile) walks the causal key blocks with Q/K/V tiles in LDS.
#include "attention.hpp"
#include "device_numeric.hpp"

namespace tsac_hip
{
namespace
{
__device__ __forceinline__ void rotate_pair(float& re, float& im, const uint16_t* c)
{
    const float cosine = bf16_to_float(c[0]), sine = bf16_to_float(c[1]);
    const float im_sine = im * sine;
    const float re_sine = re * sine;
    const float r = __builtin_fmaf(re, cosine, -im_sine);
    const float i = __builtin_fmaf(im, cosine, re_sine);
    re = round_bf16(r);
    im = round_bf16(i);
}

// ------------------------------------------------------------------ decode

// Splits each row's Q, K and V out of the projection output, applies rotary to
// Q and K when a table is given, appends K and V to the caches at `position`.
__global__ void append_kernel(const uint16_t* __restrict__ qkv, int rows, int width, int head_width,
                              const uint16_t* __restrict__ rotation, uint16_t* __restrict__ query,
                              uint16_t* keys, uint16_t* values, std::size_t row_stride)
{
    const int pairs = width / 2;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < rows * pairs;
         i += gridDim.x * blockDim.x)
    {
        const int row = i / pairs, j = 2 * (i % pairs);
        const uint16_t* src = qkv + std::size_t(row) * 3 * width;
        float qr = bf16_to_float(src[j]), qi = bf16_to_float(src[j + 1]);
        float kr = bf16_to_float(src[width + j]), ki = bf16_to_float(src[width + j + 1]);
        if (rotation)
        {
            const uint16_t* c = rotation + j % head_width;
            rotate_pair(qr, qi, c);
            rotate_pair(kr, ki, c);
        }
        query[std::size_t(row) * width + j] = float_to_bf16(qr);
        query[std::size_t(row) * width + j + 1] = float_to_bf16(qi);
        uint16_t* k = keys + std::size_t(row) * row_stride;
        uint16_t* v = values + std::size_t(row) * row_stride;
        k[j] = float_to_bf16(kr);
        k[j + 1] = float_to_bf16(ki);
        v[j] = src[2 * width + j];
        v[j + 1] = src[2 * width + j + 1];
    }
}

// One wavefront per (sequence, head, 64-key block). Partial record layout:
// [max, block sum, value sums[head_width]].
template <int HW>
__global__ __launch_bounds__(64) void decode_blocks_kernel(
    const uint16_t* __restrict__ query, const uint16_t* __restrict__ keys,
    const uint16_t* __restrict__ values, std::size_t sequence_stride, int width, int time,
    int heads, float scale, int round_values, int max_blocks, float* __restrict__ partial)
{
    const int sequence = blockIdx.x / heads, head = blockIdx.x % heads;
    const int block = blockIdx.y;
    const int start = block * 64;
    if (start >= time)
    {
        return;
    }
    const int lane = threadIdx.x;
    const int count = time - start < 64 ? time - start : 64;
    const uint16_t* q = query + std::size_t(sequence) * width + head * HW;
    const uint16_t* k = keys + std::size_t(sequence) * sequence_stride + head * HW;
    const uint16_t* v = values + std::size_t(sequence) * sequence_stride + head * HW;
    __shared__ float qf[HW];
    __shared__ float weights[64];
    for (int j = lane; j < HW; j += 64)
    {
        qf[j] = bf16_to_float(q[j]);
    }
    __syncthreads();
    float score = -__builtin_inff();
    if (lane < count)
    {
        const uint16_t* row = k + std::size_t(start + lane) * width;
        float dot = 0.0f;
#pragma unroll
        for (int c = 0; c < HW / 8; ++c)
        {
            const uint4 u = reinterpret_cast<const uint4*>(row)[c];
            const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
            for (int i = 0; i < 4; ++i)
            {
                dot = __builtin_fmaf(qf[8 * c + 2 * i], bf16_to_float(uint16_t(w[i] & 0xffff)), dot);
                dot = __builtin_fmaf(qf[8 * c + 2 * i + 1], bf16_to_float(uint16_t(w[i] >> 16)), dot);
            }
        }
        score = dot * scale;
    }
    const float maximum = group_max<wave>(score);
    float e = 0.0f;
    if (lane < count)
    {
        const float shifted = score - maximum;
        e = original_exp(shifted);
    }
    const float sum = tree_sum<wave>(e);
    weights[lane] = e;
    __syncthreads();
    float* record = partial + (std::size_t(blockIdx.x) * max_blocks + block) * (2 + HW);
    if (lane == 0)
    {
        record[0] = maximum;
        record[1] = sum;
    }
    for (int j = lane; j < HW; j += 64)
    {
        float s = 0.0f;
        for (int t = 0; t < count; ++t)
        {
            s = __builtin_fmaf(bf16_to_float(v[std::size_t(start + t) * width + j]), weights[t], s);
        }
        if (round_values)
        {
            s = round_bf16(s);
        }
        record[2 + j] = s;
    }
}

// Waves per workgroup: 16 for 64-wide heads; 8 for 128-wide ones, whose key
// rows and value words need twice the registers.
template <int HW> constexpr int decode_waves = HW == 64 ? 16 : 8;
constexpr int decode_lds_blocks = 256; // blocks whose records one workgroup's LDS holds

// Records [max, block sum, value sums[HW]] of one (sequence, head) in LDS, wave
// w computing blocks w, w + decode_waves<HW>, ...; then wave 0 merges them in
// ascending order. The merge's running maxima are a scan with the recurrence's
// own update (keep the running maximum unless it is smaller: the first of
// equal values wins), which is associative without NaNs, so every block's
// factors come at once and only the two-operation total/numerator recurrence
// stays sequential; with a NaN maximum the merge runs the plain loop.
template <int HW>
__global__ __launch_bounds__(decode_waves<HW> * 64) void decode_attention_kernel(
    const uint16_t* __restrict__ query, const uint16_t* __restrict__ keys,
    const uint16_t* __restrict__ values, std::size_t sequence_stride, int width, int time,
    int heads, float scale, int round_values, uint16_t* __restrict__ out)
{
    extern __shared__ float records[]; // [blocks][2 + HW]
    __shared__ float qf[HW];
    __shared__ float weights[decode_waves<HW>][64];
    const int sequence = blockIdx.x / heads, head = blockIdx.x % heads;
    const int lane = threadIdx.x % wave, warp = __builtin_amdgcn_readfirstlane(int(threadIdx.x / wave));
    const int blocks = (time + 63) / 64;
    const uint16_t* q = query + std::size_t(sequence) * width + head * HW;
    const uint16_t* k = keys + std::size_t(sequence) * sequence_stride + head * HW;
    const uint16_t* v = values + std::size_t(sequence) * sequence_stride + head * HW;
    for (int j = threadIdx.x; j < HW; j += blockDim.x)
    {
        qf[j] = bf16_to_float(q[j]);
    }
    __syncthreads();
    // Lane l sums value column l (HW = 64) or columns 2l and 2l + 1 (HW = 128).
    constexpr int per_lane = HW / 64;
    for (int block = warp; block < blocks; block += decode_waves<HW>)
    {
        const int start = block * 64;
        const int count = time - start < 64 ? time - start : 64;
        // This lane's key row, then every row's values, requested before any
        // is used (rows past the history repeat its last row and are not
        // used): a load under a per-row branch would be waited for on its own,
        // and keys requested after the values would wait for all of them.
        uint4 key[HW / 8];
        {
            const uint16_t* row = k + std::size_t(start + lane < time ? start + lane : time - 1) * width;
#pragma unroll
            for (int c = 0; c < HW / 8; ++c)
            {
                key[c] = reinterpret_cast<const uint4*>(row)[c];
            }
        }
        uint32_t value[64];
#pragma unroll
        for (int t = 0; t < 64; ++t)
        {
            const int row = start + t < time ? start + t : time - 1;
            const uint16_t* at = v + std::size_t(row) * width + per_lane * lane;
            value[t] = per_lane == 2 ? *reinterpret_cast<const uint32_t*>(at) : uint32_t(*at);
        }
        float score = -__builtin_inff();
        if (lane < count)
        {
            float dot = 0.0f;
#pragma unroll
            for (int c = 0; c < HW / 8; ++c)
            {
                const uint4 u = key[c];
                const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
                for (int i = 0; i < 4; ++i)
                {
                    dot = __builtin_fmaf(qf[8 * c + 2 * i], bf16_to_float(uint16_t(w[i] & 0xffff)), dot);
                    dot = __builtin_fmaf(qf[8 * c + 2 * i + 1], bf16_to_float(uint16_t(w[i] >> 16)), dot);
                }
            }
            score = dot * scale;
        }
        const float maximum = group_max<wave>(score);
        float e = 0.0f;
        if (lane < count)
        {
            e = original_exp(score - maximum);
        }
        const float sum = tree_sum<wave>(e);
        weights[warp][lane] = e;
        __builtin_amdgcn_s_waitcnt(0xc07f); // lgkmcnt(0): the wave's weights are in
        __builtin_amdgcn_wave_barrier();
        float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
        for (int t = 0; t < 64; ++t)
        {
            if (t < count)
            {
                const float w = weights[warp][t];
                if constexpr (per_lane == 2)
                {
                    s0 = __builtin_fmaf(__uint_as_float(value[t] << 16), w, s0);
                    s1 = __builtin_fmaf(__uint_as_float(value[t] & 0xffff0000u), w, s1);
                }
                else
                {
                    s0 = __builtin_fmaf(__uint_as_float(value[t] << 16), w, s0);
                }
            }
        }
        float* record = records + std::size_t(block) * (2 + HW);
        if (lane == 0)
        {
            record[0] = maximum;
            record[1] = sum;
        }
        record[2 + per_lane * lane] = round_values ? round_bf16(s0) : s0;
        if constexpr (per_lane == 2)
        {
            record[3 + per_lane * lane] = round_values ? round_bf16(s1) : s1;
        }
        __builtin_amdgcn_wave_barrier();
    }
    __syncthreads();
    if (warp != 0)
    {
        return;
    }
    // Ordered merge (src/scalar/attention.cpp:86-101).
    float numerator[2] = {0.0f, 0.0f};
    float total = 0.0f;
    bool nan = false;
    for (int b = lane; b < blocks; b += wave)
    {
        nan = nan || __builtin_isnan(records[std::size_t(b) * (2 + HW)]);
    }
    const auto step = [&](const float* record, float old_scale, float new_scale)
    {
        total = __builtin_fmaf(record[1], new_scale, total * old_scale);
#pragma unroll
        for (int i = 0; i < per_lane; ++i)
        {
            numerator[i] = __builtin_fmaf(record[2 + per_lane * lane + i], new_scale, numerator[i] * old_scale);
        }
    };
    const auto scales_of = [](float running, float maximum, float& old_scale, float& new_scale)
    {
        const float factor = original_exp(-__builtin_fabsf(maximum - running));
        old_scale = running > maximum ? 1.0f : factor;
        new_scale = running > maximum ? factor : 1.0f;
    };
    if (__any(nan))
    {
        float running = -__builtin_inff();
        for (int b = 0; b < blocks; ++b)
        {
            const float* record = records + std::size_t(b) * (2 + HW);
            const float maximum = record[0];
            float old_scale, new_scale;
            scales_of(running, maximum, old_scale, new_scale);
            step(record, old_scale, new_scale);
            running = running < maximum ? maximum : running;
        }
    }
    else
    {
        float carry = -__builtin_inff();
        for (int chunk = 0; chunk < blocks; chunk += wave)
        {
            const int b = chunk + lane;
            const float maximum = b < blocks ? records[std::size_t(b) * (2 + HW)] : -__builtin_inff();
            // Inclusive scan of the running maximum over this chunk, from `carry`.
            float inclusive = maximum;
#pragma unroll
            for (int stride = 1; stride < wave; stride *= 2)
            {
                const float left = __shfl_up(inclusive, stride, wave);
                if (lane >= stride)
                {
                    inclusive = left < inclusive ? inclusive : left;
                }
            }
            inclusive = carry < inclusive ? inclusive : carry;
            const float before = __shfl_up(inclusive, 1, wave);
            const float running = lane == 0 ? carry : before;
            float old_scale, new_scale;
            scales_of(running, maximum, old_scale, new_scale);
            const int here = blocks - chunk < wave ? blocks - chunk : wave;
            for (int i = 0; i < here; ++i)
            {
                step(records + std::size_t(chunk + i) * (2 + HW),
                     __int_as_float(__builtin_amdgcn_readlane(__float_as_int(old_scale), i)),
                     __int_as_float(__builtin_amdgcn_readlane(__float_as_int(new_scale), i)));
            }
            carry = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(inclusive), here - 1));
        }
    }
    const float reciprocal = 1.0f / total;
    uint16_t* o = out + std::size_t(sequence) * width + head * HW + per_lane * lane;
    if constexpr (per_lane == 2)
    {
        *reinterpret_cast<uint32_t*>(o) =
            float_to_bf16(numerator[0] * reciprocal) | (uint32_t(float_to_bf16(numerator[1] * reciprocal)) << 16);
    }
    else
    {
        *o = float_to_bf16(numerator[0] * reciprocal);
    }
}

template <int HW>
__global__ __launch_bounds__(64) void decode_combine_kernel(const float* __restrict__ partial,
                                                            int time, int heads, int max_blocks,
                                                            int width, uint16_t* __restrict__ out)
{
    const int sequence = blockIdx.x / heads, head = blockIdx.x % heads;
    const int blocks = (time + 63) / 64;
    const float* records = partial + std::size_t(blockIdx.x) * max_blocks * (2 + HW);
    constexpr int per_lane = (HW + 63) / 64;
    float numerator[per_lane];
#pragma unroll
    for (int i = 0; i < per_lane; ++i)
    {
        numerator[i] = 0.0f;
    }
    float running_maximum = -__builtin_inff(), total = 0.0f;
    for (int b = 0; b < blocks; ++b)
    {
        const float* record = records + std::size_t(b) * (2 + HW);
        const float maximum = record[0];
        const float difference = maximum - running_maximum;
        const float factor = original_exp(-__builtin_fabsf(difference));
        const float old_scale = running_maximum > maximum ? 1.0f : factor;
        const float new_scale = running_maximum > maximum ? factor : 1.0f;
        const float old_total = total * old_scale;
        total = __builtin_fmaf(record[1], new_scale, old_total);
#pragma unroll
        for (int i = 0; i < per_lane; ++i)
        {
            const int j = threadIdx.x + 64 * i;
            if (j < HW)
            {
                const float old = numerator[i] * old_scale;
                numerator[i] = __builtin_fmaf(record[2 + j], new_scale, old);
            }
        }
        running_maximum = running_maximum < maximum ? maximum : running_maximum;
    }
    const float reciprocal = 1.0f / total;
#pragma unroll
    for (int i = 0; i < per_lane; ++i)
    {
        const int j = threadIdx.x + 64 * i;
        if (j < HW)
        {
            out[std::size_t(sequence) * width + head * HW + j] = float_to_bf16(numerator[i] * reciprocal);
        }
    }
}

// ------------------------------------------------------------------ prefill

constexpr int tile = 64;

template <int HW> struct PrefillShared
{
    static constexpr int row = HW + 8; // BF16 elements per LDS row (16-byte pad)
    uint16_t q[tile * row];
    uint16_t k[tile * row];
    uint16_t v[tile * row];
    float p[tile][tile + 4];
};

// Loads a [64][HW] tile from rows of `source` (row stride `stride` elements)
// with optional rotary at positions first..first+63. Rows at or beyond `limit`
// are zero.
template <int HW>
__device__ __forceinline__ void load_tile(uint16_t* dst, const uint16_t* source, std::size_t stride,
                                          int first, int limit, const uint16_t* rotations)
{
    constexpr int row = PrefillShared<HW>::row;
    constexpr int chunks = HW / 8;
    for (int i = threadIdx.x; i < tile * chunks; i += blockDim.x)
    {
        const int r = i / chunks, c = i % chunks;
        const int position = first + r;
        uint4 u = make_uint4(0, 0, 0, 0);
        if (position < limit)
        {
            u = *reinterpret_cast<const uint4*>(source + std::size_t(position) * stride + c * 8);
            if (rotations)
            {
                uint32_t w[4] = {u.x, u.y, u.z, u.w};
                const uint16_t* coefficients = rotations + std::size_t(position) * HW + c * 8;
#pragma unroll
                for (int p = 0; p < 4; ++p)
                {
                    float re = bf16_to_float(uint16_t(w[p] & 0xffff));
                    float im = bf16_to_float(uint16_t(w[p] >> 16));
                    rotate_pair(re, im, coefficients + 2 * p);
                    w[p] = float_to_bf16(re) | (uint32_t(float_to_bf16(im)) << 16);
                }
                u = make_uint4(w[0], w[1], w[2], w[3]);
            }
        }
        *reinterpret_cast<uint4*>(dst + r * row + c * 8) = u;
    }
}

// Workgroup of 256 threads: thread t owns queries 4*(t/16)..+3 and, for scores,
// keys (t%16) + 16*b (b = 0..3) of the current block; for value sums it owns
// coordinates (t%16)*HW/16 .. +HW/16 of the same four queries. With that key
// placement the 16-lane butterfly on each register followed by the register
// pair tree is exactly the balanced pair tree over the block's 64 positions.
template <int HW>
__global__ __launch_bounds__(256) void prefill_kernel(
    const uint16_t* __restrict__ qkv, int width, const int* __restrict__ sequence_start,
    const int* __restrict__ sequence_length, const int* __restrict__ sequence_replay,
    const uint16_t* __restrict__ rotations, int heads, float scale, uint16_t* __restrict__ out)
{
    constexpr int row = PrefillShared<HW>::row;
    constexpr int columns = HW / 16;
    __shared__ PrefillShared<HW> shared;
    (void)heads; // the grid's z extent
    const int sequence = blockIdx.x, head = blockIdx.z;
    const int length = sequence_length[sequence];
    const int q0 = blockIdx.y * tile;
    if (q0 >= length)
    {
        return;
    }
    const int replay = sequence_replay[sequence];
    const std::size_t stride = std::size_t(3) * width;
    const uint16_t* base = qkv + std::size_t(sequence_start[sequence]) * stride + head * HW;
    const int tid = threadIdx.x, group = tid / 16, slot = tid % 16;

    load_tile<HW>(shared.q, base, stride, q0, length, rotations);

    float numerator[4][columns];
    float running_maximum[4], total[4];
#pragma unroll
    for (int a = 0; a < 4; ++a)
    {
        running_maximum[a] = -__builtin_inff();
        total[a] = 0.0f;
#pragma unroll
        for (int c = 0; c < columns; ++c)
        {
            numerator[a][c] = 0.0f;
        }
    }
    const int last_block = (q0 + tile - 1 < length - 1 ? q0 + tile - 1 : length - 1) / tile;
    for (int block = 0; block <= last_block; ++block)
    {
        const int k0 = block * tile;
        __syncthreads(); // previous block's K/V/P reads are done
        load_tile<HW>(shared.k, base + width, stride, k0, length, rotations);
        load_tile<HW>(shared.v, base + 2 * width, stride, k0, length, nullptr);
        __syncthreads();

        // Scores for 4 queries x 4 keys: serial fma chains over coordinates.
        float dot[4][4];
#pragma unroll
        for (int a = 0; a < 4; ++a)
#pragma unroll
            for (int b = 0; b < 4; ++b)
            {
                dot[a][b] = 0.0f;
            }
        for (int c = 0; c < HW / 8; ++c)
        {
            uint4 qu[4], ku[4];
#pragma unroll
            for (int a = 0; a < 4; ++a)
            {
                qu[a] = *reinterpret_cast<const uint4*>(shared.q + (4 * group + a) * row + c * 8);
                ku[a] = *reinterpret_cast<const uint4*>(shared.k + (slot + 16 * a) * row + c * 8);
            }
#pragma unroll
            for (int e = 0; e < 8; ++e)
            {
                float qv[4], kv[4];
#pragma unroll
                for (int a = 0; a < 4; ++a)
                {
                    const uint32_t qw[4] = {qu[a].x, qu[a].y, qu[a].z, qu[a].w};
                    const uint32_t kw[4] = {ku[a].x, ku[a].y, ku[a].z, ku[a].w};
                    qv[a] = bf16_to_float(uint16_t(e % 2 ? qw[e / 2] >> 16 : qw[e / 2] & 0xffff));
                    kv[a] = bf16_to_float(uint16_t(e % 2 ? kw[e / 2] >> 16 : kw[e / 2] & 0xffff));
                }
#pragma unroll
                for (int a = 0; a < 4; ++a)
#pragma unroll
                    for (int b = 0; b < 4; ++b)
                    {
                        dot[a][b] = __builtin_fmaf(qv[a], kv[b], dot[a][b]);
                    }
            }
        }
        float block_maximum[4], block_sum[4];
#pragma unroll
        for (int a = 0; a < 4; ++a)
        {
            const int query = q0 + 4 * group + a;
            float score[4];
            float maximum = -__builtin_inff();
#pragma unroll
            for (int b = 0; b < 4; ++b)
            {
                const int key = k0 + slot + 16 * b;
                const bool valid = key <= query && key < length;
                score[b] = dot[a][b] * scale;
                if (valid)
                {
                    maximum = maximum < score[b] ? score[b] : maximum;
                }
            }
            maximum = group_max<16>(maximum);
            float e[4];
#pragma unroll
            for (int b = 0; b < 4; ++b)
            {
                const int key = k0 + slot + 16 * b;
                const bool valid = key <= query && key < length;
                e[b] = 0.0f;
                if (valid)
                {
                    const float shifted = score[b] - maximum;
                    e[b] = original_exp(shifted);
                }
                shared.p[4 * group + a][slot + 16 * b] = e[b];
            }
            // Pair tree over the 64 (zero-padded) block positions; for eight or
            // fewer live positions the extra +0 levels leave the eight-wide tree
            // unchanged (src/format/categorical.cpp:44-50).
            float quarters[4];
#pragma unroll
            for (int b = 0; b < 4; ++b)
            {
                quarters[b] = tree_sum<16>(e[b]);
            }
            block_sum[a] = register_tree(quarters);
            block_maximum[a] = maximum;
        }
        __syncthreads();
        // Value sums: serial fma over the block's live keys, ascending.
#pragma unroll
        for (int a = 0; a < 4; ++a)
        {
            const int query = q0 + 4 * group + a;
            if (query >= length)
            {
                continue;
            }
            const int live = (query < k0 + tile - 1 ? query : k0 + tile - 1) - k0 + 1;
            const int count = live < length - k0 ? live : length - k0;
            float sums[columns];
#pragma unroll
            for (int c = 0; c < columns; ++c)
            {
                sums[c] = 0.0f;
            }
            for (int t = 0; t < count; ++t)
            {
                const float w = shared.p[4 * group + a][t];
                const uint16_t* vrow = shared.v + t * row + slot * columns;
#pragma unroll
                for (int c = 0; c < columns; ++c)
                {
                    sums[c] = __builtin_fmaf(bf16_to_float(vrow[c]), w, sums[c]);
                }
            }
            const bool round_values = query + 1 > 64 || query < replay;
            const float maximum = block_maximum[a];
            const float difference = maximum - running_maximum[a];
            const float factor = original_exp(-__builtin_fabsf(difference));
            const float old_scale = running_maximum[a] > maximum ? 1.0f : factor;
            const float new_scale = running_maximum[a] > maximum ? factor : 1.0f;
            const float old_total = total[a] * old_scale;
            total[a] = __builtin_fmaf(block_sum[a], new_scale, old_total);
#pragma unroll
            for (int c = 0; c < columns; ++c)
            {
                const float s = round_values ? round_bf16(sums[c]) : sums[c];
                const float old = numerator[a][c] * old_scale;
                numerator[a][c] = __builtin_fmaf(s, new_scale, old);
            }
            running_maximum[a] = running_maximum[a] < maximum ? maximum : running_maximum[a];
        }
    }
#pragma unroll
    for (int a = 0; a < 4; ++a)
    {
        const int query = q0 + 4 * group + a;
        if (query >= length)
        {
            continue;
        }
        const float reciprocal = 1.0f / total[a];
        uint16_t* o = out + (std::size_t(sequence_start[sequence]) + query) * width + head * HW +
                      slot * columns;
#pragma unroll
        for (int c = 0; c < columns; ++c)
        {
            o[c] = float_to_bf16(numerator[a][c] * reciprocal);
        }
    }
}
} // namespace

void append_qkv(const uint16_t* qkv, std::size_t rows, std::size_t width, std::size_t head_width,
                const uint16_t* rotation, uint16_t* query, uint16_t* keys, uint16_t* values,
                std::size_t row_stride, hipStream_t stream)
{
    require(width % 2 == 0 && head_width % 2 == 0 && width % head_width == 0, "append: shape");
    if (!rows)
    {
        return;
    }
    const std::size_t n = rows * width / 2;
    const unsigned grid = unsigned((n + 255) / 256 < 4096 ? (n + 255) / 256 : 4096);
    append_kernel<<<grid, 256, 0, stream>>>(qkv, int(rows), int(width), int(head_width), rotation,
                                            query, keys, values, row_stride);
    check_hip(hipGetLastError(), "append launch");
}

std::size_t decode_partial_floats(std::size_t sequences, std::size_t heads, std::size_t head_width,
                                  std::size_t time)
{
    const std::size_t blocks = (time + 63) / 64;
    return blocks <= std::size_t(decode_lds_blocks) ? 0 : sequences * heads * blocks * (2 + head_width);
}

void attention_decode(const uint16_t* query, const uint16_t* keys, const uint16_t* values,
                      std::size_t sequence_stride, std::size_t sequences, std::size_t time,
                      std::size_t heads, std::size_t head_width, float scale, bool replay,
                      float* partial, uint16_t* out, hipStream_t stream)
{
    require(time > 0 && sequences > 0, "attention: empty shape");
    require(time < (std::size_t(1) << 30) && sequences * heads < (std::size_t(1) << 31), "attention: shape too large");
    const int max_blocks = int((time + 63) / 64);
    const int width = int(heads * head_width);
    const int round_values = time > 64 || replay;
    if (max_blocks <= decode_lds_blocks)
    {
        const std::size_t lds = std::size_t(max_blocks) * (2 + head_width) * 4;
        const unsigned grid = unsigned(sequences * heads);
        switch (head_width)
        {
        case 64:
            check_hip(hipFuncSetAttribute(reinterpret_cast<const void*>(decode_attention_kernel<64>),
                                          hipFuncAttributeMaxDynamicSharedMemorySize, int(lds)),
                      "attention decode LDS");
            decode_attention_kernel<64><<<grid, decode_waves<64> * 64, lds, stream>>>(
                query, keys, values, sequence_stride, width, int(time), int(heads), scale, round_values, out);
            break;
        case 128:
            check_hip(hipFuncSetAttribute(reinterpret_cast<const void*>(decode_attention_kernel<128>),
                                          hipFuncAttributeMaxDynamicSharedMemorySize, int(lds)),
                      "attention decode LDS");
            decode_attention_kernel<128><<<grid, decode_waves<128> * 64, lds, stream>>>(
                query, keys, values, sequence_stride, width, int(time), int(heads), scale, round_values, out);
            break;
        default:
            throw Error("attention: head width must be 64 or 128");
        }
        check_hip(hipGetLastError(), "attention decode launch");
        return;
    }
    require(partial != nullptr, "attention: long histories need the partial scratch");
    const dim3 grid(unsigned(sequences * heads), unsigned(max_blocks));
    switch (head_width)
    {
    case 64:
        decode_blocks_kernel<64><<<grid, 64, 0, stream>>>(query, keys, values, sequence_stride,
                                                          width, int(time), int(heads), scale,
                                                          round_values, max_blocks, partial);
        decode_combine_kernel<64><<<unsigned(sequences * heads), 64, 0, stream>>>(
            partial, int(time), int(heads), max_blocks, width, out);
        break;
    case 128:
        decode_blocks_kernel<128><<<grid, 64, 0, stream>>>(query, keys, values, sequence_stride,
                                                           width, int(time), int(heads), scale,
                                                           round_values, max_blocks, partial);
        decode_combine_kernel<128><<<unsigned(sequences * heads), 64, 0, stream>>>(
            partial, int(time), int(heads), max_blocks, width, out);
        break;
    default:
        throw Error("attention: head width must be 64 or 128");
    }
    check_hip(hipGetLastError(), "attention decode launch");
}

void attention_prefill(const uint16_t* qkv, std::size_t width, std::size_t heads,
                       std::size_t head_width, const int* sequence_start,
                       const int* sequence_length, const int* sequence_replay,
                       std::size_t sequences, std::size_t max_length, const uint16_t* rotations,
                       float scale, uint16_t* out, hipStream_t stream)
{
    require(width == heads * head_width, "attention: width mismatch");
    if (!sequences || !max_length)
    {
        return;
    }
    const dim3 grid(unsigned(sequences), unsigned((max_length + tile - 1) / tile), unsigned(heads));
    switch (head_width)
    {
    case 64:
        prefill_kernel<64><<<grid, 256, 0, stream>>>(qkv, int(width), sequence_start, sequence_length,
                                                     sequence_replay, rotations, int(heads), scale, out);
        break;
    case 128:
        prefill_kernel<128><<<grid, 256, 0, stream>>>(qkv, int(width), sequence_start,
                                                      sequence_length, sequence_replay, rotations,
                                                      int(heads), scale, out);
        break;
    default:
        throw Error("attention: head width must be 64 or 128");
    }
    check_hip(hipGetLastError(), "attention prefill launch");
}
} // namespace tsac_hip
