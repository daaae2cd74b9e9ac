// Causal multi-head attention with the reference's exact arithmetic
// (src/scalar/attention.cpp:12-131):
//   * scores: one serial fma chain over the head coordinates (ascending), times scale;
//   * keys in 64-position blocks: block max, original_exp(score - max), pair-tree
//     block sum, per-coordinate serial fma value sums (BF16-rounded when the
//     query's history exceeds 64 positions or during replay);
//   * blocks merged in ascending order with the online-softmax recurrence.
// Matrix cores would reorder those sums, so everything runs on the VALU.
//
// Decode (one query per sequence): each (sequence, head)'s 64-key blocks are
// spread over several workgroups of one launch, one wave per block; the last
// workgroup to arrive merges the block records in ascending order.
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

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// Waves per decode workgroup; each wave computes one 64-key block's record.
constexpr int decode_waves = 4;


// Workgroups per (sequence, head) for a history of `blocks` key blocks.
constexpr int decode_splits(int blocks)
{
    return (blocks + decode_waves - 1) / decode_waves;
}

// One query per (sequence, head) over its `time` cached keys, split over
// decode_splits(blocks) workgroups of decode_waves waves: wave w of split s
// computes the record [max, block sum, value sums[HW]] of block
// s * decode_waves + w. With one split the records stay in LDS; otherwise
// they go to `partial` ([sequence * heads + head][blocks][2 + HW]) and each
// workgroup counts its arrival in `arrivals[sequence * heads + head]` (zero
// on entry, zero again on exit): the last to arrive copies every record into
// LDS and merges them in ascending block order, so the counter only hands
// the merge over and the summation order is the single-workgroup one.
//
// A block's key and value rows are read whole (16 bytes per lane, so a load
// covers 64 / (HW / 8) rows) and pass through LDS: each lane takes its key
// row, then its value column.
//
// The merge's running maxima are a scan with the recurrence's own update
// (keep the running maximum unless it is smaller: the first of equal values
// wins), which is associative without NaNs, so every block's factors come at
// once and only the two-operation total/numerator recurrence stays
// sequential; with a NaN maximum the merge runs the plain loop.
template <int HW>
__global__ __launch_bounds__(decode_waves * 64) void decode_attention_kernel(
    const uint16_t* __restrict__ query, const uint16_t* __restrict__ keys,
    const uint16_t* __restrict__ values, std::size_t sequence_stride, int width, int time,
    int heads, float scale, int round_values, float* __restrict__ partial, unsigned* __restrict__ arrivals,
    uint16_t* __restrict__ out)
{
    constexpr int chunks = HW / 8;            // 16-byte chunks per row
    constexpr int rows_per_load = 64 / chunks;
    extern __shared__ float records[];        // [blocks][2 + HW]
    __shared__ uint4 staged[decode_waves][64 * chunks]; // each wave's key rows, then value rows
    __shared__ float weights[decode_waves][64];
    __shared__ float4 factors[64]; // the merge's per-block (old scale, new scale, block sum)
    __shared__ int merging;
    const int blocks = (time + 63) / 64;
    const int splits = decode_splits(blocks);
    const int pair = blockIdx.x / splits, split = blockIdx.x % splits;
    const int sequence = pair / heads, head = pair % heads;
    const int lane = threadIdx.x % wave, warp = __builtin_amdgcn_readfirstlane(int(threadIdx.x / wave));
    const uint16_t* k = keys + std::size_t(sequence) * sequence_stride + head * HW;
    const uint16_t* v = values + std::size_t(sequence) * sequence_stride + head * HW;
    // Lane l sums value column l (HW = 64) or columns 2l and 2l + 1 (HW = 128).
    constexpr int per_lane = HW / 64;
    float* const shared_records = partial + std::size_t(pair) * blocks * (2 + HW);
    const int block = split * decode_waves + warp;
    if (block < blocks)
    {
        const int start = block * 64;
        const int count = time - start < 64 ? time - start : 64;
        // The block's key rows and value rows, whole rows at a time (16 bytes
        // per lane, so a load covers 64 / (HW / 8) rows), all requested
        // before any is used. Rows past the history lie beyond the buffers'
        // ends and read zero; their scores are dropped and their values not
        // used. The row offset goes in the range-checked vector offset (the
        // scalar offset is not checked).
        const __amdgpu_buffer_rsrc_t key_rows =
            __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(k), 0, time * width * 2, 0x00020000);
        const __amdgpu_buffer_rsrc_t value_rows =
            __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(v), 0, time * width * 2, 0x00020000);
        const int lane_offset = (lane / chunks) * width * 2 + (lane % chunks) * 16;
        uint4 key_data[chunks], rows[chunks];
#pragma unroll
        for (int i = 0; i < chunks; ++i)
        {
            const u32x4 r = __builtin_amdgcn_raw_buffer_load_b128(
                key_rows, lane_offset + (start + i * rows_per_load) * width * 2, 0, 0);
            key_data[i] = make_uint4(r.x, r.y, r.z, r.w);
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < chunks; ++i)
        {
            const u32x4 r = __builtin_amdgcn_raw_buffer_load_b128(
                value_rows, lane_offset + (start + i * rows_per_load) * width * 2, 0, 0);
            rows[i] = make_uint4(r.x, r.y, r.z, r.w);
        }
        __builtin_amdgcn_sched_barrier(0); // every load issued before the first wait
        // Keys through LDS to one row per lane; chunk c of row r is kept at
        // r * chunks + (c ^ (r % 8)), so neither the row-wise writes nor the
        // lane-per-row reads meet in a bank.
#pragma unroll
        for (int i = 0; i < chunks; ++i)
        {
            const int r = i * rows_per_load + lane / chunks, c = lane % chunks;
            staged[warp][r * chunks + (c ^ (r & 7))] = key_data[i];
        }
        __builtin_amdgcn_s_waitcnt(0xc07f); // lgkmcnt(0)
        __builtin_amdgcn_wave_barrier();
        uint4 key[chunks];
#pragma unroll
        for (int c = 0; c < chunks; ++c)
        {
            key[c] = staged[warp][lane * chunks + (c ^ (lane & 7))];
        }
        // The query, uniform over the workgroup, in scalar registers.
        const uint32_t* q = reinterpret_cast<const uint32_t*>(query + std::size_t(sequence) * width + head * HW);
        float dot = 0.0f;
#pragma unroll
        for (int c = 0; c < chunks; ++c)
        {
            const uint4 u = key[c];
            const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
            for (int i = 0; i < 4; ++i)
            {
                const uint32_t pair_q = __builtin_amdgcn_readfirstlane(q[4 * c + i]);
                dot = __builtin_fmaf(__uint_as_float(pair_q << 16), __uint_as_float(w[i] << 16), dot);
                dot = __builtin_fmaf(__uint_as_float(pair_q & 0xffff0000u), __uint_as_float(w[i] & 0xffff0000u), dot);
            }
        }
        const float score = lane < count ? dot * scale : -__builtin_inff();
        const float maximum = group_max<wave>(score);
        float e = 0.0f;
        if (lane < count)
        {
            e = original_exp(score - maximum);
        }
        const float sum = tree_sum<wave>(e);
        weights[warp][lane] = e;
#pragma unroll
        for (int i = 0; i < chunks; ++i)
        {
            staged[warp][i * 64 + lane] = rows[i];
        }
        __builtin_amdgcn_s_waitcnt(0xc07f); // lgkmcnt(0): the wave's weights and values are in
        __builtin_amdgcn_wave_barrier();
        const uint16_t* column16 = reinterpret_cast<const uint16_t*>(staged[warp]) + lane;
        const uint32_t* column32 = reinterpret_cast<const uint32_t*>(staged[warp]) + lane;
        float s0 = 0.0f, s1 = 0.0f;
        const auto accumulate = [&](int t)
        {
            const float w = weights[warp][t];
            if constexpr (per_lane == 2)
            {
                const uint32_t p = column32[t * 64];
                s0 = __builtin_fmaf(__uint_as_float(p << 16), w, s0);
                s1 = __builtin_fmaf(__uint_as_float(p & 0xffff0000u), w, s1);
            }
            else
            {
                s0 = __builtin_fmaf(__uint_as_float(uint32_t(column16[t * 64]) << 16), w, s0);
            }
        };
        if (count == 64)
        {
#pragma unroll
            for (int t = 0; t < 64; ++t)
            {
                accumulate(t);
            }
        }
        else
        {
            for (int t = 0; t < count; ++t)
            {
                accumulate(t);
            }
        }
        const std::size_t at = std::size_t(block) * (2 + HW);
        // Records for the merge of another workgroup go out as device-coherent
        // stores, so no cache needs writing back before the arrival is counted.
        const auto put = [&](int i, float value)
        {
            if (splits == 1)
            {
                records[at + i] = value;
            }
            else
            {
                __hip_atomic_store(shared_records + at + i, value, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        };
        if (lane == 0)
        {
            put(0, maximum);
            put(1, sum);
        }
        put(2 + per_lane * lane, round_values ? round_bf16(s0) : s0);
        if constexpr (per_lane == 2)
        {
            put(3 + per_lane * lane, round_values ? round_bf16(s1) : s1);
        }
    }
    if (splits > 1)
    {
        // Every wave's records are written before the workgroup counts its
        // arrival; the last to arrive resets the counter and merges.
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (threadIdx.x == 0)
        {
            const unsigned before =
                __hip_atomic_fetch_add(arrivals + pair, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            merging = before == unsigned(splits - 1);
            if (merging)
            {
                __hip_atomic_store(arrivals + pair, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
        __syncthreads();
        if (!merging)
        {
            return;
        }
    }
    else
    {
        __syncthreads();
    }
    if (warp != 0)
    {
        return;
    }
    // Ordered merge (src/scalar/attention.cpp:86-101) by one wave, over
    // chunks of 64 blocks: lane b holds block b's maximum and sum, every lane
    // its value sums of all 64 blocks (read from LDS with one split, with
    // device-coherent loads from `partial` otherwise, all requested at once).
    const auto scales_of = [](float running, float maximum, float& old_scale, float& new_scale)
    {
        const float factor = original_exp(-__builtin_fabsf(maximum - running));
        old_scale = running > maximum ? 1.0f : factor;
        new_scale = running > maximum ? factor : 1.0f;
    };
    float numerator[per_lane];
#pragma unroll
    for (int c = 0; c < per_lane; ++c)
    {
        numerator[c] = 0.0f;
    }
    float total = 0.0f;
    float carry = -__builtin_inff();
    for (int chunk = 0; chunk < blocks; chunk += wave)
    {
        const int here = blocks - chunk < wave ? blocks - chunk : wave;
        const bool live = lane < here;
        // Straight-line loads in groups of eight blocks, every one requested
        // before the first is waited for. A group may read up to seven
        // records past the last block (the records are followed by that much
        // padding); those values are replaced below.
        float first[2];
        float column[wave][per_lane];
        const auto gather = [&](auto load)
        {
            const int b = chunk + (live ? lane : here - 1);
            first[0] = load(std::size_t(b) * (2 + HW));
            first[1] = load(std::size_t(b) * (2 + HW) + 1);
            const std::size_t base = std::size_t(chunk) * (2 + HW) + 2 + per_lane * lane;
#pragma unroll
            for (int g = 0; g < wave / 8; ++g)
            {
                if (g * 8 < here)
                {
#pragma unroll
                    for (int j = 0; j < 8; ++j)
                    {
#pragma unroll
                        for (int c = 0; c < per_lane; ++c)
                        {
                            column[g * 8 + j][c] = load(base + std::size_t(g * 8 + j) * (2 + HW) + c);
                        }
                    }
                }
            }
        };
        if (splits == 1)
        {
            gather([&](std::size_t at) { return records[at]; });
        }
        else
        {
            gather([&](std::size_t at)
                   { return __hip_atomic_load(shared_records + at, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); });
        }
        // Lanes past the last block step with old scale 1, new scale 0 and
        // sums of -0, which leave the total and numerators exactly as they
        // are, so the steps need no per-block branch.
        const float maximum = live ? first[0] : -__builtin_inff();
        const float block_sum = live ? first[1] : -0.0f;
        float old_scale = 1.0f, new_scale = 0.0f;
        if (__any(__builtin_isnan(maximum)))
        {
            // The plain running maximum, one block at a time.
            float running = carry;
            for (int i = 0; i < here; ++i)
            {
                const float m = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(maximum), i));
                float o, n;
                scales_of(running, m, o, n);
                if (lane == i)
                {
                    old_scale = o;
                    new_scale = n;
                }
                running = running < m ? m : running;
            }
            carry = running;
        }
        else
        {
            const float scanned = running_max_scan(maximum);
            const float inclusive = carry < scanned ? scanned : carry;
            scales_of(previous_lane(inclusive, carry), maximum, old_scale, new_scale);
            carry = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(inclusive), here - 1));
        }
        // Each block's factors go through LDS, so the steps read them as
        // operands (one broadcast read per block) instead of moving them lane
        // by lane into scalar registers.
        factors[lane] = make_float4(live ? old_scale : 1.0f, live ? new_scale : 0.0f, block_sum, 0.0f);
        __builtin_amdgcn_s_waitcnt(0xc07f); // lgkmcnt(0)
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int g = 0; g < wave / 8; ++g)
        {
            if (g * 8 < here)
            {
#pragma unroll
                for (int j = 0; j < 8; ++j)
                {
                    const float4 f = factors[g * 8 + j];
                    total = __builtin_fmaf(f.z, f.y, total * f.x);
#pragma unroll
                    for (int c = 0; c < per_lane; ++c)
                    {
                        const float sum = g * 8 + j < here ? column[g * 8 + j][c] : -0.0f;
                        numerator[c] = __builtin_fmaf(sum, f.y, numerator[c] * f.x);
                    }
                }
            }
        }
        __builtin_amdgcn_wave_barrier(); // the factors are read before the next chunk's are written
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


// ------------------------------------------------------------------ prefill

constexpr int tile = 64;

// With 64-wide heads the key tile is widened to fp32 as it is stored, once
// per block, instead of by each of the 16 threads that read a key row (the
// workgroup still fits three to a CU); 128-wide heads keep BF16 keys.
template <int HW> constexpr bool wide_keys = HW == 64;

template <int HW> struct PrefillShared
{
    static constexpr int row = HW + 8;  // BF16 elements per LDS row (16-byte pad)
    static constexpr int key_row = HW + 4; // fp32 elements per widened key row
    uint16_t q[tile * row];
    uint16_t k[wide_keys<HW> ? 8 : tile * row];
    float kf[wide_keys<HW> ? tile * key_row : 4];
    uint16_t v[tile * row];
    float p[tile][tile + 4];
};

// Loads a [64][HW] tile from rows of `source` (row stride `stride` elements)
// with optional rotary at positions first..first+63. Rows at or beyond `limit`
// are zero. With a float destination the values are stored widened (rows of
// key_row floats).
template <int HW, class T>
__device__ __forceinline__ void load_tile(T* dst, const uint16_t* source, std::size_t stride,
                                          int first, int limit, const uint16_t* rotations)
{
    constexpr bool widen = sizeof(T) == 4;
    constexpr int row = widen ? PrefillShared<HW>::key_row : PrefillShared<HW>::row;
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
        if constexpr (widen)
        {
            const uint32_t w[4] = {u.x, u.y, u.z, u.w};
            float4* out = reinterpret_cast<float4*>(dst + r * row + c * 8);
            out[0] = make_float4(__uint_as_float(w[0] << 16), __uint_as_float(w[0] & 0xffff0000u),
                                 __uint_as_float(w[1] << 16), __uint_as_float(w[1] & 0xffff0000u));
            out[1] = make_float4(__uint_as_float(w[2] << 16), __uint_as_float(w[2] & 0xffff0000u),
                                 __uint_as_float(w[3] << 16), __uint_as_float(w[3] & 0xffff0000u));
        }
        else
        {
            *reinterpret_cast<uint4*>(dst + r * row + c * 8) = u;
        }
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
        if constexpr (wide_keys<HW>)
        {
            load_tile<HW>(shared.kf, base + width, stride, k0, length, rotations);
        }
        else
        {
            load_tile<HW>(shared.k, base + width, stride, k0, length, rotations);
        }
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
            float4 kf[4][2];
#pragma unroll
            for (int a = 0; a < 4; ++a)
            {
                qu[a] = *reinterpret_cast<const uint4*>(shared.q + (4 * group + a) * row + c * 8);
                if constexpr (wide_keys<HW>)
                {
                    const float4* k = reinterpret_cast<const float4*>(
                        shared.kf + (slot + 16 * a) * PrefillShared<HW>::key_row + c * 8);
                    kf[a][0] = k[0];
                    kf[a][1] = k[1];
                }
                else
                {
                    ku[a] = *reinterpret_cast<const uint4*>(shared.k + (slot + 16 * a) * row + c * 8);
                }
            }
#pragma unroll
            for (int e = 0; e < 8; ++e)
            {
                float qv[4], kv[4];
#pragma unroll
                for (int a = 0; a < 4; ++a)
                {
                    const uint32_t qw[4] = {qu[a].x, qu[a].y, qu[a].z, qu[a].w};
                    qv[a] = bf16_to_float(uint16_t(e % 2 ? qw[e / 2] >> 16 : qw[e / 2] & 0xffff));
                    if constexpr (wide_keys<HW>)
                    {
                        const float4 h = kf[a][e / 4];
                        const float k4[4] = {h.x, h.y, h.z, h.w};
                        kv[a] = k4[e % 4];
                    }
                    else
                    {
                        const uint32_t kw[4] = {ku[a].x, ku[a].y, ku[a].z, ku[a].w};
                        kv[a] = bf16_to_float(uint16_t(e % 2 ? kw[e / 2] >> 16 : kw[e / 2] & 0xffff));
                    }
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
        // Value sums: serial fma over each query's live keys, ascending. Keys
        // are the outer loop, so each value row read and widened serves the
        // thread's four queries; a query's chain stops at its own last key.
        int count[4];
#pragma unroll
        for (int a = 0; a < 4; ++a)
        {
            const int query = q0 + 4 * group + a;
            const int live = (query < k0 + tile - 1 ? query : k0 + tile - 1) - k0 + 1;
            count[a] = query >= length ? 0 : live < length - k0 ? live : length - k0;
        }
        // Queries past the sequence (count 0) are never merged, so they need
        // not stop the others' unchecked loop.
        int common = tile, most = 0;
#pragma unroll
        for (int a = 0; a < 4; ++a)
        {
            if (count[a] > 0)
            {
                common = min(common, count[a]);
                most = max(most, count[a]);
            }
        }
        common = min(common, most);
        float sums[4][columns];
#pragma unroll
        for (int a = 0; a < 4; ++a)
        {
#pragma unroll
            for (int c = 0; c < columns; ++c)
            {
                sums[a][c] = 0.0f;
            }
        }
        const auto accumulate = [&](int t, const float (&w)[4], bool every)
        {
            const uint16_t* vrow = shared.v + t * row + slot * columns;
            float value[columns];
#pragma unroll
            for (int c = 0; c < columns; ++c)
            {
                value[c] = bf16_to_float(vrow[c]);
            }
#pragma unroll
            for (int a = 0; a < 4; ++a)
            {
                if (every || t < count[a])
                {
#pragma unroll
                    for (int c = 0; c < columns; ++c)
                    {
                        sums[a][c] = __builtin_fmaf(value[c], w[a], sums[a][c]);
                    }
                }
            }
        };
        int t = 0;
        for (; t + 4 <= common; t += 4)
        {
            float4 w4[4];
#pragma unroll
            for (int a = 0; a < 4; ++a)
            {
                w4[a] = *reinterpret_cast<const float4*>(&shared.p[4 * group + a][t]);
            }
            accumulate(t, {w4[0].x, w4[1].x, w4[2].x, w4[3].x}, true);
            accumulate(t + 1, {w4[0].y, w4[1].y, w4[2].y, w4[3].y}, true);
            accumulate(t + 2, {w4[0].z, w4[1].z, w4[2].z, w4[3].z}, true);
            accumulate(t + 3, {w4[0].w, w4[1].w, w4[2].w, w4[3].w}, true);
        }
        for (; t < most; ++t)
        {
            accumulate(t, {shared.p[4 * group][t], shared.p[4 * group + 1][t], shared.p[4 * group + 2][t],
                           shared.p[4 * group + 3][t]},
                       false);
        }
#pragma unroll
        for (int a = 0; a < 4; ++a)
        {
            const int query = q0 + 4 * group + a;
            if (query >= length)
            {
                continue;
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
                const float s = round_values ? round_bf16(sums[a][c]) : sums[a][c];
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

namespace
{
__global__ void clear_arrivals(unsigned* words, std::size_t count)
{
    for (std::size_t i = blockIdx.x * std::size_t(blockDim.x) + threadIdx.x; i < count;
         i += std::size_t(gridDim.x) * blockDim.x)
    {
        words[i] = 0;
    }
}
} // namespace

std::size_t decode_partial_floats(std::size_t sequences, std::size_t heads, std::size_t head_width,
                                  std::size_t time)
{
    const std::size_t blocks = (time + 63) / 64;
    // Seven records of padding: the merge reads whole groups of eight.
    return decode_splits(int(blocks)) > 1 ? (sequences * heads * blocks + 7) * (2 + head_width) : 0;
}

std::size_t decode_arrival_counters(std::size_t sequences, std::size_t heads, std::size_t time)
{
    return decode_splits(int((time + 63) / 64)) > 1 ? sequences * heads : 0;
}

void clear_arrival_counters(unsigned* counters, std::size_t count, hipStream_t stream)
{
    if (count)
    {
        const std::size_t groups = (count + 255) / 256;
        clear_arrivals<<<unsigned(groups < 1024 ? groups : 1024), 256, 0, stream>>>(counters, count);
        check_hip(hipGetLastError(), "attention counter clear launch");
    }
}

void attention_decode(const uint16_t* query, const uint16_t* keys, const uint16_t* values,
                      std::size_t sequence_stride, std::size_t sequences, std::size_t time,
                      std::size_t heads, std::size_t head_width, float scale, bool replay,
                      float* partial, unsigned* arrivals, uint16_t* out, hipStream_t stream)
{
    require(time > 0 && sequences > 0, "attention: empty shape");
    require(time < (std::size_t(1) << 30) && sequences * heads < (std::size_t(1) << 24), "attention: shape too large");
    require(head_width == 64 || head_width == 128, "attention: head width must be 64 or 128");
    require(time * heads * head_width * 2 < (std::size_t(1) << 31), "attention: history too long for one decode");
    const int max_blocks = int((time + 63) / 64);
    const int width = int(heads * head_width);
    const int round_values = time > 64 || replay;
    const std::size_t pairs = sequences * heads;
    require(!decode_partial_floats(sequences, heads, head_width, time) || partial != nullptr,
            "attention: this history needs the decode records scratch");
    require(!decode_arrival_counters(sequences, heads, time) || arrivals != nullptr,
            "attention: this history needs the decode arrival counters");
    const int splits = decode_splits(max_blocks);
    require(pairs * splits < (std::size_t(1) << 31), "attention: too many workgroups for one decode");
    // Records stay in LDS only with one split (then with the merge's seven
    // records of padding).
    const std::size_t lds = splits == 1 ? std::size_t(max_blocks + 7) * (2 + head_width) * 4 : 0;
    const unsigned grid = unsigned(pairs * splits);
    const auto launch = [&](auto kernel)
    {
        check_hip(hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                      hipFuncAttributeMaxDynamicSharedMemorySize, int(lds)),
                  "attention decode LDS");
        kernel<<<grid, decode_waves * 64, lds, stream>>>(query, keys, values, sequence_stride, width, int(time),
                                                        int(heads), scale, round_values, partial, arrivals, out);
    };
    if (head_width == 64)
    {
        launch(decode_attention_kernel<64>);
    }
    else
    {
        launch(decode_attention_kernel<128>);
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
