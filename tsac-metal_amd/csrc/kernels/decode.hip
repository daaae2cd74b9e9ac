// Decode-side kernels (see decode.hpp). Arithmetic is shared with the batched
// path through row_ops.hpp / device_numeric.hpp, so both passes produce the same
// bits: the same BF8L quantiser, LayerNorm, embedding sums, exact int8 block
// dots and ordered per-block fma chain (src/scalar/packed_linear.cpp:16-27),
// attention recurrence (src/scalar/attention.cpp:62-101), softmax
// (src/common/probability.cpp:96-122) and categorical bisection
// (src/format/categorical.cpp:119-142) with the range decoder
// (src/format/range.cpp:131-151).
//
// These launches are latency-bound (a few lanes per step), so every kernel
// issues its independent global loads first and overlaps them with its
// prologue arithmetic.
#include "decode.hpp"
#include "row_ops.hpp"
#include "step_ops.hpp"

namespace tsac_hip
{
namespace
{
using namespace step;
// ------------------------------------------------------------------ fused projection

template <int V, Input I>
__device__ __forceinline__ void input_row(const FusedLinear& a, int m, int lane, int8_t* q_row,
                                          float* s_row, bool write_prefix)
{
    constexpr int K = wave * V;
    uint16_t v[V];
    if constexpr (I == Input::bf16 || I == Input::layer_norm)
    {
        load_row<V>(a.x + std::size_t(m) * a.x_stride + lane * V, v);
        if constexpr (I == Input::layer_norm)
        {
            layer_norm_lane<V>(v, a.gain, a.beta, lane);
        }
    }
    else if constexpr (I == Input::embed_sum)
    {
        // src/common/cpu_transformer.tpp:205-224: copy book 0, add later books in order.
        const uint16_t* t = a.tokens + std::size_t(m) * a.token_stride;
        load_row<V>(a.embeddings + std::size_t(t[0]) * K + lane * V, v);
        for (int b = 1; b < a.books; ++b)
        {
            uint16_t e[V];
            load_row<V>(a.embeddings + (std::size_t(b) * a.alphabet + t[b]) * K + lane * V, e);
#pragma unroll
            for (int i = 0; i < V; ++i)
            {
                v[i] = float_to_bf16(bf16_to_float(v[i]) + bf16_to_float(e[i]));
            }
        }
    }
    else
    {
        const int token = a.tokens[std::size_t(m) * a.token_stride + a.token_offset];
        load_row<V>(a.embeddings + (std::size_t(a.book) * a.alphabet + token) * K + lane * V, v);
        if (a.x)
        {
            uint16_t p[V];
            load_row<V>(a.x + std::size_t(m) * K + lane * V, p);
#pragma unroll
            for (int i = 0; i < V; ++i)
            {
                v[i] = float_to_bf16(bf16_to_float(p[i]) + bf16_to_float(v[i]));
            }
        }
        if (write_prefix)
        {
            store_row<V>(a.prefix_out + std::size_t(m) * K + lane * V, v);
        }
    }
    bf8l_lane<V>(v, lane, q_row, s_row, a.error);
}

constexpr int fused_waves = 8;

// One workgroup per 64-row weight tile. Waves split the tile's K/16 segments
// (blocks x 16) evenly; exact int32 partial dots meet in LDS and the ordered
// fma chain runs per (row pair, column).
template <int V, Input I>
__global__ __launch_bounds__(fused_waves * wave) void fused_linear_kernel(const FusedLinear a)
{
    constexpr int K = wave * V, blocks = K / 256;
    constexpr int waves_per_block = blocks >= fused_waves ? 1 : fused_waves / blocks;
    constexpr int wave_segments = segments / waves_per_block;
    constexpr int rounds = blocks > fused_waves ? blocks / fused_waves : 1;
    constexpr int slots = blocks * waves_per_block; // partial-dot slots per (column, row)
    __shared__ __attribute__((aligned(16))) int8_t q[max_columns * K];
    __shared__ float scales[max_columns * blocks];
    __shared__ int dots[slots * max_columns * tile_rows];
    const int lane = threadIdx.x % wave;
    const int warp = __builtin_amdgcn_readfirstlane(int(threadIdx.x / wave));
    const int tile = blockIdx.x;
    const int M = a.M, N = int(a.w.N);

    // 1. Weight loads of the first round, issued before anything else.
    const int first_block = rounds > 1 ? warp : warp / waves_per_block;
    const int first_segment = rounds > 1 ? 0 : (warp % waves_per_block) * wave_segments;
    uint4 w[wave_segments];
    {
        const int8_t* base = a.w.values + tile_offset(tile, first_block, first_segment, blocks) + lane * 16;
#pragma unroll
        for (int s = 0; s < wave_segments; ++s)
        {
            w[s] = *reinterpret_cast<const uint4*>(base + s * tile_rows * 16);
        }
    }
    // Chain constants for this thread's (row pair, column).
    const int pair = threadIdx.x % 32, column = threadIdx.x / 32;
    const int n0 = tile * tile_rows + 2 * pair;
    const float bias0 = a.w.bias[n0], bias1 = a.w.bias[n0 + 1];
    float ws0[blocks], ws1[blocks];
#pragma unroll
    for (int b = 0; b < blocks; ++b)
    {
        const float2 s = *reinterpret_cast<const float2*>(a.w.scales + std::size_t(b) * N + n0);
        ws0[b] = s.x;
        ws1[b] = s.y;
    }

    // 2. Inputs: one row per wave, quantised into LDS.
    if (warp < M)
    {
        input_row<V, I>(a, warp, lane, q + warp * K, scales + warp * blocks, tile == 0);
    }
    __syncthreads();

    // 3. Exact partial dots.
#pragma unroll
    for (int r = 0; r < rounds; ++r)
    {
        const int b = rounds > 1 ? warp + r * fused_waves : first_block;
        if (r > 0)
        {
            const int8_t* base = a.w.values + tile_offset(tile, b, 0, blocks) + lane * 16;
#pragma unroll
            for (int s = 0; s < wave_segments; ++s)
            {
                w[s] = *reinterpret_cast<const uint4*>(base + s * tile_rows * 16);
            }
        }
        const int slot = b * waves_per_block + (rounds > 1 ? 0 : warp % waves_per_block);
        for (int m = 0; m < M; ++m)
        {
            const uint4* x = reinterpret_cast<const uint4*>(q + m * K + b * 256 + first_segment * 16);
            int dot = 0;
#pragma unroll
            for (int s = 0; s < wave_segments; ++s)
            {
                const uint4 u = x[s];
                dot = __builtin_amdgcn_sdot4(int(w[s].x), int(u.x), dot, false);
                dot = __builtin_amdgcn_sdot4(int(w[s].y), int(u.y), dot, false);
                dot = __builtin_amdgcn_sdot4(int(w[s].z), int(u.z), dot, false);
                dot = __builtin_amdgcn_sdot4(int(w[s].w), int(u.w), dot, false);
            }
            dots[(slot * max_columns + m) * tile_rows + lane] = dot;
        }
    }
    __syncthreads();

    // 4. Ordered chain: ascending blocks, one fma each (the exact block dot is
    //    the integer sum of its partial slots).
    if (column >= M)
    {
        return;
    }
    const int m = column;
    float sum0 = 0.0f, sum1 = 0.0f;
#pragma unroll
    for (int b = 0; b < blocks; ++b)
    {
        int d0 = 0, d1 = 0;
#pragma unroll
        for (int p = 0; p < waves_per_block; ++p)
        {
            const int* d = dots + ((b * waves_per_block + p) * max_columns + m) * tile_rows + 2 * pair;
            d0 += d[0];
            d1 += d[1];
        }
        const float as = scales[m * blocks + b];
        const float scale0 = ws0[b] * as;
        const float scale1 = ws1[b] * as;
        sum0 = __builtin_fmaf(float(d0), scale0, sum0);
        sum1 = __builtin_fmaf(float(d1), scale1, sum1);
    }
    uint16_t y0 = float_to_bf16(sum0 + bias0);
    uint16_t y1 = float_to_bf16(sum1 + bias1);
    switch (a.output)
    {
    case Output::plain:
        break;
    case Output::residual:
    {
        const uint16_t* r = a.residual + std::size_t(m) * a.residual_stride + n0;
        y0 = float_to_bf16(bf16_to_float(r[0]) + bf16_to_float(y0));
        y1 = float_to_bf16(bf16_to_float(r[1]) + bf16_to_float(y1));
        break;
    }
    case Output::gelu:
        y0 = gelu_bf16(y0);
        y1 = gelu_bf16(y1);
        break;
    case Output::qkv:
    {
        const int position = a.position ? *a.position : a.fixed_position;
        const int width = a.width;
        float re = bf16_to_float(y0), im = bf16_to_float(y1);
        if (n0 < 2 * width && a.rotations)
        {
            rotate(re, im, a.rotations + std::size_t(position) * a.head_width + n0 % a.head_width);
        }
        const uint32_t packed = float_to_bf16(re) | (uint32_t(float_to_bf16(im)) << 16);
        uint16_t* dst;
        if (n0 < width)
        {
            dst = a.query + std::size_t(m) * width + n0;
        }
        else if (n0 < 2 * width)
        {
            dst = a.keys + std::size_t(m) * a.lane_stride + std::size_t(position) * width + (n0 - width);
        }
        else
        {
            dst = a.values + std::size_t(m) * a.lane_stride + std::size_t(position) * width + (n0 - 2 * width);
        }
        *reinterpret_cast<uint32_t*>(dst) = packed;
        return;
    }
    }
    *reinterpret_cast<uint32_t*>(a.y + std::size_t(m) * a.y_stride + n0) = y0 | (uint32_t(y1) << 16);
}

template <int V> void launch_fused(const FusedLinear& a, hipStream_t stream)
{
    const dim3 grid(unsigned(a.w.N / tile_rows)), block(fused_waves * wave);
    switch (a.input)
    {
    case Input::bf16:
        fused_linear_kernel<V, Input::bf16><<<grid, block, 0, stream>>>(a);
        break;
    case Input::layer_norm:
        fused_linear_kernel<V, Input::layer_norm><<<grid, block, 0, stream>>>(a);
        break;
    case Input::embed_sum:
        fused_linear_kernel<V, Input::embed_sum><<<grid, block, 0, stream>>>(a);
        break;
    case Input::embed_accumulate:
        fused_linear_kernel<V, Input::embed_accumulate><<<grid, block, 0, stream>>>(a);
        break;
    }
}

// ------------------------------------------------------------------ attention

constexpr int step_waves = 8;

// One workgroup per (lane, head); wave w owns key blocks w, w + waves, ...
// Every lane of a wave loads its key row and its value columns of the block up
// front, so one memory round trip precedes the serial fma chains.
template <int HW>
__global__ __launch_bounds__(step_waves * wave) void attention_step_kernel(
    const uint16_t* __restrict__ query, const uint16_t* __restrict__ keys,
    const uint16_t* __restrict__ values, long long lane_stride, int width, int heads, float scale,
    const int* position_ptr, int fixed_position, int replay, uint16_t* __restrict__ out)
{
    constexpr int per_lane = HW / 64; // value columns per lane (adjacent)
    extern __shared__ float partial[]; // [blocks][2 + HW]
    __shared__ float qf[HW];
    __shared__ float weights[step_waves][64];
    const int lane_index = blockIdx.x / heads, head = blockIdx.x % heads;
    const int lane = threadIdx.x % wave;
    const int warp = threadIdx.x / wave;
    const int waves = blockDim.x / wave;
    const int time = (position_ptr ? *position_ptr : fixed_position) + 1;
    const int blocks = (time + 63) / 64;
    const bool round_values = time > 64 || replay;
    const uint16_t* k = keys + std::size_t(lane_index) * lane_stride + head * HW;
    const uint16_t* v = values + std::size_t(lane_index) * lane_stride + head * HW;
    // Key row of this lane and value columns [per_lane*lane, +per_lane) of every
    // row of one block; the first block's loads are issued before the query is
    // staged.
    uint4 key[HW / 8];
    uint32_t value[64];
    const auto load_block = [&](int block)
    {
        const int start = block * 64;
        const int count = time - start < 64 ? time - start : 64;
        if (lane < count)
        {
            const uint4* row = reinterpret_cast<const uint4*>(k + std::size_t(start + lane) * width);
#pragma unroll
            for (int c = 0; c < HW / 8; ++c)
            {
                key[c] = row[c];
            }
        }
#pragma unroll
        for (int t = 0; t < 64; ++t)
        {
            value[t] = 0;
            if (t < count)
            {
                const uint16_t* src = v + std::size_t(start + t) * width + per_lane * lane;
                value[t] = per_lane == 2 ? *reinterpret_cast<const uint32_t*>(src) : uint32_t(src[0]);
            }
        }
    };
    if (warp < blocks)
    {
        load_block(warp);
    }
    for (int j = threadIdx.x; j < HW; j += blockDim.x)
    {
        qf[j] = bf16_to_float(query[std::size_t(lane_index) * width + head * HW + j]);
    }
    __syncthreads();
    for (int block = warp; block < blocks; block += waves)
    {
        if (block != warp)
        {
            load_block(block);
        }
        const int start = block * 64;
        const int count = time - start < 64 ? time - start : 64;
        float score = -__builtin_inff();
        if (lane < count)
        {
            float dot = 0.0f;
#pragma unroll
            for (int c = 0; c < HW / 8; ++c)
            {
                const uint32_t w4[4] = {key[c].x, key[c].y, key[c].z, key[c].w};
#pragma unroll
                for (int i = 0; i < 4; ++i)
                {
                    dot = __builtin_fmaf(qf[8 * c + 2 * i], bf16_to_float(uint16_t(w4[i] & 0xffff)), dot);
                    dot = __builtin_fmaf(qf[8 * c + 2 * i + 1], bf16_to_float(uint16_t(w4[i] >> 16)), dot);
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
        weights[warp][lane] = e;
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
        float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
        for (int t = 0; t < 64; ++t)
        {
            if (t < count)
            {
                const float wt = weights[warp][t];
                s0 = __builtin_fmaf(bf16_to_float(uint16_t(value[t] & 0xffff)), wt, s0);
                if (per_lane == 2)
                {
                    s1 = __builtin_fmaf(bf16_to_float(uint16_t(value[t] >> 16)), wt, s1);
                }
            }
        }
        float* record = partial + std::size_t(block) * (2 + HW);
        if (lane == 0)
        {
            record[0] = maximum;
            record[1] = sum;
        }
        record[2 + per_lane * lane] = round_values ? round_bf16(s0) : s0;
        if (per_lane == 2)
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
    float numerator[per_lane];
#pragma unroll
    for (int i = 0; i < per_lane; ++i)
    {
        numerator[i] = 0.0f;
    }
    float running_maximum = -__builtin_inff(), total = 0.0f;
    for (int b = 0; b < blocks; ++b)
    {
        const float* record = partial + std::size_t(b) * (2 + HW);
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
            const float old = numerator[i] * old_scale;
            numerator[i] = __builtin_fmaf(record[2 + per_lane * lane + i], new_scale, old);
        }
        running_maximum = running_maximum < maximum ? maximum : running_maximum;
    }
    const float reciprocal = 1.0f / total;
    uint16_t* o = out + std::size_t(lane_index) * width + head * HW + per_lane * lane;
#pragma unroll
    for (int i = 0; i < per_lane; ++i)
    {
        o[i] = float_to_bf16(numerator[i] * reciprocal);
    }
}

// ------------------------------------------------------------------ norms

template <int V>
__global__ __launch_bounds__(256) void layer_norm_add_kernel(const uint16_t* x, int rows,
                                                             const uint16_t* __restrict__ gain,
                                                             const uint16_t* __restrict__ bias,
                                                             const uint16_t* __restrict__ add_row,
                                                             uint16_t* out)
{
    constexpr int width = wave * V;
    const int lane = threadIdx.x % wave;
    const int row = blockIdx.x * 4 + threadIdx.x / wave;
    if (row >= rows)
    {
        return;
    }
    uint16_t v[V];
    load_row<V>(x + std::size_t(row) * width + lane * V, v);
    layer_norm_lane<V>(v, gain, bias, lane);
    if (add_row)
    {
        uint16_t p[V];
        load_row<V>(add_row + lane * V, p);
#pragma unroll
        for (int i = 0; i < V; ++i)
        {
            v[i] = float_to_bf16(bf16_to_float(v[i]) + bf16_to_float(p[i]));
        }
    }
    store_row<V>(out + std::size_t(row) * width + lane * V, v);
}

// ------------------------------------------------------------------ sampling

constexpr int sample_waves = 8;
// Payload bytes staged per launch: each of at most 8 symbols consumes at most
// 10 decisions x 2 bytes, so 256 bytes always cover a launch.
constexpr int window = 256;

// Up to `sample_waves` lanes: one wavefront each for the softmax, masses and
// top decisions, then wave 0 decodes the lanes' symbols in stream order.
__global__ __launch_bounds__(sample_waves * wave) void sample_kernel(const Sample a)
{
    __shared__ float nodes[sample_waves][1024];
    __shared__ uint16_t leaves[sample_waves][1024];
    __shared__ uint16_t top[sample_waves][64];
    __shared__ int valid[sample_waves];
    __shared__ int rows[sample_waves];
    __shared__ __attribute__((aligned(16))) uint8_t bytes[window];
    __shared__ DecoderState shared_state;
    const int lane = threadIdx.x % wave, warp = threadIdx.x / wave;
    const int step = a.step ? *a.step : a.fixed_step;
    const int i = warp;
    const bool active = i < a.lanes;
    // Independent loads first: logits, row offset, decoder state.
    uint16_t v[16];
    int row = 0;
    if (active)
    {
        load_row<16>(a.logits + std::size_t(i) * 1024 + lane * 16, v);
        row = a.row_base[i] + step * a.step_stride + a.book;
    }
    if (a.state && threadIdx.x == 0)
    {
        shared_state = *a.state;
    }
    __syncthreads();
    // The payload window after the current offset, held in a register until
    // the softmax is done.
    uint32_t byte = 0;
    const unsigned long long base_offset = a.state ? shared_state.offset : 0;
    if (a.state && threadIdx.x < window && base_offset + threadIdx.x < a.payload_bytes)
    {
        byte = a.payload[base_offset + threadIdx.x];
    }
    if (active)
    {
        if (lane == 0)
        {
            rows[warp] = row;
        }
        // Softmax (src/common/probability.cpp:96-122).
        float maximum = -__builtin_inff();
        bool finite = true;
#pragma unroll
        for (int k = 0; k < 16; ++k)
        {
            const float value = bf16_to_float(v[k]);
            finite = finite && is_finite(value);
            maximum = maximum < value ? value : maximum;
        }
        if (!finite)
        {
            a.error[0] = 1u;
        }
        maximum = group_max<wave>(maximum);
        float e[16], leaves_sum[16];
#pragma unroll
        for (int k = 0; k < 16; ++k)
        {
            const float shifted = bf16_to_float(v[k]) - maximum;
            e[k] = original_exp(shifted);
            leaves_sum[k] = e[k];
        }
        const float total = row_sum<16>(leaves_sum);
        const float reciprocal = 1.0f / total;
        float p[16];
#pragma unroll
        for (int k = 0; k < 16; ++k)
        {
            v[k] = float_to_bf16(e[k] * reciprocal);
            p[k] = bf16_to_float(v[k]);
        }
        if (a.distributions)
        {
            store_row<16>(a.distributions + std::size_t(row) * 1024 + lane * 16, v);
        }
        if (a.state || a.splits)
        {
            store_row<16>(&leaves[warp][lane * 16], v);
            const bool ok = build_masses(p, lane, nodes[warp]);
            wait_shared_memory();
            if (a.state)
            {
                build_top_decisions(lane, Masses{nodes[warp], leaves[warp]}, top[warp]);
            }
            if (lane == 0)
            {
                valid[warp] = ok;
            }
        }
    }
    if (threadIdx.x < window)
    {
        bytes[threadIdx.x] = uint8_t(byte);
    }
    __syncthreads();
    if (warp != 0)
    {
        return;
    }
    // Wave 0 decodes the lanes' symbols in stream order.
    DecoderState s = a.state ? shared_state : DecoderState{};
    const ByteWindow staged{bytes, window, base_offset, a.payload, a.payload_bytes};
    for (int w = 0; w < a.lanes; ++w)
    {
        const int r = __builtin_amdgcn_readfirstlane(rows[w]);
        int token;
        if (a.known)
        {
            token = a.known[r];
            if (a.splits)
            {
                const uint16_t q = path_split(Masses{nodes[w], leaves[w]}, token, lane);
                if (lane < 10)
                {
                    a.splits[std::size_t(r) * 16 + lane] = q;
                }
            }
        }
        else
        {
            if (!__builtin_amdgcn_readfirstlane(valid[w]))
            {
                s.failed = 1;
            }
            token = decode_symbol(top[w], Masses{nodes[w], leaves[w]}, s, staged);
        }
        if (lane == 0)
        {
            a.current[std::size_t(w) * a.books + a.book] = uint16_t(token);
            a.tokens[r] = uint16_t(token);
        }
    }
    if (a.state && lane == 0)
    {
        *a.state = s;
        if (s.failed)
        {
            a.error[1] = 1u;
        }
    }
}

__global__ void gather_frame_kernel(const uint16_t* tokens, const int* row_base, int frame,
                                    int step_stride, int books, int lanes, uint16_t* dst)
{
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < lanes * books; i += gridDim.x * blockDim.x)
    {
        const int lane = i / books, b = i % books;
        dst[i] = tokens[std::size_t(row_base[lane]) + std::size_t(frame) * step_stride + b];
    }
}

__global__ void set_counters_kernel(int* counters, int position, int step)
{
    counters[0] = position;
    counters[1] = step;
}

__global__ void advance_counters_kernel(int* counters)
{
    counters[0] += 1;
    counters[1] += 1;
}
} // namespace

void fused_linear(const FusedLinear& a, hipStream_t stream)
{
    require(a.M >= 1 && a.M <= max_columns, "fused linear: 1..8 columns");
    require(a.w.N % tile_rows == 0 && a.w.K % 256 == 0, "fused linear: shape");
    require(a.error != nullptr, "fused linear: error word");
    switch (a.w.K)
    {
    case 256:
        launch_fused<4>(a, stream);
        break;
    case 512:
        launch_fused<8>(a, stream);
        break;
    case 1024:
        launch_fused<16>(a, stream);
        break;
    case 2048:
        launch_fused<32>(a, stream);
        break;
    case 4096:
        launch_fused<64>(a, stream);
        break;
    default:
        throw Error("fused linear: K must be one of 256, 512, 1024, 2048, 4096");
    }
    check_hip(hipGetLastError(), "fused linear launch");
}

void attention_step(const uint16_t* query, const uint16_t* keys, const uint16_t* values,
                    long long lane_stride, std::size_t lanes, std::size_t width,
                    std::size_t heads, std::size_t head_width, float scale, const int* position,
                    int fixed_position, std::size_t max_time, bool replay, uint16_t* out,
                    hipStream_t stream)
{
    require(lanes > 0 && max_time > 0 && width == heads * head_width, "attention step: shape");
    const std::size_t blocks = (max_time + 63) / 64;
    const std::size_t lds = blocks * (2 + head_width) * sizeof(float);
    require(lds <= 64 * 1024, "attention step: history too long");
    const unsigned grid = unsigned(lanes * heads);
    // With a host-known position only the needed wavefronts are launched.
    const std::size_t needed = position ? blocks : (std::size_t(fixed_position) + 64) / 64;
    const unsigned threads = unsigned(std::min<std::size_t>(needed, step_waves) * wave);
    switch (head_width)
    {
    case 64:
        attention_step_kernel<64><<<grid, threads, lds, stream>>>(
            query, keys, values, lane_stride, int(width), int(heads), scale, position, fixed_position,
            replay ? 1 : 0, out);
        break;
    case 128:
        attention_step_kernel<128><<<grid, threads, lds, stream>>>(
            query, keys, values, lane_stride, int(width), int(heads), scale, position, fixed_position,
            replay ? 1 : 0, out);
        break;
    default:
        throw Error("attention: head width must be 64 or 128");
    }
    check_hip(hipGetLastError(), "attention step launch");
}

void layer_norm_add(const uint16_t* x, std::size_t rows, std::size_t width, const uint16_t* gain,
                    const uint16_t* bias, const uint16_t* add_row, uint16_t* out, hipStream_t stream)
{
    if (!rows)
    {
        return;
    }
    const unsigned grid = unsigned((rows + 3) / 4);
    switch (width)
    {
    case 256:
        layer_norm_add_kernel<4><<<grid, 256, 0, stream>>>(x, int(rows), gain, bias, add_row, out);
        break;
    case 512:
        layer_norm_add_kernel<8><<<grid, 256, 0, stream>>>(x, int(rows), gain, bias, add_row, out);
        break;
    case 1024:
        layer_norm_add_kernel<16><<<grid, 256, 0, stream>>>(x, int(rows), gain, bias, add_row, out);
        break;
    case 2048:
        layer_norm_add_kernel<32><<<grid, 256, 0, stream>>>(x, int(rows), gain, bias, add_row, out);
        break;
    default:
        throw Error("layer norm: width must be one of 256, 512, 1024, 2048");
    }
    check_hip(hipGetLastError(), "layer norm launch");
}

void sample_step(const Sample& a, hipStream_t stream)
{
    require(a.lanes > 0 && a.lanes <= sample_waves && a.current && a.tokens && a.row_base && a.error,
            "sample: arguments");
    require(a.known || a.state, "sample: needs known tokens or a decoder");
    sample_kernel<<<1, sample_waves * wave, 0, stream>>>(a);
    check_hip(hipGetLastError(), "sample launch");
}

void gather_frame(const uint16_t* tokens, const int* row_base, int frame, int step_stride, int books,
                  int lanes, uint16_t* dst, hipStream_t stream)
{
    if (lanes <= 0)
    {
        return;
    }
    const int n = lanes * books;
    gather_frame_kernel<<<(n + 255) / 256, 256, 0, stream>>>(tokens, row_base, frame, step_stride, books,
                                                             lanes, dst);
    check_hip(hipGetLastError(), "gather launch");
}

void set_counters(int* counters, int position, int step, hipStream_t stream)
{
    set_counters_kernel<<<1, 1, 0, stream>>>(counters, position, step);
    check_hip(hipGetLastError(), "counter launch");
}

void advance_counters(int* counters, hipStream_t stream)
{
    advance_counters_kernel<<<1, 1, 0, stream>>>(counters);
    check_hip(hipGetLastError(), "counter launch");
}
} // namespace tsac_hip
