// DAC convolutions with fused Snake/residual epilogues, and the RVQ encoder
// and decoder (dac.hpp).
#include "dac.hpp"

#include <algorithm>
#include <cstring>

namespace tsac_hip
{
namespace
{
constexpr int lanes = 64;
constexpr int conv_waves = 4;
constexpr int conv_threads = conv_waves * lanes;

// Weights and biases are written before the launches and never during them:
// reads through the constant address space become scalar loads.
template <class T> using constant_ptr = const __attribute__((address_space(4))) T*;
template <class T> __device__ __forceinline__ constant_ptr<T> constant(const T* p)
{
    return (constant_ptr<T>)(p);
}

__device__ __forceinline__ float from_bits(uint32_t bits)
{
    return __uint_as_float(bits);
}

// sin(phase)^2 as src/scalar/dsp.cpp:47-84 computes it: quadrant = the
// nearest integer to phase * 2/pi (ties to even), a two-term Cody-Waite
// reduction, then the odd or even minimax polynomial by the quadrant's parity.
// The parity is that of the reference's int32 conversion, which is even for
// every float at or beyond 2^24 (and the indefinite value beyond 2^31).
__device__ __forceinline__ float sine_squared(float phase)
{
    const float reduced = phase * from_bits(0x3f22f983);
    const float quadrant = __builtin_rintf(reduced);
    const bool odd = __builtin_fabsf(quadrant) < 16777216.0f && (int(quadrant) & 1) != 0;
    float x = __builtin_fmaf(quadrant, from_bits(0xbfc90000), phase);
    x = __builtin_fmaf(quadrant, from_bits(0xb9fdaa22), x);
    const float x2 = x * x;
    float value;
    if (!odd)
    {
        float polynomial = __builtin_fmaf(from_bits(0xb94ca1f9), x2, from_bits(0x3c08839e));
        polynomial = __builtin_fmaf(polynomial, x2, from_bits(0xbe2aaaa3));
        const float cube = x * x2;
        value = __builtin_fmaf(cube, polynomial, x);
    }
    else
    {
        float polynomial = __builtin_fmaf(from_bits(0x37ccf5ce), x2, from_bits(0xbab6061a));
        polynomial = __builtin_fmaf(polynomial, x2, from_bits(0x3d2aaaa5));
        polynomial = __builtin_fmaf(polynomial, x2, from_bits(0xbf000000));
        value = __builtin_fmaf(polynomial, x2, 1.0f);
    }
    return value * value;
}

// Snake of src/scalar/dsp.cpp:86-111: y + sin^2(a y) / (a + eps).
__device__ __forceinline__ float snake(float y, float a, bool& finite)
{
    const float phase = a * y;
    finite = finite && __builtin_isfinite(phase);
    const float squared = sine_squared(phase);
    const float denominator = a + from_bits(0x3089705f);
    const float result = y + squared / denominator;
    finite = finite && __builtin_isfinite(result);
    return result;
}

// One wave: 64 output frames (one per lane) x CH output channels. Ordinary
// convolutions take consecutive frames; transposed ones the frames of one
// residue class mod the stride, so every tap is either valid for the whole wave
// or only at its edges. Each input value loaded serves CH serial sums; layers
// with few frames take CH = 8, 4 or 2 so that their grid still fills the SIMDs
// (each sum stays one serial chain, so CH changes no value).
template <bool Transposed, int CH> __global__ __launch_bounds__(conv_threads) void conv_kernel(const ConvArgs a)
{
    static_assert(dac_channel_block % CH == 0, "channel groups within the weights' padding");
    const int lane = threadIdx.x % lanes;
    const int block = blockIdx.y * conv_waves + __builtin_amdgcn_readfirstlane(int(threadIdx.x / lanes));
    const ConvShape s = a.conv.shape;
    const int out_padded = a.conv.out_padded;
    if (block * CH >= out_padded)
    {
        return;
    }
    const int c0 = block * CH;
    const int out_frames = s.output_frames(a.frames);
    int f;
    int first_tap = 0, tap_step = 1;
    if constexpr (Transposed)
    {
        const int residue = blockIdx.x % s.stride, tile = blockIdx.x / s.stride;
        f = residue + s.stride * (tile * lanes + lane);
        first_tap = (residue + s.padding) % s.stride;
        tap_step = s.stride;
    }
    else
    {
        f = blockIdx.x * lanes + lane;
    }
    const bool in_range = f < out_frames && f >= a.first && f < a.last;
    float sum[CH];
#pragma unroll
    for (int j = 0; j < CH; ++j)
    {
        sum[j] = 0.0f;
    }
    const float* x = a.x.data;
    const long long xc = a.x.channel, xf = a.x.frame;
    const float* w = a.conv.w + c0;
    for (int tap = first_tap; tap < s.kernel; tap += tap_step)
    {
        long long source;
        bool valid;
        if constexpr (Transposed)
        {
            const int position = f + s.padding - tap * s.dilation;
            valid = in_range && position >= 0;
            source = position / s.stride;
        }
        else
        {
            const int position = f * s.stride + tap * s.dilation - s.padding;
            valid = in_range && position >= 0;
            source = position;
        }
        valid = valid && source < a.frames;
        if (!valid)
        {
            continue;
        }
        const float* xs = x + (a.x.phases > 1 ? (source % a.x.phases) * a.x.phase + (source / a.x.phases) * xf
                                              : source * xf);
        const float* wt = w + std::size_t(tap) * s.in * out_padded;
        // About 64 products per lane between the loads' issue and their use.
        constexpr int ahead = 64 / CH < 16 ? 64 / CH : 16;
#pragma unroll ahead
        for (int i = 0; i < s.in; ++i)
        {
            const float xv = xs[i * xc];
            const constant_ptr<float> wv = constant(wt + std::size_t(i) * out_padded);
#pragma unroll
            for (int j = 0; j < CH; ++j)
            {
                const float product = xv * wv[j];
                sum[j] = sum[j] + product;
            }
        }
    }
    if (!in_range)
    {
        return;
    }
    bool finite = true;
    const constant_ptr<float> bias = constant(a.conv.bias);
#pragma unroll
    for (int j = 0; j < CH; ++j)
    {
        const int c = c0 + j;
        if (c >= s.out)
        {
            break;
        }
        float y = sum[j] + bias[c];
        if (a.residual.data)
        {
            y = a.residual.data[c * a.residual.channel + f * a.residual.frame] + y;
        }
        finite = finite && __builtin_isfinite(y);
        if (a.out.data)
        {
            a.out.data[c * a.out.channel + f * a.out.frame] = y;
        }
        if (a.activated.data)
        {
            const long long at = a.activated.phases > 1 ? (f % a.activated.phases) * a.activated.phase +
                                                              (f / a.activated.phases) * a.activated.frame
                                                        : f * a.activated.frame;
            a.activated.data[c * a.activated.channel + at] = snake(y, a.alpha[c], finite);
        }
    }
    if (!finite)
    {
        a.error[0] = 1u;
    }
}

// ---------------------------------------------------------------- RVQ

__device__ __forceinline__ float shuffle(float v, int source)
{
    return __shfl(v, source, lanes);
}

// One wave per frame: the codebooks in order, each its input projection (an
// ordinary 1024 -> 8 pointwise convolution: serial sums over the inputs, then
// the bias), the normalised search (src/weights/preparation.cpp:62-84 and
// src/common/rvq.cpp:131-151) and the chosen vector's projection subtracted
// from the residual (src/common/rvq.tpp:40-57).
__global__ __launch_bounds__(lanes) void rvq_encode_kernel(const RvqBook* books, int count, const float* latent,
                                                         long long stride, int frames, uint16_t* tokens,
                                                         int token_stride, uint32_t* error)
{
    __shared__ float residual[1024];
    const int frame = blockIdx.x, lane = threadIdx.x;
    if (frame >= frames)
    {
        return;
    }
    bool finite = true;
    for (int i = lane; i < 1024; i += lanes)
    {
        residual[i] = latent[i * stride + frame];
        finite = finite && __builtin_isfinite(residual[i]);
    }
    __syncthreads();
    for (int b = 0; b < count; ++b)
    {
        const RvqBook book = books[b];
        float projected = 0.0f;
        if (lane < 8)
        {
            const float* w = book.input_weights + lane * 1024;
            for (int i = 0; i < 1024; ++i)
            {
                const float product = residual[i] * w[i];
                projected = projected + product;
            }
            projected = projected + book.input_bias[lane];
        }
        float q[8];
#pragma unroll
        for (int i = 0; i < 8; ++i)
        {
            q[i] = shuffle(projected, i);
            finite = finite && __builtin_isfinite(q[i]);
        }
        // normalize_search: squares reduced by adjacent pairs, RMS with epsilon, 1/sqrt(8).
        float squares[8];
#pragma unroll
        for (int i = 0; i < 8; ++i)
        {
            squares[i] = q[i] * q[i];
        }
#pragma unroll
        for (int width = 8; width > 1; width /= 2)
        {
#pragma unroll
            for (int i = 0; i < width / 2; ++i)
            {
                squares[i] = squares[2 * i] + squares[2 * i + 1];
            }
        }
        const float mean = squares[0] * (1.0f / 8.0f);
        const float inverse_rms = 1.0f / __builtin_sqrtf(mean + from_bits(0x2b8cbccc));
        const float inverse_width = 1.0f / __builtin_sqrtf(8.0f);
        float query[8];
#pragma unroll
        for (int i = 0; i < 8; ++i)
        {
            const float normalized = q[i] * inverse_rms;
            query[i] = normalized * inverse_width;
        }
        // Each lane scans its entries in ascending order with a strict >, so it
        // keeps its first maximum; the lanes' winners then merge to the largest
        // value, the lowest index among equals: the serial scan's choice.
        float best = -__builtin_inff();
        int chosen = 1024;
        for (int e = lane; e < 1024; e += lanes)
        {
            float similarity = 0.0f;
#pragma unroll
            for (int i = 0; i < 8; ++i)
            {
                similarity = __builtin_fmaf(book.search[e * 8 + i], query[i], similarity);
            }
            if (similarity > best)
            {
                best = similarity;
                chosen = e;
            }
        }
#pragma unroll
        for (int offset = 1; offset < lanes; offset *= 2)
        {
            const float other = __shfl_xor(best, offset, lanes);
            const int other_index = __shfl_xor(chosen, offset, lanes);
            if (other > best || (other == best && other_index < chosen))
            {
                best = other;
                chosen = other_index;
            }
        }
        const int token = chosen >= 1024 ? 0 : chosen;
        if (lane == 0)
        {
            tokens[std::size_t(frame) * token_stride + b] = uint16_t(token);
        }
        __syncthreads(); // every lane has read the residual for the projection above
        float vector[8];
#pragma unroll
        for (int i = 0; i < 8; ++i)
        {
            vector[i] = book.codebook[token * 8 + i];
        }
        for (int j = lane; j < 1024; j += lanes)
        {
            float sum = 0.0f;
#pragma unroll
            for (int i = 0; i < 8; ++i)
            {
                sum = __builtin_fmaf(book.output_weights[j * 8 + i], vector[i], sum);
            }
            residual[j] = residual[j] - (sum + book.output_bias[j]);
            finite = finite && __builtin_isfinite(residual[j]);
        }
        __syncthreads();
    }
    if (!finite)
    {
        error[0] = 1u;
    }
}

// latent[j][frame] = 0 + the books' projections in book order (src/common/rvq.cpp:84-127).
__global__ __launch_bounds__(256) void rvq_decode_kernel(const RvqBook* books, int count, const uint16_t* tokens,
                                                        int token_stride, int frames, float* latent,
                                                        long long stride, uint32_t* error)
{
    const int j = blockIdx.y * 256 + threadIdx.x, frame = blockIdx.x;
    if (j >= 1024 || frame >= frames)
    {
        return;
    }
    float value = 0.0f;
    for (int b = 0; b < count; ++b)
    {
        const RvqBook book = books[b];
        const int token = tokens[std::size_t(frame) * token_stride + b];
        float sum = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i)
        {
            sum = __builtin_fmaf(book.output_weights[j * 8 + i], book.codebook[token * 8 + i], sum);
        }
        value = value + (sum + book.output_bias[j]);
    }
    latent[j * stride + frame] = value;
    if (!__builtin_isfinite(value))
    {
        error[0] = 1u;
    }
}
} // namespace

void dac_conv_layout(const ConvShape& s, const float* stored, float* out, int out_padded)
{
    std::fill(out, out + std::size_t(s.kernel) * s.in * out_padded, 0.0f);
    for (int tap = 0; tap < s.kernel; ++tap)
    {
        for (int i = 0; i < s.in; ++i)
        {
            for (int o = 0; o < s.out; ++o)
            {
                const std::size_t index = s.transposed ? o + std::size_t(tap) * s.out + std::size_t(i) * s.out * s.kernel
                                                       : i + std::size_t(tap) * s.in + std::size_t(o) * s.in * s.kernel;
                out[(std::size_t(tap) * s.in + i) * out_padded + o] = stored[index];
            }
        }
    }
}

namespace
{
int compute_units()
{
    static const int count = []
    {
        int device = 0, units = 0;
        check_hip(hipGetDevice(&device), "hipGetDevice");
        check_hip(hipDeviceGetAttribute(&units, hipDeviceAttributeMultiprocessorCount, device),
                  "hipDeviceGetAttribute");
        return units > 0 ? units : 1;
    }();
    return count;
}
} // namespace

void dac_conv(const ConvArgs& a, hipStream_t stream)
{
    const ConvShape& s = a.conv.shape;
    require(a.frames > 0 && a.x.data && a.error && (a.out.data || a.activated.data), "dac convolution: arguments");
    require(!a.activated.data || a.alpha, "dac convolution: Snake needs its alpha");
    require(a.conv.out_padded % dac_channel_block == 0 && a.conv.out_padded >= s.out, "dac convolution: layout");
    require(!s.transposed || s.dilation == 1, "dac convolution: dilated transposed convolution");
    require(a.x.phases >= 1 && a.activated.phases >= 1 && a.out.phases == 1 && a.residual.phases == 1,
            "dac convolution: only the input and the Snake output may be polyphase");
    const int out_frames = s.output_frames(a.frames);
    require(out_frames > 0, "dac convolution has no output frames");
    const unsigned tiles = s.transposed
                               ? unsigned(((out_frames + s.stride - 1) / s.stride + lanes - 1) / lanes) * s.stride
                               : unsigned((out_frames + lanes - 1) / lanes);
    // 16 channels per wave while the grid gives every SIMD four waves, else
    // the widest group that gives two, down to 2 (measured on the 400-frame
    // chunks: 8 channels beat 16 at 2,496 waves, 4 lost to 8 at 3,328).
    // A strided (downsampling) convolution on frames in plain order keeps 16:
    // its lanes read frames `stride` apart, so each load touches up to 16
    // cache lines, and fewer channels per load multiply those loads (measured
    // on the 400-frame analysis chunks: 256 -> 512 channels, stride 8, 884 us
    // at 16 channels per wave, 2,478 us at 8). On polyphase input (phases ==
    // stride) its lanes read consecutive addresses.
    const std::size_t simds = std::size_t(compute_units()) * 4;
    const auto waves = [&](int ch) { return std::size_t(tiles) * std::size_t(a.conv.out_padded / ch); };
    const bool strided = !s.transposed && s.stride > 1 && a.x.phases != s.stride;
    const int ch = strided || waves(16) >= 4 * simds ? 16
                   : waves(8) >= 2 * simds             ? 8
                   : waves(4) >= 2 * simds             ? 4
                                                       : 2;
    const unsigned grid_y = unsigned((a.conv.out_padded / ch + conv_waves - 1) / conv_waves);
    const auto launch = [&](auto kernel) { kernel<<<dim3(tiles, grid_y), conv_threads, 0, stream>>>(a); };
    if (s.transposed)
    {
        ch == 16 ? launch(conv_kernel<true, 16>) : ch == 8 ? launch(conv_kernel<true, 8>)
            : ch == 4 ? launch(conv_kernel<true, 4>) : launch(conv_kernel<true, 2>);
    }
    else
    {
        ch == 16 ? launch(conv_kernel<false, 16>) : ch == 8 ? launch(conv_kernel<false, 8>)
            : ch == 4 ? launch(conv_kernel<false, 4>) : launch(conv_kernel<false, 2>);
    }
    check_hip(hipGetLastError(), "dac convolution launch");
}

void rvq_encode(const RvqBook* books, int count, const float* latent, long long stride, int frames, uint16_t* tokens,
                int token_stride, uint32_t* error, hipStream_t stream)
{
    require(count >= 1 && count <= 12 && frames >= 0, "rvq encode: arguments");
    if (!frames)
    {
        return;
    }
    rvq_encode_kernel<<<unsigned(frames), lanes, 0, stream>>>(books, count, latent, stride, frames, tokens,
                                                             token_stride, error);
    check_hip(hipGetLastError(), "rvq encode launch");
}

void rvq_decode(const RvqBook* books, int count, const uint16_t* tokens, int token_stride, int frames, float* latent,
                long long stride, uint32_t* error, hipStream_t stream)
{
    require(count >= 1 && count <= 12 && frames >= 0, "rvq decode: arguments");
    if (!frames)
    {
        return;
    }
    rvq_decode_kernel<<<dim3(unsigned(frames), 4), 256, 0, stream>>>(books, count, tokens, token_stride, frames,
                                                                    latent, stride, error);
    check_hip(hipGetLastError(), "rvq decode launch");
}
} // namespace tsac_hip
