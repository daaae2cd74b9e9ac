// DAC analysis/synthesis and the residual vector quantizer on the GPU
// (src/common/{analysis,synthesis}.tpp, src/scalar/dsp.cpp, src/common/rvq.{cpp,tpp}).
//
// Every value is computed with the scalar reference's operations in its order:
// a convolution output is one serial sum (taps ascending, input channels
// ascending within a tap, each term a product then an addition, out-of-range
// taps skipped) plus the bias; Snake is x + sin^2(a x) / (a + eps) with the
// reference's own quadrant reduction and polynomials; the RVQ search and
// projections are the reference's ordered FMA chains. So the results are the
// reference CPU path's bits.
//
// Signals are channel-major, signal[c * channel_stride + t * frame_stride], so
// a wave's 64 lanes (consecutive frames) read consecutive addresses; the strides
// also let the first convolution read interleaved PCM and the last write it.
#pragma once

#include "kernels.hpp"

namespace tsac_hip
{
// Output channels one wave computes (weights padded to a multiple).
constexpr int dac_channel_block = 16;

struct ConvShape
{
    int in = 0, out = 0, kernel = 0, stride = 1, padding = 0, dilation = 1;
    bool transposed = false;
    // Convolution::output_frames (src/common/dsp.tpp:157-173).
    __host__ __device__ int output_frames(int frames) const
    {
        const int span = (kernel - 1) * dilation + 1;
        if (!transposed)
        {
            const int padded = frames + 2 * padding;
            return padded < span ? 0 : (padded - span) / stride + 1;
        }
        const int full = (frames - 1) * stride + span;
        return full > 2 * padding ? full - 2 * padding : 0;
    }
};

// Device weights of one convolution: w[tap][in][out_padded] (out fastest,
// out_padded a multiple of dac_channel_block, zero beyond `out`), bias [out].
struct ConvWeights
{
    ConvShape shape;
    const float* w = nullptr;
    const float* bias = nullptr;
    int out_padded = 0;
};

struct Strided
{
    float* data = nullptr;
    long long channel = 0, frame = 0; // element strides
    // Polyphase frames (phases > 1): frame t at (t % phases) * phase + (t / phases) * frame,
    // so a convolution of stride `phases` reads its lanes' frames contiguously.
    // Only a convolution's input and its Snake output may be polyphase.
    int phases = 1;
    long long phase = 0;
};

// y = conv(x) + bias; then optionally y = residual + y; stores y to `out` and
// snake(y) with `alpha` to `activated` (either may be null). error[0] is set when
// a stored value or a Snake phase is not finite.
struct ConvArgs
{
    ConvWeights conv;
    Strided x;
    int frames = 0; // input frames
    Strided residual; // same shape as the output, or data == null
    Strided out;
    Strided activated;
    const float* alpha = nullptr;
    uint32_t* error = nullptr;
    // Output frames outside [first, last) are neither computed nor stored.
    int first = 0, last = 1 << 30;
};

void dac_conv(const ConvArgs& args, hipStream_t stream);

// Host re-layout of a prepared convolution (stored axes, axis 0 fastest:
// ordinary [in, kernel, out], transposed [out, kernel, in]) into w[tap][in][out_padded].
void dac_conv_layout(const ConvShape& shape, const float* stored, float* device_layout, int out_padded);

// RVQ tensors of one codebook on the device.
struct RvqBook
{
    const float* codebook = nullptr;       // [1024][8]
    const float* search = nullptr;         // [1024][8] normalised
    const float* input_weights = nullptr;  // [8][1024]
    const float* input_bias = nullptr;     // [8]
    const float* output_weights = nullptr; // [1024][8]
    const float* output_bias = nullptr;    // [1024]
};

// Up to 12 books, in a device array.
// latent [1024][frames] channel-major (frame stride 1, channel stride `stride`);
// tokens [frame][token_stride] (book b at +b).
void rvq_encode(const RvqBook* books, int count, const float* latent, long long stride, int frames,
                uint16_t* tokens, int token_stride, uint32_t* error, hipStream_t stream);
// latent [1024][frames] (channel stride `stride`) = sum over books of the projections.
void rvq_decode(const RvqBook* books, int count, const uint16_t* tokens, int token_stride, int frames,
                float* latent, long long stride, uint32_t* error, hipStream_t stream);
} // namespace tsac_hip
