// The DAC codec around the probability model: prepared DAC analysis/synthesis
// and quantizer weights on the device (DacModel), and the reference's audio
// framing (src/common/audio_analyzer.cpp: headers, entropy batch, fast framing).
#pragma once

#include "../kernels/dac.hpp"
#include "runtime.hpp"

#include <optional>

namespace tsac_hip
{
// One convolution as the DAC source stores it: dims are the stored axes (axis 0
// fastest; ordinary [in, kernel, out], transposed [out, kernel, in]); either
// float32 `values`, or int8 `quantized` with BF16 `scales` [outer][rows/32][align8(cols)];
// the weight-norm gain per stored column; the bias per output channel.
struct DacConvolutionSource
{
    uint32_t dims[3] = {0, 0, 0};
    const float* values = nullptr;
    const int8_t* quantized = nullptr;
    const uint16_t* scales = nullptr;
    const float* gain = nullptr;
    const float* bias = nullptr;
};

// One quantizer codebook, prepared as the packed RVQ roles hold it
// (src/weights/pack_main.cpp:244-300).
struct RvqSource
{
    const float* codebook = nullptr;       // [1024][8]
    const float* search = nullptr;         // [1024][8]
    const float* input_weights = nullptr;  // [8][1024]
    const float* input_bias = nullptr;     // [8]
    const float* output_weights = nullptr; // [1024][8]
    const float* output_bias = nullptr;    // [1024]
};

// Convolution `index` of a DAC graph (src/models/contract.cpp:55-84, strides
// and dilations of src/common/{analysis,synthesis}.tpp, padding of
// src/common/dsp.tpp:105-113).
ConvShape dac_conv_shape(bool synthesis, unsigned channels, unsigned index);
// Channels of Snake activation `index` (src/models/contract.cpp:109-116).
std::size_t dac_activation_width(bool synthesis, unsigned index);

// The reference runtime's preparation of a DAC convolution
// (src/common/dsp.tpp:117-155): BF8 expansion then DAC weight-norm folding
// (src/weights/normalization.cpp:47-95), into the stored layout.
std::vector<float> prepare_dac_convolution(const DacConvolutionSource& source, const ConvShape& shape);

// fold_dac_weight_norm_into (src/weights/normalization.cpp:47-95), in place on
// `columns` stored columns of `fan_in` values: each column's squares reduced by
// a balanced adjacent-pair tree (an odd tail carried up), RMS-normalised, times
// 1/sqrt(fan_in), times the column's gain.
void fold_dac_weight_norm(std::vector<float>& w, const float* gain, std::size_t fan_in, std::size_t columns);

// The packer's quantizer preparation for one codebook (src/weights/pack_main.cpp:244-300):
// normalize_search of each codebook row (src/weights/preparation.cpp:62-84) and the
// DAC weight-norm folds of in_proj (fan-in 1024) and out_proj (fan-in 8).
void prepare_rvq(const float* codebook, const float* in_v, const float* in_g, const float* out_v, const float* out_g,
                 float* search, float* input_weights, float* output_weights);

class DacModel
{
public:
    DacModel(unsigned channels, unsigned books, const DacConvolutionSource* analysis,
             const float* const* analysis_alpha, const DacConvolutionSource* synthesis,
             const float* const* synthesis_alpha, const RvqSource* rvq, const Limits& limits);
    unsigned channels() const
    {
        return channels_;
    }
    unsigned books() const
    {
        return books_;
    }
    int device() const
    {
        return device_;
    }
    const Limits& limits() const
    {
        return limits_;
    }
    const ConvWeights& convolution(bool synthesis, unsigned index) const
    {
        return convolutions_[synthesis ? 30 + index : index];
    }
    const float* alpha(bool synthesis, unsigned index) const
    {
        return alphas_[synthesis ? 29 + index : index];
    }
    const RvqBook* rvq() const
    {
        return rvq_.as<RvqBook>();
    }

private:
    unsigned channels_, books_;
    int device_ = 0;
    Limits limits_;
    DeviceBuffer weights_, rvq_;
    std::vector<ConvWeights> convolutions_;
    std::vector<const float*> alphas_;
};

// EncodeOptions (include/tsac/audio_analyzer.hpp:16-22).
struct EncodeOptions
{
    uint8_t method = 1; // 0 fast, 1 normal
    unsigned codebooks = 0;
    bool separate_channels = false;
    std::optional<uint16_t> entropy_batch;
};

// select_entropy_batch (src/format/entropy.cpp:10-23).
uint16_t select_entropy_batch(std::size_t frames, int requested);
// audio_header (src/common/audio_analyzer.cpp:78-108) for `samples` frames of
// `channels`-channel PCM.
Header audio_header(std::size_t samples, std::size_t channels, const EncodeOptions& options, const Limits& limits);
// audio_chunk_frames (src/common/audio_analyzer.cpp:166-170).
std::size_t audio_chunk_frames(std::size_t target, const Limits& limits);
// pack_fast / unpack_fast (src/format/container.cpp:82-135): 10-bit symbols, MSB first.
std::vector<uint8_t> pack_fast(const Header& header, const uint16_t* tokens, std::size_t count, const Limits& limits);
std::vector<uint16_t> unpack_fast(const uint8_t* bytes, std::size_t length, const Limits& limits);
} // namespace tsac_hip
