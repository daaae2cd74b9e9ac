// The original TSAC model files (tsac_{mono,stereo}_q8.bin for the probability
// model, dac_{mono,stereo}_q8.bin for the codec): a reader of their record
// format (src/weights/source_model.cpp) and the packer's preparation of their
// tensors (src/weights/pack_main.cpp) into the inputs of Model and DacModel.
#pragma once

#include "audio.hpp"

#include <span>
#include <string>
#include <string_view>

namespace tsac_hip
{
// Tensor storage codes of the record header (src/weights/source_model.hpp:11-17).
enum class Storage : uint32_t
{
    f32 = 0,
    bf16 = 1,
    bf8 = 0x8000b,  // int8 with one BF16 scale per 32 rows of axis 0
    bf8l = 0x8000e, // int8 with one BF16 scale per 256 rows of axis 0
};

// Parser limits (the file-format part of include/tsac/types.hpp:21-31).
struct SourceLimits
{
    std::size_t file_bytes = std::size_t{512} * 1024 * 1024;
    std::size_t tensor_elements = std::size_t{128} * 1024 * 1024;
    std::size_t tensors = 10000;
    std::size_t metadata_bytes = std::size_t{1024} * 1024;
    std::size_t name_bytes = 4096;
};

struct SourceTensor
{
    std::string name;
    Storage storage = Storage::f32;
    std::vector<std::size_t> dims; // axis 0 fastest
    std::size_t elements = 0;
    std::size_t payload_offset = 0, payload_bytes = 0;
    std::size_t data_plane_bytes = 0; // int8 plane (quantized) or the whole payload
};

class SourceModel
{
public:
    static SourceModel parse(std::vector<uint8_t> bytes, const SourceLimits& limits);
    static SourceModel load(const std::string& path, const SourceLimits& limits);

    const std::vector<SourceTensor>& tensors() const
    {
        return tensors_;
    }
    const std::string& metadata() const
    {
        return metadata_;
    }
    const SourceTensor& tensor(std::string_view name) const;
    bool has(std::string_view name) const;
    std::span<const uint8_t> payload(const SourceTensor& tensor) const;
    // Every element as float32 in storage order (src/weights/source_model.cpp:284-329).
    std::vector<float> dequantize(std::string_view name) const;

private:
    std::vector<uint8_t> bytes_;
    std::string metadata_;
    std::vector<SourceTensor> tensors_;
};

// DacConfig of a codec file (src/weights/source_model.cpp:168-213): output
// channels and codebooks (9 mono, 12 stereo), after checking the shapes and the
// quantizer inventory.
struct SourceDacConfig
{
    unsigned channels = 0, books = 0;
};
SourceDacConfig source_dac_config(const SourceModel& dac);
// TransformerConfig (src/weights/source_model.cpp:215-266): the codebook count
// after checking the complete tensor inventory.
unsigned source_transformer_books(const SourceModel& transformer);

// Everything Model's constructor takes, as host pointers.
struct ModelDesc
{
    Geometry geometry;
    const LinearHost* projections = nullptr;
    const uint16_t* const* gain = nullptr;
    const uint16_t* const* bias = nullptr;
    const uint16_t* positions = nullptr;
    const uint16_t* rotations = nullptr;
    const uint16_t* embeddings = nullptr;
};

// The packer's preparation of a probability model (src/weights/pack_main.cpp:305-391):
// int8 projections and their BF16 block scales widened to float32, float32
// biases (zero for cb_proj), LayerNorm gains/biases, codebook positions and the
// rotary table rounded to BF16, and the feedback embeddings, which are the
// codec's codebook projections (project_codebook of every symbol) rounded to
// BF16. The arrays stay owned here; desc() points into them.
class PreparedTransformer
{
public:
    PreparedTransformer(const SourceModel& transformer, const SourceModel& dac);
    const ModelDesc& desc() const
    {
        return desc_;
    }

private:
    struct Linear
    {
        std::vector<int8_t> values;
        std::vector<float> scales, bias;
    };
    std::vector<Linear> linears_;
    std::vector<std::vector<uint16_t>> gains_, biases_;
    std::vector<uint16_t> positions_, rotations_, embeddings_;
    std::vector<LinearHost> projections_;
    std::vector<const uint16_t*> gain_rows_, bias_rows_;
    ModelDesc desc_;
};

// The packer's preparation of a codec (src/weights/pack_main.cpp:172-300): the
// 30 + 30 convolutions as stored (BF8 planes or float32) with their gains and
// biases, the 29 + 29 Snake alphas, and per codebook the codebook, normalised
// search vectors and weight-norm-folded projections.
class PreparedDac
{
public:
    explicit PreparedDac(const SourceModel& dac);
    unsigned channels() const
    {
        return channels_;
    }
    unsigned books() const
    {
        return books_;
    }
    const DacConvolutionSource* analysis() const
    {
        return convolutions_.data();
    }
    const DacConvolutionSource* synthesis() const
    {
        return convolutions_.data() + 30;
    }
    const float* const* analysis_alpha() const
    {
        return alpha_rows_.data();
    }
    const float* const* synthesis_alpha() const
    {
        return alpha_rows_.data() + 29;
    }
    const RvqSource* rvq() const
    {
        return rvq_.data();
    }

private:
    unsigned channels_ = 0, books_ = 0;
    std::vector<std::vector<float>> floats_; // float32 planes, gains, biases, alphas, RVQ
    std::vector<std::vector<int8_t>> quantized_;
    std::vector<std::vector<uint16_t>> scales_;
    std::vector<DacConvolutionSource> convolutions_;
    std::vector<const float*> alpha_rows_;
    std::vector<RvqSource> rvq_;
};
} // namespace tsac_hip
