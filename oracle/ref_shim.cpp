// TEST INFRASTRUCTURE ONLY. A C-ABI over the reference's own scalar kernels,
// numerics, range coder, source-file reader, audio files and command line,
// compiled where they lie under the reference tree by oracle/Makefile into
// oracle/_ref/libtsacref.so. Tests use it to pin the C oracle function by
// function; nothing else loads it. The reference's composition classes
// (CpuTransformer, the DAC graphs, the quantizer) are in ref_model.cpp.
#include "common/numeric.hpp"
#include "common/numeric/probability.hpp"
#include "common/probability.hpp"
#include "common/transformer.hpp"
#include "format/categorical.hpp"
#include "format/container.hpp"
#include "format/entropy.hpp"
#include "format/range.hpp"
#include "scalar/kernels.hpp"
#include "scalar/dsp.hpp"
#include "weights/normalization.hpp"
#include "weights/preparation.hpp"
#include "weights/source_model.hpp"
#include "audio.hpp"
#include "cli.hpp"

#include "tsac_oracle.h"

#include <algorithm>
#include <cstring>
#include <string>

using namespace tsac;

namespace tsac
{
// Defined in src/common/rvq.cpp, declared there only by src/common/rvq.tpp.
std::uint16_t nearest_rvq_index(std::span<const float, 8> input, std::span<const float> vectors);
} // namespace tsac

namespace
{
thread_local std::string last_error;

template <class F> int guarded(F&& f)
{
    try
    {
        f();
        return 0;
    }
    catch (const std::exception& e)
    {
        last_error = e.what();
        return 1;
    }
}

// R4 interleave of src/common/packed_linear.tpp:56-72, the layout that
// scalar::Kernels::linear_column indexes.
std::vector<std::int8_t> r4(const std::int8_t* values, std::size_t input, std::size_t output)
{
    std::vector<std::int8_t> packed(input * output);
    for (std::size_t out = 0; out < output; out += 4)
        for (std::size_t b = 0; b < input / 256; ++b)
            for (std::size_t q = 0; q < 64; ++q)
                for (std::size_t row = 0; row < 4; ++row)
                    std::memcpy(packed.data() + out * input + b * 1024 + q * 16 + row * 4,
                                values + (out + row) * input + b * 256 + q * 4, 4);
    return packed;
}

struct RefLinear
{
    std::size_t input = 0, output = 0;
    std::vector<std::int8_t> weights;
    std::vector<float> scales, bias;

    RefLinear() = default;
    RefLinear(const orc_linear& l, std::size_t k, std::size_t n)
        : input(k), output(n), weights(r4(l.values, k, n)), scales(l.scales, l.scales + k / 256 * n),
          bias(l.bias, l.bias + n)
    {
    }

    // The glue of PackedLinear::apply_into (src/common/packed_linear.tpp:264-302).
    void apply(std::span<const std::uint16_t> x, std::vector<std::uint16_t>& y) const
    {
        const auto columns = x.size() / input;
        std::vector<float> expanded(x.size());
        for (std::size_t i = 0; i < x.size(); ++i)
            expanded[i] = probability_float(x[i]);
        const auto quantized = scalar::bf8l(expanded);
        std::vector<float> activation_scales(quantized.scales.size());
        for (std::size_t i = 0; i < activation_scales.size(); ++i)
            activation_scales[i] = probability_float(quantized.scales[i]);
        y.resize(columns * output);
        const auto blocks = input / 256;
        for (std::size_t c = 0; c < columns; ++c)
            scalar::Kernels::linear_column(
                weights, scales, bias, input, output,
                std::span(quantized.values).subspan(c * input, input),
                std::span(activation_scales).subspan(c * blocks, blocks),
                std::span(y).subspan(c * output, output));
    }
};

} // namespace

extern "C"
{
const char* ref_last_error()
{
    return last_error.c_str();
}

std::uint16_t ref_bf16(float x)
{
    return probability_bf16(x);
}

float ref_exp(float z)
{
    return detail::probability::original_exp(z);
}

void ref_exp_batch(const float* z, std::size_t count, float* out)
{
    for (std::size_t i = 0; i < count; ++i)
        out[i] = detail::probability::original_exp(z[i]);
}

void ref_bf16_batch(const float* x, std::size_t count, std::uint16_t* out)
{
    for (std::size_t i = 0; i < count; ++i)
        out[i] = probability_bf16(x[i]);
}

float ref_probability_sum(const float* values, std::size_t count)
{
    return probability_sum(std::span(values, count));
}

std::uint16_t ref_conditional_q15(float left, float mass)
{
    return conditional_q15(left, mass);
}

int ref_bf8l(const float* values, std::size_t count, std::int8_t* q, std::uint16_t* scales)
{
    return guarded(
        [&]
        {
            const auto r = scalar::bf8l(std::span(values, count));
            std::memcpy(q, r.values.data(), count);
            std::memcpy(scales, r.scales.data(), r.scales.size() * 2);
        });
}

int ref_qlinear(const std::int8_t* w, const float* ws, const float* bias, std::size_t K,
                std::size_t N, const std::uint16_t* x, std::size_t M, std::uint16_t* y)
{
    return guarded(
        [&]
        {
            const orc_linear l{w, ws, bias};
            RefLinear linear(l, K, N);
            std::vector<std::uint16_t> out;
            linear.apply(std::span(x, M * K), out);
            std::memcpy(y, out.data(), out.size() * 2);
        });
}

int ref_layer_norm(const std::uint16_t* x, const std::uint16_t* gain, const std::uint16_t* bias,
                   std::size_t n, std::uint16_t* out)
{
    return guarded(
        [&]
        {
            const auto r = probability_layer_norm_bf16(std::span(x, n), std::span(gain, n),
                                                       std::span(bias, n));
            std::memcpy(out, r.data(), n * 2);
        });
}

std::uint16_t ref_gelu(std::uint16_t x)
{
    return probability_gelu_bf16(x);
}

void ref_gelu_table(std::uint16_t* values, std::size_t n)
{
    probability_gelu_bf16(std::span(values, n));
}

std::uint16_t ref_add_bf16(std::uint16_t a, std::uint16_t b)
{
    return probability_add_bf16(a, b);
}

int ref_rotary(const std::uint16_t* v, const std::uint16_t* c, std::size_t n, std::uint16_t* out)
{
    return guarded(
        [&]
        {
            const auto r = probability_rotary_bf16(std::span(v, n), std::span(c, n));
            std::memcpy(out, r.data(), n * 2);
        });
}

int ref_softmax(const std::uint16_t* x, std::size_t n, std::uint16_t* out)
{
    return guarded(
        [&]
        {
            const auto r = probability_softmax_bf16(std::span(x, n));
            std::memcpy(out, r.data(), n * 2);
        });
}

int ref_attention(const std::uint16_t* q, const std::uint16_t* k, const std::uint16_t* v,
                  std::size_t time, std::size_t heads, std::size_t hw, float scale, int prefill,
                  std::uint16_t* out)
{
    return guarded(
        [&]
        {
            const auto width = heads * hw;
            const auto r = scalar::attention_bf16(std::span(q, width), std::span(k, time * width),
                                                  std::span(v, time * width), heads, hw, scale,
                                                  prefill != 0, false);
            std::memcpy(out, r.data(), width * 2);
        });
}

std::uint32_t ref_token_crc32(const std::uint16_t* tokens, std::size_t count)
{
    return token_crc32(std::span(tokens, count));
}

int ref_range_encode(const float* probabilities, const std::uint16_t* symbols, std::size_t count,
                     std::size_t alphabet, std::uint8_t* out, std::size_t capacity,
                     std::size_t* written)
{
    return guarded(
        [&]
        {
            RangeEncoder encoder;
            for (std::size_t i = 0; i < count; ++i)
                encode_categorical(encoder, std::span(probabilities + i * alphabet, alphabet),
                                   symbols[i]);
            const auto bytes = encoder.finish();
            detail::require(bytes.size() <= capacity, "capacity");
            std::memcpy(out, bytes.data(), bytes.size());
            *written = bytes.size();
        });
}

// ---- DAC and RVQ primitives (src/scalar/dsp.cpp, src/weights/*.cpp, src/common/rvq.cpp)

int ref_conv1d(const orc_conv* c, const float* w, const float* bias, const float* x, std::size_t frames,
               std::size_t groups, float* y)
{
    return guarded(
        [&]
        {
            const Conv1dConfig config{c->in, c->out, c->kernel, c->stride, c->padding, c->dilation,
                                      c->transposed ? ConvolutionKind::transposed : ConvolutionKind::ordinary};
            const std::size_t count = c->in * c->kernel * c->out;
            const scalar::Conv1d conv(config, std::span(w, count), std::span(bias, c->out));
            const auto out = conv.apply(std::span(x, frames * groups * c->in), SignalShape{c->in, frames, groups});
            std::memcpy(y, out.values.data(), out.values.size() * sizeof(float));
        });
}

int ref_snake(const float* x, std::size_t count, std::size_t channels, const float* alpha, float* out)
{
    return guarded(
        [&]
        {
            Signal result;
            scalar::snake_dac_into(std::span(x, count), SignalShape{channels, count / channels, 1},
                                   std::span(alpha, channels), result);
            std::memcpy(out, result.values.data(), count * sizeof(float));
        });
}

int ref_fold_dac_weight_norm(const float* v, const float* g, std::size_t fan_in, std::size_t columns, float* out)
{
    return guarded(
        [&]
        {
            const auto w = fold_dac_weight_norm(std::span(v, fan_in * columns), std::span(g, columns), fan_in);
            std::memcpy(out, w.data(), w.size() * sizeof(float));
        });
}

void ref_normalize_search(const float* input, float* output)
{
    weights::normalize_search(std::span<const float, 8>(input, 8), std::span<float, 8>(output, 8));
}

std::uint16_t ref_nearest_rvq(const float* input, const float* vectors)
{
    return nearest_rvq_index(std::span<const float, 8>(input, 8), std::span(vectors, 8192));
}

void ref_project_codebook(std::uint16_t index, const float* codebook, const float* weights, const float* bias,
                          float* out)
{
    weights::project_codebook(index, std::span(codebook, 8192), std::span(weights, 8192), std::span(bias, 1024),
                              std::span(out, 1024), true);
}

// SourceModel (src/weights/source_model.cpp) on an in-memory file: 0 when it
// parses (tensor count to *tensors), nonzero when the reference rejects it.
int ref_source_parse(const std::uint8_t* bytes, std::size_t length, std::uint64_t file_bytes,
                     std::uint64_t metadata_bytes, std::size_t* tensors)
{
    return guarded(
        [&]
        {
            Limits limits;
            if (file_bytes)
            {
                limits.file_bytes = file_bytes;
            }
            if (metadata_bytes)
            {
                limits.metadata_bytes = metadata_bytes;
            }
            const auto model = packing::SourceModel::parse(Bytes(bytes, bytes + length), limits);
            *tensors = model.tensors().size();
        });
}

int ref_source_dequantize(const std::uint8_t* bytes, std::size_t length, const char* name, float* out,
                          std::size_t capacity)
{
    return guarded(
        [&]
        {
            const auto model = packing::SourceModel::parse(Bytes(bytes, bytes + length));
            const auto values = model.dequantize(name);
            detail::require(values.size() <= capacity, "capacity");
            std::memcpy(out, values.data(), values.size() * sizeof(float));
        });
}

int ref_source_configs(const std::uint8_t* bytes, std::size_t length, unsigned* channels, unsigned* dac_books,
                       unsigned* transformer_books)
{
    return guarded(
        [&]
        {
            const auto model = packing::SourceModel::parse(Bytes(bytes, bytes + length));
            *channels = *dac_books = *transformer_books = 0;
            try
            {
                const auto c = model.dac_config();
                *channels = c.channels;
                *dac_books = c.codebooks;
            }
            catch (const std::exception&)
            {
            }
            try
            {
                *transformer_books = model.transformer_config().codebooks;
            }
            catch (const std::exception&)
            {
            }
        });
}

// The command-line codec's audio files and options (src/audio.cpp, src/cli.cpp).
int ref_pcm16_input(const std::uint8_t* bytes, std::size_t length, unsigned channels, float* out,
                    std::size_t capacity, std::size_t* frames)
{
    return guarded(
        [&]
        {
            const auto signal = pcm16_input(ByteView(bytes, length), channels);
            detail::require(signal.values.size() <= capacity, "capacity");
            std::memcpy(out, signal.values.data(), signal.values.size() * sizeof(float));
            *frames = signal.shape.frames;
        });
}

int ref_wave_input(const std::uint8_t* bytes, std::size_t length, float* out, std::size_t capacity,
                   std::size_t* frames, unsigned* channels)
{
    return guarded(
        [&]
        {
            const auto signal = wave_input(ByteView(bytes, length));
            detail::require(signal.values.size() <= capacity, "capacity");
            std::memcpy(out, signal.values.data(), signal.values.size() * sizeof(float));
            *frames = signal.shape.frames;
            *channels = unsigned(signal.shape.channels);
        });
}

int ref_pcm16_wave(const float* samples, std::size_t frames, unsigned channels, std::uint64_t pcm_bytes,
                   std::uint8_t* out, std::size_t capacity, std::size_t* length)
{
    return guarded(
        [&]
        {
            Limits limits;
            if (pcm_bytes)
            {
                limits.pcm_bytes = pcm_bytes;
            }
            const auto bytes = pcm16_wave(std::span(samples, frames * channels), {channels, frames, 1}, limits);
            detail::require(bytes.size() <= capacity, "capacity");
            std::memcpy(out, bytes.data(), bytes.size());
            *length = bytes.size();
        });
}

// parse_cli: fields [command, threads, quality, channels, batch, verbose, fast,
// separate, help, metal, input index, output index] (-1 for an absent path).
int ref_parse_cli(std::size_t count, const char* const* arguments, long long* fields)
{
    return guarded(
        [&]
        {
            std::vector<std::string_view> args(arguments, arguments + count);
            const auto o = parse_cli(args);
            const auto index = [&](const std::filesystem::path& p) -> long long
            {
                if (p.empty())
                {
                    return -1;
                }
                for (std::size_t i = 0; i < count; ++i)
                {
                    if (p == std::filesystem::path(arguments[i]))
                    {
                        return (long long)i;
                    }
                }
                return -2;
            };
            const long long values[12] = {o.command, o.threads, o.quality, o.channels, o.batch, o.verbose,
                                          o.fast,    o.separate, o.help,  o.metal,    index(o.input),
                                          index(o.output)};
            std::memcpy(fields, values, sizeof values);
        });
}
}
