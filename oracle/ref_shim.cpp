// TEST INFRASTRUCTURE ONLY. A C-ABI over the reference's own scalar sources,
// compiled where they lie under the reference tree by oracle/Makefile into
// oracle/_ref/libtsacref.so. Tests use it to pin the C oracle; nothing else
// loads it.
//
// The reference's composition class (CpuTransformer, src/common/cpu_transformer.tpp)
// is not buildable here: it needs TransformerModel, whose sources need the
// generated adapter_offsets.hpp. RefBackend below therefore assembles the same
// layer sequence from the reference's compiled kernels and plugs it into the
// reference's own TransformerPredictor / pack_normal / unpack_normal.
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

struct RefBackend final : TransformerBackend
{
    orc_geometry g;
    std::vector<RefLinear> linears;
    std::vector<std::vector<std::uint16_t>> gain, bias;
    std::vector<std::uint16_t> positions, rotations, embeddings;
    Header header;

    struct Lane
    {
        std::vector<std::vector<std::uint16_t>> tk, tv, ck, cv;
        std::vector<std::uint16_t> conditioning, input, prefix, prefix_tokens, logits, distribution;
        std::vector<float> probabilities, exponents;
    };
    std::vector<Lane> lanes;

    explicit RefBackend(const orc_model_desc& d) : g(d.geometry)
    {
        const std::size_t stacked = 4 * std::size_t(g.temporal_layers + g.codebook_layers);
        for (std::size_t i = 0; i < stacked + 3; ++i)
        {
            std::size_t k, n;
            if (i == stacked || i == stacked + 1)
                k = g.latent, n = g.width;
            else if (i == stacked + 2)
                k = g.width, n = g.alphabet;
            else
                switch (i % 4)
                {
                case 0:
                    k = g.width, n = 3 * std::size_t(g.width);
                    break;
                case 1:
                    k = g.width, n = g.width;
                    break;
                case 2:
                    k = g.width, n = g.ffn;
                    break;
                default:
                    k = g.ffn, n = g.width;
                }
            linears.emplace_back(d.projections[i], k, n);
        }
        const std::size_t norms = 2 * std::size_t(g.temporal_layers + g.codebook_layers) + 2;
        for (std::size_t i = 0; i < norms; ++i)
        {
            gain.emplace_back(d.norm_gain[i], d.norm_gain[i] + g.width);
            bias.emplace_back(d.norm_bias[i], d.norm_bias[i] + g.width);
        }
        positions.assign(d.positions, d.positions + std::size_t(g.books) * g.width);
        rotations.assign(d.rotations, d.rotations + std::size_t(g.context) * g.head_width);
        embeddings.assign(d.embeddings,
                          d.embeddings + std::size_t(g.books) * g.alphabet * g.latent);
    }

    bool independent_lanes() const override
    {
        return true;
    }

    void reset(const Header& h, std::size_t count) override
    {
        validate_header(h);
        header = h;
        lanes.assign(count, {});
        for (auto& l : lanes)
        {
            l.tk.resize(g.temporal_layers);
            l.tv.resize(g.temporal_layers);
            l.ck.resize(g.codebook_layers);
            l.cv.resize(g.codebook_layers);
        }
    }

    void reset_temporal(std::size_t lane) override
    {
        for (auto& k : lanes.at(lane).tk)
            k.clear();
        for (auto& v : lanes.at(lane).tv)
            v.clear();
    }

    void reset_codebook(std::size_t lane) override
    {
        auto& l = lanes.at(lane);
        l.prefix_tokens.clear();
        for (auto& k : l.ck)
            k.clear();
        for (auto& v : l.cv)
            v.clear();
    }

    void embed(std::span<const std::uint16_t> tokens, std::vector<std::uint16_t>& out) const
    {
        out.resize(g.latent);
        for (std::size_t book = 0; book < tokens.size(); ++book)
        {
            const auto e = std::span(embeddings)
                               .subspan((book * g.alphabet + tokens[book]) * g.latent, g.latent);
            if (book == 0)
                std::copy(e.begin(), e.end(), out.begin());
            else
                scalar::add_bf16(out, e);
        }
    }

    // Layer sequence of TransformerGraph::evaluate_stack (src/common/cpu_transformer.tpp:133-175).
    void stack(bool temporal, std::vector<std::uint16_t>& input, std::size_t position,
               const std::uint16_t* rotation, bool replay,
               std::vector<std::vector<std::uint16_t>>& keys,
               std::vector<std::vector<std::uint16_t>>& values) const
    {
        const std::size_t w = g.width, hw = g.head_width;
        const std::size_t layers = temporal ? g.temporal_layers : g.codebook_layers;
        const std::size_t pbase = temporal ? 0 : 4 * std::size_t(g.temporal_layers);
        const std::size_t nbase = temporal ? 0 : 2 * std::size_t(g.temporal_layers) + 1;
        std::vector<std::uint16_t> normalized(w), qkv, query, key, projected, mlp;
        std::vector<float> v(w), sq(w);
        AttentionWorkspace workspace;
        for (std::size_t i = 0; i < layers; ++i)
        {
            const std::size_t p = pbase + 4 * i, n = nbase + 2 * i;
            probability_layer_norm_bf16_into(input, gain[n], bias[n], normalized, v, sq);
            linears[p].apply(normalized, qkv);
            query.assign(qkv.begin(), qkv.begin() + w);
            key.assign(qkv.begin() + w, qkv.begin() + 2 * w);
            if (rotation)
            {
                const std::span<const std::uint16_t> c(rotation, hw);
                for (std::size_t head = 0; head < g.heads; ++head)
                {
                    auto qh = std::span(query).subspan(head * hw, hw);
                    auto kh = std::span(key).subspan(head * hw, hw);
                    probability_rotary_bf16_into(qh, c, qh);
                    probability_rotary_bf16_into(kh, c, kh);
                }
            }
            detail::require(keys[i].size() == position * w, "cache position mismatch");
            keys[i].insert(keys[i].end(), key.begin(), key.end());
            values[i].insert(values[i].end(), qkv.begin() + 2 * w, qkv.end());
            scalar::attention_bf16_into(query, keys[i], values[i], workspace, g.heads, hw,
                                        g.attention_scale, replay, false);
            linears[p + 1].apply(workspace.output, projected);
            scalar::add_bf16(input, projected);
            probability_layer_norm_bf16_into(input, gain[n + 1], bias[n + 1], normalized, v, sq);
            linears[p + 2].apply(normalized, mlp);
            probability_gelu_bf16(std::span(mlp));
            linears[p + 3].apply(mlp, projected);
            scalar::add_bf16(input, projected);
        }
        const std::size_t f = nbase + 2 * layers;
        probability_layer_norm_bf16_into(input, gain[f], bias[f], input, v, sq);
    }

    void temporal_step(std::size_t lane, std::size_t position,
                       std::span<const std::uint16_t> feedback, bool replay) override
    {
        auto& l = lanes.at(lane);
        std::vector<std::uint16_t> embedded;
        embed(feedback, embedded);
        const std::size_t stacked = 4 * std::size_t(g.temporal_layers + g.codebook_layers);
        linears[stacked].apply(embedded, l.conditioning);
        stack(true, l.conditioning, position, rotations.data() + position * g.head_width, replay,
              l.tk, l.tv);
    }

    std::span<const float> codebook_step(std::size_t lane, std::size_t book,
                                         std::span<const std::uint16_t> prefix) override
    {
        auto& l = lanes.at(lane);
        const std::size_t stacked = 4 * std::size_t(g.temporal_layers + g.codebook_layers);
        if (book == 0)
            l.input = l.conditioning;
        else
        {
            embed(prefix, l.prefix);
            linears[stacked + 1].apply(l.prefix, l.input);
        }
        scalar::add_bf16(l.input, std::span(positions).subspan(book * g.width, g.width));
        stack(false, l.input, book, nullptr, false, l.ck, l.cv);
        linears[stacked + 2].apply(l.input, l.logits);
        l.distribution.resize(g.alphabet);
        l.exponents.resize(g.alphabet);
        probability_softmax_bf16_into(l.logits, l.distribution, l.exponents);
        l.probabilities.resize(g.alphabet);
        std::transform(l.distribution.begin(), l.distribution.end(), l.probabilities.begin(),
                       probability_float);
        return l.probabilities;
    }
};

Header header_of(const orc_header& h)
{
    Header r;
    r.method = h.method;
    r.groups = h.groups;
    r.model_channels = h.model_channels;
    r.codebooks = h.codebooks;
    r.frames = h.frames;
    r.batch = h.batch;
    return r;
}

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

int ref_pack_normal(const orc_model_desc* desc, const orc_header* header,
                    const std::uint16_t* tokens, std::size_t count, std::uint8_t* out,
                    std::size_t capacity, std::size_t* written)
{
    return guarded(
        [&]
        {
            RefBackend backend(*desc);
            TransformerPredictor predictor(backend);
            const auto bytes = pack_normal(header_of(*header), std::span(tokens, count), predictor);
            detail::require(bytes.size() <= capacity, "capacity");
            std::memcpy(out, bytes.data(), bytes.size());
            *written = bytes.size();
        });
}

// The reference's pack_normal with an EntropyObserver that records, per symbol
// in the order the observer sees them, before_symbol's position and
// after_symbol's bit count (src/format/entropy.cpp:86-100).
int ref_pack_normal_observed(const orc_model_desc* desc, const orc_header* header,
                             const std::uint16_t* tokens, std::size_t count, std::uint8_t* out,
                             std::size_t capacity, std::size_t* written, std::uint32_t* bits,
                             std::uint64_t* positions)
{
    return guarded(
        [&]
        {
            RefBackend backend(*desc);
            TransformerPredictor predictor(backend);
            std::size_t before = 0, after = 0;
            EntropyObserver observer{
                [&](const EntropyPosition& p)
                {
                    detail::require(before == after && before < count, "observer order");
                    std::uint64_t* r = positions + 6 * before;
                    r[0] = p.frame;
                    r[1] = p.group;
                    r[2] = p.codebook;
                    r[3] = p.lane;
                    r[4] = p.step;
                    r[5] = p.token_offset;
                    ++before;
                },
                [&](const EntropyPosition& p, std::size_t n)
                {
                    detail::require(after + 1 == before && positions[6 * after + 5] == p.token_offset,
                                    "observer order");
                    bits[after++] = static_cast<std::uint32_t>(n);
                }};
            const auto bytes =
                pack_normal(header_of(*header), std::span(tokens, count), predictor, Limits{}, observer);
            detail::require(bytes.size() <= capacity && after == count, "capacity");
            std::memcpy(out, bytes.data(), bytes.size());
            *written = bytes.size();
        });
}

int ref_unpack_normal(const orc_model_desc* desc, const std::uint8_t* bytes, std::size_t length,
                      std::uint16_t* tokens, std::size_t capacity, std::size_t* count)
{
    return guarded(
        [&]
        {
            RefBackend backend(*desc);
            TransformerPredictor predictor(backend);
            const auto t = unpack_normal(ByteView(bytes, length), predictor);
            detail::require(t.size() <= capacity, "capacity");
            std::memcpy(tokens, t.data(), t.size() * 2);
            *count = t.size();
        });
}

int ref_distributions(const orc_model_desc* desc, const orc_header* header,
                      const std::uint16_t* tokens, std::size_t count, std::uint16_t* out)
{
    return guarded(
        [&]
        {
            RefBackend backend(*desc);
            TransformerPredictor predictor(backend);
            auto h = header_of(*header);
            h.method = 1;
            detail::require(count == h.symbol_count(), "token count");
            predictor.reset(h);
            const auto alphabet = desc->geometry.alphabet;
            visit_entropy_positions(h,
                                    [&](const EntropyPosition& p)
                                    {
                                        const auto probs = predictor.predict(p);
                                        for (std::size_t i = 0; i < alphabet; ++i)
                                            out[p.token_offset * alphabet + i] =
                                                probability_bf16(probs[i]);
                                        predictor.commit(p, tokens[p.token_offset]);
                                    });
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
