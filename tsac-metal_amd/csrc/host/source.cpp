// Reader of the original model files and the packer's preparation
// (source.hpp). The record layout and the preparation rules are the
// reference's (src/weights/source_model.cpp, src/weights/pack_main.cpp); the
// arithmetic of the prepared values (BF16 rounding, weight-norm folding, the
// codebook projections) is the reference's too, so a model prepared here
// computes what the reference computes from the same files.
#include "source.hpp"

#include <bit>
#include <charconv>
#include <cmath>
#include <cstring>
#include <fstream>
#include <unordered_set>

namespace tsac_hip
{
namespace
{
constexpr uint32_t file_magic = 0x23f4aefb, record_magic = 0x23f4aefa;
constexpr std::size_t record_header = 16, max_rank = 8;

std::size_t align_to(std::size_t n, std::size_t a)
{
    return checked_mul(checked_add(n, a - 1) / a, a);
}

uint32_t read_u32(const std::vector<uint8_t>& bytes, std::size_t offset)
{
    require(offset <= bytes.size() && bytes.size() - offset >= 4, "model file truncated");
    return uint32_t(bytes[offset]) | (uint32_t(bytes[offset + 1]) << 8) | (uint32_t(bytes[offset + 2]) << 16) |
           (uint32_t(bytes[offset + 3]) << 24);
}

float widen_bf16(uint16_t bits)
{
    return std::bit_cast<float>(uint32_t(bits) << 16);
}

// probability_bf16 (src/common/numeric/bf16.hpp:9-13): ties to even on the bits.
uint16_t round_bf16(float value)
{
    const uint32_t b = std::bit_cast<uint32_t>(value);
    return uint16_t((uint64_t(b) + 0x7fff + ((b >> 16) & 1)) >> 16);
}

bool quantized(Storage s)
{
    return s == Storage::bf8 || s == Storage::bf8l;
}

std::size_t block_rows(Storage s)
{
    return s == Storage::bf8 ? 32 : 256;
}

// Where a quantized tensor's BF16 scales sit: one scale per `block` values of
// axis 0, for each column of axis 1 (the column count rounded up to 8 in the
// plane), repeated for every slice of the remaining axes.
struct ScalePlane
{
    std::size_t rows, columns, slices, block, stride;
    std::size_t elements() const
    {
        return checked_mul(checked_mul(rows / block, stride), slices);
    }
};

ScalePlane scale_plane(const SourceTensor& t)
{
    const std::size_t block = block_rows(t.storage);
    require(t.dims.size() >= 2 && t.dims[0] % block == 0,
            "a quantized tensor needs two or more axes, the first a whole number of scale blocks");
    return {t.dims[0], t.dims[1], t.elements / t.dims[0] / t.dims[1], block, align_to(t.dims[1], 8)};
}

uint16_t payload_u16(std::span<const uint8_t> payload, std::size_t offset)
{
    require(offset + 2 <= payload.size(), "tensor payload truncated");
    return uint16_t(payload[offset] | (payload[offset + 1] << 8));
}

void require_dims(const SourceModel& m, const std::string& name, std::initializer_list<std::size_t> dims,
                  const char* what)
{
    require(m.tensor(name).dims == std::vector<std::size_t>(dims), (std::string(what) + ": " + name).c_str());
}
} // namespace

// ---------------------------------------------------------------- the record format

SourceModel SourceModel::load(const std::string& path, const SourceLimits& limits)
{
    std::ifstream file(path, std::ios::binary | std::ios::ate);
    require(bool(file), ("cannot open model file: " + path).c_str());
    const auto end = file.tellg();
    require(end >= 0 && std::size_t(end) <= limits.file_bytes, "model file exceeds the size limit");
    std::vector<uint8_t> bytes(static_cast<std::size_t>(end));
    file.seekg(0);
    require(bytes.empty() || bool(file.read(reinterpret_cast<char*>(bytes.data()), std::streamsize(bytes.size()))),
            "cannot read the whole model file");
    return parse(std::move(bytes), limits);
}

SourceModel SourceModel::parse(std::vector<uint8_t> bytes, const SourceLimits& limits)
{
    require(bytes.size() <= limits.file_bytes, "model file exceeds the size limit");
    require(read_u32(bytes, 0) == file_magic, "not a TSAC model file (magic)");
    const std::size_t metadata = read_u32(bytes, 4);
    require(metadata > 0 && metadata <= limits.metadata_bytes, "model metadata length out of range");
    require(bytes.size() - 8 >= metadata, "model file truncated");
    SourceModel m;
    m.metadata_.assign(reinterpret_cast<const char*>(bytes.data()) + 8, metadata);
    std::unordered_set<std::string> names;
    std::size_t at = 8 + metadata;
    while (at < bytes.size())
    {
        require(m.tensors_.size() < limits.tensors, "too many tensors in the model file");
        require(bytes.size() - at >= record_header, "model file truncated");
        require(read_u32(bytes, at) == record_magic, "bad tensor record (magic)");
        SourceTensor t;
        const uint32_t storage = read_u32(bytes, at + 4);
        require(storage == uint32_t(Storage::f32) || storage == uint32_t(Storage::bf16) ||
                    storage == uint32_t(Storage::bf8) || storage == uint32_t(Storage::bf8l),
                "unsupported tensor storage");
        t.storage = Storage(storage);
        const std::size_t rank = read_u32(bytes, at + 8), name_bytes = read_u32(bytes, at + 12);
        require(rank >= 1 && rank <= max_rank, "tensor rank out of range");
        require(name_bytes >= 1 && name_bytes <= limits.name_bytes, "tensor name length out of range");
        at += record_header;
        t.elements = 1;
        for (std::size_t axis = 0; axis < rank; ++axis)
        {
            const std::size_t d = read_u32(bytes, at);
            require(d > 0, "tensor has an empty axis");
            t.elements = checked_mul(t.elements, d);
            require(t.elements <= limits.tensor_elements, "tensor exceeds the element limit");
            t.dims.push_back(d);
            at += 4;
        }
        require(bytes.size() - at >= name_bytes, "model file truncated");
        t.name.assign(reinterpret_cast<const char*>(bytes.data()) + at, name_bytes);
        for (const char c : t.name)
        {
            require(c >= 32 && c < 127, "tensor name is not printable ASCII");
        }
        require(names.insert(t.name).second, "tensor name appears twice");
        at += name_bytes;
        t.payload_offset = at;
        if (quantized(t.storage))
        {
            t.data_plane_bytes = align_to(t.elements, 256);
            t.payload_bytes = checked_add(t.data_plane_bytes, align_to(checked_mul(scale_plane(t).elements(), 2), 256));
        }
        else
        {
            t.payload_bytes = checked_mul(t.elements, t.storage == Storage::f32 ? 4 : 2);
            t.data_plane_bytes = t.payload_bytes;
        }
        require(bytes.size() - at >= t.payload_bytes, "model file truncated");
        at += t.payload_bytes;
        m.tensors_.push_back(std::move(t));
    }
    require(!m.tensors_.empty(), "model file holds no tensors");
    m.bytes_ = std::move(bytes);
    return m;
}

const SourceTensor& SourceModel::tensor(std::string_view name) const
{
    for (const auto& t : tensors_)
    {
        if (t.name == name)
        {
            return t;
        }
    }
    throw Error("model file has no tensor " + std::string(name));
}

bool SourceModel::has(std::string_view name) const
{
    for (const auto& t : tensors_)
    {
        if (t.name == name)
        {
            return true;
        }
    }
    return false;
}

std::span<const uint8_t> SourceModel::payload(const SourceTensor& t) const
{
    return std::span<const uint8_t>(bytes_.data() + t.payload_offset, t.payload_bytes);
}

std::vector<float> SourceModel::dequantize(std::string_view name) const
{
    const SourceTensor& t = tensor(name);
    const auto p = payload(t);
    std::vector<float> out(t.elements);
    if (t.storage == Storage::f32)
    {
        std::memcpy(out.data(), p.data(), t.elements * 4);
    }
    else if (t.storage == Storage::bf16)
    {
        for (std::size_t i = 0; i < t.elements; ++i)
        {
            out[i] = widen_bf16(payload_u16(p, 2 * i));
        }
    }
    else
    {
        // value[(o*columns + c)*rows + b*block + r] = int8 * scale[(o*rows/block + b)*padded + c]
        const ScalePlane s = scale_plane(t);
        const std::size_t blocks = s.rows / s.block;
        for (std::size_t o = 0; o < s.slices; ++o)
        {
            for (std::size_t c = 0; c < s.columns; ++c)
            {
                for (std::size_t b = 0; b < blocks; ++b)
                {
                    const float scale = widen_bf16(payload_u16(p, t.data_plane_bytes + 2 * ((o * blocks + b) * s.stride + c)));
                    const std::size_t first = (o * s.columns + c) * s.rows + b * s.block;
                    for (std::size_t r = 0; r < s.block; ++r)
                    {
                        out[first + r] = float(std::bit_cast<int8_t>(p[first + r])) * scale;
                    }
                }
            }
        }
    }
    return out;
}

// ---------------------------------------------------------------- configurations

SourceDacConfig source_dac_config(const SourceModel& dac)
{
    const auto& exit = dac.tensor("decoder.model.6.weight_v").dims;
    require(exit.size() == 3 && exit[0] == 96 && exit[1] == 7 && (exit[2] == 1 || exit[2] == 2),
            "unsupported DAC output channels");
    SourceDacConfig config{unsigned(exit[2]), exit[2] == 1 ? 9u : 12u};
    const char* shape = "unsupported DAC tensor shape";
    require_dims(dac, "decoder.model.0.weight_v", {1024, 7, 1536}, shape);
    require_dims(dac, "decoder.model.0.weight_g", {1, 1, 1536}, shape);
    require_dims(dac, "decoder.model.0.bias", {1536}, shape);
    require_dims(dac, "decoder.model.6.weight_g", {1, 1, config.channels}, shape);
    require_dims(dac, "decoder.model.6.bias", {config.channels}, shape);
    for (unsigned book = 0; book < config.books; ++book)
    {
        const std::string q = "quantizer.quantizers." + std::to_string(book);
        require_dims(dac, q + ".codebook.weight", {8, 1024}, shape);
        require_dims(dac, q + ".out_proj.weight_v", {8, 1, 1024}, shape);
        require_dims(dac, q + ".out_proj.weight_g", {1, 1, 1024}, shape);
        require_dims(dac, q + ".out_proj.bias", {1024}, shape);
    }
    // Every quantizer tensor belongs to a book below the count, named without
    // leading zeros.
    constexpr std::string_view prefix = "quantizer.quantizers.";
    for (const auto& t : dac.tensors())
    {
        if (!std::string_view(t.name).starts_with(prefix))
        {
            continue;
        }
        const std::string_view rest = std::string_view(t.name).substr(prefix.size());
        const std::size_t dot = rest.find('.');
        unsigned book = 0;
        const auto parsed = std::from_chars(rest.data(), rest.data() + (dot == rest.npos ? rest.size() : dot), book);
        require(dot != rest.npos && parsed.ec == std::errc{} && parsed.ptr == rest.data() + dot &&
                    book < config.books && rest.substr(0, dot) == std::to_string(book),
                "unsupported DAC quantizer inventory");
    }
    return config;
}

unsigned source_transformer_books(const SourceModel& m)
{
    const auto& wpe = m.tensor("codebook_decoder.wpe").dims;
    require(wpe.size() == 2 && wpe[0] == 512 && (wpe[1] == 9 || wpe[1] == 12),
            "unsupported Transformer codebook positions");
    const unsigned books = unsigned(wpe[1]);
    const char* shape = "unsupported Transformer tensor shape";
    std::size_t count = 0;
    const auto expect = [&](const std::string& name, std::initializer_list<std::size_t> dims)
    {
        require_dims(m, name, dims, shape);
        ++count;
    };
    for (const auto& [stack, layers] : {std::pair<std::string, unsigned>{"", 12}, {"codebook_decoder.", 3}})
    {
        for (unsigned l = 0; l < layers; ++l)
        {
            const std::string h = stack + "h" + std::to_string(l) + "/";
            for (const char* norm : {"ln_1/", "ln_2/"})
            {
                expect(h + norm + "g", {512});
                expect(h + norm + "b", {512});
            }
            expect(h + "attn/c_attn/w", {512, 1536});
            expect(h + "attn/c_attn/b", {1536});
            expect(h + "attn/c_proj/w", {512, 512});
            expect(h + "attn/c_proj/b", {512});
            expect(h + "mlp/c_fc/w", {512, 2048});
            expect(h + "mlp/c_fc/b", {2048});
            expect(h + "mlp/c_proj/w", {2048, 512});
            expect(h + "mlp/c_proj/b", {512});
        }
        expect(stack + "ln_f/g", {512});
        expect(stack + "ln_f/b", {512});
    }
    expect("codebook_decoder.wpe", {512, books});
    expect("cb_proj", {1024, 512});
    expect("codebook_decoder.cb_proj", {1024, 512});
    expect("proj_f/w", {512, 1024});
    expect("proj_f/b", {1024});
    expect("rotary_embed", {128, 1024});
    require(m.tensors().size() == count, "unsupported Transformer tensor inventory");
    return books;
}

// ---------------------------------------------------------------- the probability model

namespace
{
// Projection names in Model's order: 4 per temporal layer, 4 per codebook
// layer, then the two latent projections and the output head
// (src/models/contract.cpp:88-110).
std::vector<std::string> projection_names()
{
    std::vector<std::string> names;
    for (const auto& [stack, layers] : {std::pair<std::string, unsigned>{"", 12}, {"codebook_decoder.", 3}})
    {
        for (unsigned l = 0; l < layers; ++l)
        {
            const std::string h = stack + "h" + std::to_string(l) + "/";
            for (const char* p : {"attn/c_attn/w", "attn/c_proj/w", "mlp/c_fc/w", "mlp/c_proj/w"})
            {
                names.push_back(h + p);
            }
        }
    }
    names.push_back("cb_proj");
    names.push_back("codebook_decoder.cb_proj");
    names.push_back("proj_f/w");
    return names;
}

// Norm stems in Model's order: per temporal layer ln_1, ln_2, then the
// temporal ln_f, per codebook layer ln_1, ln_2, then the codebook ln_f
// (src/models/contract.cpp:201-211).
std::vector<std::string> norm_names()
{
    std::vector<std::string> names;
    for (const auto& [stack, layers] : {std::pair<std::string, unsigned>{"", 12}, {"codebook_decoder.", 3}})
    {
        for (unsigned l = 0; l < layers; ++l)
        {
            names.push_back(stack + "h" + std::to_string(l) + "/ln_1/");
            names.push_back(stack + "h" + std::to_string(l) + "/ln_2/");
        }
        names.push_back(stack + "ln_f/");
    }
    return names;
}

std::vector<uint16_t> bf16_weights(const std::vector<float>& values)
{
    std::vector<uint16_t> out(values.size());
    for (std::size_t i = 0; i < values.size(); ++i)
    {
        out[i] = round_bf16(values[i]);
        require((out[i] & 0x7f80u) != 0x7f80u, "nonfinite BF16 weight");
    }
    return out;
}

void require_finite(const std::vector<float>& values)
{
    for (const float v : values)
    {
        require(std::isfinite(v), "nonfinite prepared weights");
    }
}

// project_codebook (src/weights/preparation.cpp:95-114) with fused products:
// out[j] = fma chain over the 8 coordinates, then the bias.
void project_codebook(std::size_t symbol, const float* codebook, const float* weights, const float* bias, float* out)
{
    for (std::size_t j = 0; j < 1024; ++j)
    {
        float sum = 0.0f;
        for (std::size_t i = 0; i < 8; ++i)
        {
            sum = std::fma(weights[j * 8 + i], codebook[symbol * 8 + i], sum);
        }
        out[j] = sum + bias[j];
        require(std::isfinite(out[j]), "nonfinite RVQ value");
    }
}
} // namespace

PreparedTransformer::PreparedTransformer(const SourceModel& transformer, const SourceModel& dac)
{
    const unsigned books = source_transformer_books(transformer);
    const SourceDacConfig config = source_dac_config(dac);
    require(config.books == books, "the Transformer and DAC files disagree on the codebook count");
    Geometry& g = desc_.geometry;
    g = Geometry{};
    g.books = books;
    g.channels = config.channels;

    // Projections (src/weights/pack_main.cpp:305-361): the BF8L int8 plane is
    // the [N][K] value matrix (axis 0, the input, fastest); scales widen from
    // the padded [K/256][align8(N)] BF16 plane; biases are the "/b" tensors,
    // zero for the cb_proj tensors.
    const auto names = projection_names();
    linears_.resize(names.size());
    for (std::size_t i = 0; i < names.size(); ++i)
    {
        const SourceTensor& t = transformer.tensor(names[i]);
        require(t.storage == Storage::bf8l, "Transformer projections must be BF8L");
        const auto [K, N] = g.projection_shape(i);
        require(t.dims.size() == 2 && t.dims[0] == K && t.dims[1] == N, "unsupported Transformer packing shape");
        const auto p = transformer.payload(t);
        Linear& l = linears_[i];
        l.values.resize(K * N);
        std::memcpy(l.values.data(), p.data(), K * N);
        const std::size_t padded = align_to(N, 8);
        l.scales.resize(K / 256 * N);
        for (std::size_t b = 0; b < K / 256; ++b)
        {
            for (std::size_t n = 0; n < N; ++n)
            {
                l.scales[b * N + n] = widen_bf16(payload_u16(p, t.data_plane_bytes + 2 * (b * padded + n)));
            }
        }
        if (names[i].ends_with("/w"))
        {
            l.bias = transformer.dequantize(names[i].substr(0, names[i].size() - 1) + "b");
        }
        else
        {
            l.bias.assign(N, 0.0f);
        }
        require_finite(l.scales);
        require_finite(l.bias);
        projections_.push_back({l.values.data(), l.scales.data(), l.bias.data()});
    }
    // Norms, positions and the rotary table as BF16 (src/weights/pack_main.cpp:362-370).
    for (const auto& stem : norm_names())
    {
        gains_.push_back(bf16_weights(transformer.dequantize(stem + "g")));
        biases_.push_back(bf16_weights(transformer.dequantize(stem + "b")));
    }
    for (std::size_t i = 0; i < gains_.size(); ++i)
    {
        gain_rows_.push_back(gains_[i].data());
        bias_rows_.push_back(biases_[i].data());
    }
    positions_ = bf16_weights(transformer.dequantize("codebook_decoder.wpe")); // [books][512]
    rotations_ = bf16_weights(transformer.dequantize("rotary_embed"));         // [1024][128]
    // Feedback embeddings (src/weights/pack_main.cpp:372-389): every symbol's
    // codebook projection through the weight-norm-folded out_proj, as BF16.
    embeddings_.resize(std::size_t(books) * 1024 * 1024);
    std::vector<float> column(1024);
    for (unsigned book = 0; book < books; ++book)
    {
        const std::string q = "quantizer.quantizers." + std::to_string(book);
        const auto codebook = dac.dequantize(q + ".codebook.weight");
        auto w = dac.dequantize(q + ".out_proj.weight_v");
        const auto gain = dac.dequantize(q + ".out_proj.weight_g");
        const auto bias = dac.dequantize(q + ".out_proj.bias");
        fold_dac_weight_norm(w, gain.data(), 8, 1024);
        for (std::size_t symbol = 0; symbol < 1024; ++symbol)
        {
            project_codebook(symbol, codebook.data(), w.data(), bias.data(), column.data());
            uint16_t* row = embeddings_.data() + (std::size_t(book) * 1024 + symbol) * 1024;
            for (std::size_t j = 0; j < 1024; ++j)
            {
                row[j] = round_bf16(column[j]);
            }
        }
    }
    desc_.projections = projections_.data();
    desc_.gain = gain_rows_.data();
    desc_.bias = bias_rows_.data();
    desc_.positions = positions_.data();
    desc_.rotations = rotations_.data();
    desc_.embeddings = embeddings_.data();
}

// ---------------------------------------------------------------- the codec

namespace
{
// Tensor stems of a DAC graph's 30 convolutions and 29 Snake activations in
// graph order (src/weights/pack_main.cpp:580-610): the entry convolution;
// per stage (analysis) three residual units (k7, k1) and the downsampling, or
// (synthesis) the upsampling and three residual units; the exit convolution.
struct GraphNames
{
    std::vector<std::string> convolutions, activations;
};

GraphNames graph_names(bool synthesis)
{
    const std::string prefix = synthesis ? "decoder.model." : "encoder.block.";
    GraphNames n;
    n.convolutions.push_back(prefix + "0");
    for (unsigned stage = 0; stage < 4; ++stage)
    {
        const std::string block = prefix + std::to_string(stage + 1) + ".block.";
        if (synthesis)
        {
            n.activations.push_back(block + "0");
            n.convolutions.push_back(block + "1");
        }
        for (unsigned unit = 0; unit < 3; ++unit)
        {
            const std::string residual = block + std::to_string(unit + (synthesis ? 2 : 0)) + ".block.";
            n.activations.push_back(residual + "0");
            n.convolutions.push_back(residual + "1");
            n.activations.push_back(residual + "2");
            n.convolutions.push_back(residual + "3");
        }
        if (!synthesis)
        {
            n.activations.push_back(block + "3");
            n.convolutions.push_back(block + "4");
        }
    }
    n.activations.push_back(prefix + "5");
    n.convolutions.push_back(prefix + "6");
    return n;
}
} // namespace

PreparedDac::PreparedDac(const SourceModel& dac)
{
    const SourceDacConfig config = source_dac_config(dac);
    channels_ = config.channels;
    books_ = config.books;
    const float snake_epsilon = std::bit_cast<float>(uint32_t{0x3089705f});
    const auto keep = [&](std::vector<float> v) -> const float*
    {
        floats_.push_back(std::move(v));
        return floats_.back().data();
    };
    // The stored planes are kept as they are; DacModel expands and folds them
    // (src/common/dsp.tpp:117-155), the packer only checks that it can
    // (src/weights/pack_main.cpp:184-193).
    for (bool synthesis : {false, true})
    {
        const GraphNames names = graph_names(synthesis);
        for (unsigned i = 0; i < 30; ++i)
        {
            const std::string& stem = names.convolutions[i];
            const SourceTensor& v = dac.tensor(stem + ".weight_v");
            const ConvShape shape = dac_conv_shape(synthesis, channels_, i);
            const std::vector<std::size_t> dims =
                shape.transposed ? std::vector<std::size_t>{std::size_t(shape.out), std::size_t(shape.kernel), std::size_t(shape.in)}
                                 : std::vector<std::size_t>{std::size_t(shape.in), std::size_t(shape.kernel), std::size_t(shape.out)};
            require(v.dims == dims, ("unsupported DAC convolution shape: " + stem).c_str());
            require(v.storage == Storage::f32 || v.storage == Storage::bf8, "DAC convolutions must be float32 or BF8");
            require_dims(dac, stem + ".weight_g", {1, 1, dims[2]}, "unsupported DAC gain shape");
            require_dims(dac, stem + ".bias", {std::size_t(shape.out)}, "unsupported DAC bias shape");
            DacConvolutionSource c;
            for (int a = 0; a < 3; ++a)
            {
                c.dims[a] = uint32_t(dims[a]);
            }
            const auto p = dac.payload(v);
            if (v.storage == Storage::f32)
            {
                c.values = keep(dac.dequantize(v.name));
            }
            else
            {
                quantized_.emplace_back(v.elements);
                std::memcpy(quantized_.back().data(), p.data(), v.elements);
                c.quantized = quantized_.back().data();
                const std::size_t count = scale_plane(v).elements();
                scales_.emplace_back(count);
                for (std::size_t k = 0; k < count; ++k)
                {
                    scales_.back()[k] = payload_u16(p, v.data_plane_bytes + 2 * k);
                }
                c.scales = scales_.back().data();
            }
            c.gain = keep(dac.dequantize(stem + ".weight_g"));
            c.bias = keep(dac.dequantize(stem + ".bias"));
            convolutions_.push_back(c);
        }
        for (unsigned i = 0; i < 29; ++i)
        {
            const std::string name = names.activations[i] + ".alpha";
            require_dims(dac, name, {dac_activation_width(synthesis, i), 1, 1}, "unsupported DAC activation shape");
            auto alpha = dac.dequantize(name);
            for (const float a : alpha)
            {
                require(std::isfinite(a + snake_epsilon) && a + snake_epsilon != 0.0f, "invalid Snake denominator");
            }
            alpha_rows_.push_back(keep(std::move(alpha)));
        }
    }
    // Quantizer (src/weights/pack_main.cpp:244-300): codebook, normalised search
    // vectors, weight-norm-folded input and output projections, biases.
    for (unsigned book = 0; book < books_; ++book)
    {
        const std::string q = "quantizer.quantizers." + std::to_string(book);
        require_dims(dac, q + ".in_proj.weight_v", {1024, 1, 8}, "unsupported DAC tensor shape");
        require_dims(dac, q + ".in_proj.weight_g", {1, 1, 8}, "unsupported DAC tensor shape");
        require_dims(dac, q + ".in_proj.bias", {8}, "unsupported DAC tensor shape");
        const auto codebook = dac.dequantize(q + ".codebook.weight");
        const auto in_v = dac.dequantize(q + ".in_proj.weight_v");
        const auto in_g = dac.dequantize(q + ".in_proj.weight_g");
        const auto out_v = dac.dequantize(q + ".out_proj.weight_v");
        const auto out_g = dac.dequantize(q + ".out_proj.weight_g");
        std::vector<float> search(8192), input(8192), output(8192);
        prepare_rvq(codebook.data(), in_v.data(), in_g.data(), out_v.data(), out_g.data(), search.data(),
                    input.data(), output.data());
        RvqSource r;
        r.codebook = keep(codebook);
        r.search = keep(std::move(search));
        r.input_weights = keep(std::move(input));
        r.input_bias = keep(dac.dequantize(q + ".in_proj.bias"));
        r.output_weights = keep(std::move(output));
        r.output_bias = keep(dac.dequantize(q + ".out_proj.bias"));
        rvq_.push_back(r);
    }
}
} // namespace tsac_hip
