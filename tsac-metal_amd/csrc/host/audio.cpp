// DAC model preparation, audio framing and the chunked analysis/synthesis
// drivers (audio.hpp, Session::analyze / synthesize / encode_audio / decode_audio).
#include "audio.hpp"

#include <algorithm>
#include <bit>
#include <cmath>
#include <cstring>

namespace tsac_hip
{
namespace
{
constexpr std::size_t hop = 512;
constexpr unsigned analysis_strides[4] = {2, 4, 8, 8}, synthesis_strides[4] = {8, 8, 4, 2};
constexpr unsigned dilations[3] = {1, 3, 9};

float bf16_float(uint16_t bits)
{
    return std::bit_cast<float>(uint32_t(bits) << 16);
}

} // namespace

void fold_dac_weight_norm(std::vector<float>& w, const float* gain, std::size_t fan_in, std::size_t columns)
{
    require(fan_in > 0 && w.size() == fan_in * columns, "weight normalization shape mismatch");
    const float width = static_cast<float>(fan_in);
    const float inverse_width = 1.0f / std::sqrt(width);
    const float reciprocal_width = 1.0f / width;
    std::vector<float> tree(fan_in);
    for (std::size_t c = 0; c < columns; ++c)
    {
        float* column = w.data() + c * fan_in;
        for (std::size_t i = 0; i < fan_in; ++i)
        {
            require(std::isfinite(column[i]) && std::isfinite(gain[c]), "nonfinite weight normalization value");
            tree[i] = column[i] * column[i];
        }
        for (std::size_t n = fan_in; n > 1; n = (n + 1) / 2)
        {
            for (std::size_t i = 0; i < n / 2; ++i)
            {
                tree[i] = tree[2 * i] + tree[2 * i + 1];
            }
            if (n % 2)
            {
                tree[n / 2] = tree[n - 1];
            }
        }
        const float mean = tree[0] * reciprocal_width;
        require(mean > 0 && std::isfinite(mean), "invalid weight normalization norm");
        const float inverse_rms = 1.0f / std::sqrt(mean);
        for (std::size_t i = 0; i < fan_in; ++i)
        {
            const float normalized = column[i] * inverse_rms;
            const float unit = normalized * inverse_width;
            column[i] = unit * gain[c];
            require(std::isfinite(column[i]), "nonfinite weight normalization value");
        }
    }
}

ConvShape dac_conv_shape(bool synthesis, unsigned channels, unsigned index)
{
    require(index < 30 && (channels == 1 || channels == 2), "invalid DAC convolution");
    int first, kernel, last, stride = 1, dilation = 1;
    bool transposed = false;
    if (index == 0)
    {
        first = synthesis ? 1024 : int(channels), kernel = 7, last = synthesis ? 1536 : 64;
    }
    else if (index == 29)
    {
        first = synthesis ? 96 : 1024, kernel = synthesis ? 7 : 3, last = synthesis ? int(channels) : 1024;
    }
    else
    {
        const unsigned stage = (index - 1) / 7, within = (index - 1) % 7;
        const int width = synthesis ? (1536 >> stage) : (64 << stage);
        const int s = int(synthesis ? synthesis_strides[stage] : analysis_strides[stage]);
        if (synthesis && within == 0)
        {
            first = width / 2, kernel = 2 * s, last = width, stride = s, transposed = true;
        }
        else if (!synthesis && within == 6)
        {
            first = width, kernel = 2 * s, last = 2 * width, stride = s;
        }
        else
        {
            const unsigned residual = synthesis ? within - 1 : within;
            const int w = synthesis ? width / 2 : width;
            first = w, last = w, kernel = residual % 2 == 0 ? 7 : 1;
            dilation = residual % 2 == 0 ? int(dilations[residual / 2]) : 1;
        }
    }
    ConvShape s;
    s.in = transposed ? last : first;
    s.out = transposed ? first : last;
    s.kernel = kernel;
    s.stride = stride;
    s.dilation = dilation;
    s.padding = stride == 1 ? (kernel - 1) * dilation / 2 : (stride + 1) / 2;
    s.transposed = transposed;
    return s;
}

std::size_t dac_activation_width(bool synthesis, unsigned index)
{
    require(index < 29, "invalid DAC activation");
    if (index == 28)
    {
        return synthesis ? 96 : 1024;
    }
    return synthesis ? (1536u >> (index / 7)) / (index % 7 == 0 ? 1u : 2u) : (64u << (index / 7));
}

std::vector<float> prepare_dac_convolution(const DacConvolutionSource& source, const ConvShape& shape)
{
    const std::size_t rows = source.dims[0], cols = source.dims[1], outer = source.dims[2];
    const std::size_t first = shape.transposed ? shape.out : shape.in, last = shape.transposed ? shape.in : shape.out;
    require(rows == first && cols == std::size_t(shape.kernel) && outer == last, "unsupported DAC convolution shape");
    require(source.gain && source.bias && (source.values || (source.quantized && source.scales)),
            "missing DAC convolution tensor");
    const std::size_t count = rows * cols * outer;
    std::vector<float> w(count);
    if (source.values)
    {
        std::memcpy(w.data(), source.values, count * sizeof(float));
    }
    else
    {
        // weights::expand_into for BF8 (src/weights/preparation.cpp:31-56).
        require(rows % 32 == 0, "invalid quantized source shape");
        const std::size_t padded = (cols + 7) / 8 * 8;
        for (std::size_t column = 0; column < cols * outer; ++column)
        {
            for (std::size_t b = 0; b < rows / 32; ++b)
            {
                const float scale = bf16_float(source.scales[(column / cols * (rows / 32) + b) * padded + column % cols]);
                for (std::size_t i = 0; i < 32; ++i)
                {
                    const std::size_t k = column * rows + b * 32 + i;
                    w[k] = static_cast<float>(source.quantized[k]) * scale;
                }
            }
        }
    }
    fold_dac_weight_norm(w, source.gain, rows * cols, outer);
    return w;
}

void prepare_rvq(const float* codebook, const float* in_v, const float* in_g, const float* out_v, const float* out_g,
                 float* search, float* input_weights, float* output_weights)
{
    constexpr float epsilon = std::bit_cast<float>(uint32_t{0x2b8cbccc});
    for (std::size_t symbol = 0; symbol < 1024; ++symbol)
    {
        const float* row = codebook + symbol * 8;
        float tree[8];
        for (int i = 0; i < 8; ++i)
        {
            require(std::isfinite(row[i]), "nonfinite RVQ value");
            tree[i] = row[i] * row[i];
        }
        for (int n = 8; n > 1; n /= 2)
        {
            for (int i = 0; i < n / 2; ++i)
            {
                tree[i] = tree[2 * i] + tree[2 * i + 1];
            }
        }
        require(std::isfinite(tree[0]), "invalid RVQ normalization norm");
        const float mean = tree[0] * (1.0f / 8.0f);
        const float inverse_rms = 1.0f / std::sqrt(mean + epsilon);
        const float inverse_width = 1.0f / std::sqrt(8.0f);
        for (int i = 0; i < 8; ++i)
        {
            const float normalized = row[i] * inverse_rms;
            search[symbol * 8 + i] = normalized * inverse_width;
        }
    }
    std::vector<float> w(in_v, in_v + 8192);
    fold_dac_weight_norm(w, in_g, 1024, 8);
    std::memcpy(input_weights, w.data(), 8192 * sizeof(float));
    w.assign(out_v, out_v + 8192);
    fold_dac_weight_norm(w, out_g, 8, 1024);
    std::memcpy(output_weights, w.data(), 8192 * sizeof(float));
}

DacModel::DacModel(unsigned channels, unsigned books, const DacConvolutionSource* analysis,
                   const float* const* analysis_alpha, const DacConvolutionSource* synthesis,
                   const float* const* synthesis_alpha, const RvqSource* rvq, const Limits& limits)
    : channels_(channels), books_(books), limits_(limits)
{
    require(channels == 1 || channels == 2, "DAC model channels must be 1 or 2");
    require(books >= 1 && books <= (channels == 1 ? 9u : 12u), "DAC model codebooks out of range");
    require(analysis && synthesis && analysis_alpha && synthesis_alpha && rvq, "missing DAC model tensor");
    check_hip(hipGetDevice(&device_), "hipGetDevice");
    // Layout: every convolution's w[tap][in][out_padded] and bias, then every
    // activation's alpha, each 256-byte aligned.
    const auto align = [](std::size_t n) { return (n + 255) / 256 * 256; };
    std::size_t bytes = 0;
    std::vector<std::size_t> offsets;
    for (unsigned g = 0; g < 2; ++g)
    {
        for (unsigned i = 0; i < 30; ++i)
        {
            const ConvShape s = dac_conv_shape(g == 1, channels, i);
            const std::size_t padded = (s.out + dac_channel_block - 1) / dac_channel_block * dac_channel_block;
            offsets.push_back(bytes);
            bytes += align(std::size_t(s.kernel) * s.in * padded * 4) + align(std::size_t(s.out) * 4);
        }
    }
    for (unsigned g = 0; g < 2; ++g)
    {
        for (unsigned i = 0; i < 29; ++i)
        {
            offsets.push_back(bytes);
            bytes += align(dac_activation_width(g == 1, i) * 4);
        }
    }
    weights_ = DeviceBuffer(bytes);
    auto* base = weights_.as<uint8_t>();
    std::vector<float> layout;
    for (unsigned g = 0; g < 2; ++g)
    {
        const DacConvolutionSource* sources = g ? synthesis : analysis;
        for (unsigned i = 0; i < 30; ++i)
        {
            const ConvShape s = dac_conv_shape(g == 1, channels, i);
            const int padded = (s.out + dac_channel_block - 1) / dac_channel_block * dac_channel_block;
            const std::vector<float> prepared = prepare_dac_convolution(sources[i], s);
            for (int o = 0; o < s.out; ++o)
            {
                require(std::isfinite(sources[i].bias[o]), "nonfinite DSP value");
            }
            layout.assign(std::size_t(s.kernel) * s.in * padded, 0.0f);
            dac_conv_layout(s, prepared.data(), layout.data(), padded);
            uint8_t* w = base + offsets[g * 30 + i];
            uint8_t* b = w + align(layout.size() * 4);
            check_hip(hipMemcpy(w, layout.data(), layout.size() * 4, hipMemcpyHostToDevice), "upload DAC weights");
            check_hip(hipMemcpy(b, sources[i].bias, std::size_t(s.out) * 4, hipMemcpyHostToDevice), "upload DAC bias");
            convolutions_.push_back({s, reinterpret_cast<const float*>(w), reinterpret_cast<const float*>(b), padded});
        }
    }
    constexpr float epsilon = std::bit_cast<float>(uint32_t{0x3089705f});
    for (unsigned g = 0; g < 2; ++g)
    {
        const float* const* alphas = g ? synthesis_alpha : analysis_alpha;
        for (unsigned i = 0; i < 29; ++i)
        {
            const std::size_t width = dac_activation_width(g == 1, i);
            require(alphas[i] != nullptr, "missing DAC activation");
            for (std::size_t c = 0; c < width; ++c)
            {
                const float a = alphas[i][c];
                require(std::isfinite(a) && std::isfinite(a + epsilon) && a + epsilon != 0.0f,
                        "invalid Snake denominator");
            }
            uint8_t* a = base + offsets[60 + g * 29 + i];
            check_hip(hipMemcpy(a, alphas[i], width * 4, hipMemcpyHostToDevice), "upload DAC alpha");
            alphas_.push_back(reinterpret_cast<const float*>(a));
        }
    }
    // Quantizer tensors, then the device array of RvqBook pointers into them.
    constexpr std::size_t book_floats = 8192 + 8192 + 8192 + 8 + 8192 + 1024;
    rvq_ = DeviceBuffer(align(books * sizeof(RvqBook)) + std::size_t(books) * align(book_floats * 4 + 5 * 256));
    auto* rvq_base = rvq_.as<uint8_t>();
    std::vector<RvqBook> table(books);
    std::size_t cursor = align(books * sizeof(RvqBook));
    for (unsigned b = 0; b < books; ++b)
    {
        const RvqSource& r = rvq[b];
        require(r.codebook && r.search && r.input_weights && r.input_bias && r.output_weights && r.output_bias,
                "missing RVQ tensor");
        const std::pair<const float*, std::size_t> parts[6] = {{r.codebook, 8192}, {r.search, 8192},
                                                               {r.input_weights, 8192}, {r.input_bias, 8},
                                                               {r.output_weights, 8192}, {r.output_bias, 1024}};
        const float* device[6];
        for (int p = 0; p < 6; ++p)
        {
            for (std::size_t i = 0; i < parts[p].second; ++i)
            {
                require(std::isfinite(parts[p].first[i]), "nonfinite RVQ value");
            }
            check_hip(hipMemcpy(rvq_base + cursor, parts[p].first, parts[p].second * 4, hipMemcpyHostToDevice),
                      "upload RVQ tensor");
            device[p] = reinterpret_cast<const float*>(rvq_base + cursor);
            cursor += align(parts[p].second * 4);
        }
        table[b] = {device[0], device[1], device[2], device[3], device[4], device[5]};
    }
    check_hip(hipMemcpy(rvq_base, table.data(), books * sizeof(RvqBook), hipMemcpyHostToDevice), "upload RVQ table");
}

uint16_t select_entropy_batch(std::size_t frames, int requested)
{
    require(requested >= 0 && requested <= 65535, "entropy batch must be 0..65535");
    if (requested)
    {
        return uint16_t(requested);
    }
    std::size_t batch = frames / 1024 + (frames % 1024 != 0);
    if (batch > 8)
    {
        batch = (batch + 7) & ~std::size_t{7};
    }
    return uint16_t(std::clamp<std::size_t>(batch, 1, 128));
}

Header audio_header(std::size_t samples, std::size_t channels, const EncodeOptions& options, const Limits& limits)
{
    require(channels > 0 && channels <= 127, "PCM must have 1..127 channels");
    require(checked_mul(samples, channels) <= limits.tensor_elements, "PCM samples are above Limits::tensor_elements");
    require(options.method <= 1, "coding method must be fast (0) or normal (1)");
    Header h;
    h.method = options.method;
    h.model_channels = channels == 2 && !options.separate_channels ? 2 : 1;
    h.groups = uint8_t(channels / h.model_channels);
    const unsigned maximum = h.model_channels == 2 ? 12 : 9;
    require(options.codebooks <= maximum, "codebook count above the audio model's maximum");
    h.codebooks = uint8_t(options.codebooks ? options.codebooks : maximum);
    h.frames = (samples + hop - 1) / hop;
    require(!options.entropy_batch || *options.entropy_batch > 0, "normal stream header has an entropy batch of 0");
    require(h.method == 1 || !options.entropy_batch, "an entropy batch needs normal coding");
    if (h.method == 1)
    {
        h.batch = select_entropy_batch(h.frames, options.entropy_batch.value_or(0));
    }
    validate_header(h, limits);
    require(checked_mul(h.frames * hop, channels) <= limits.tensor_elements,
            "padded PCM samples are above Limits::tensor_elements");
    return h;
}

std::size_t audio_chunk_frames(std::size_t target, const Limits& limits)
{
    const std::size_t available = limits.tensor_elements / (std::size_t{96} * hop);
    return std::min(target, available > 22 ? available - 22 : std::size_t{1});
}

std::vector<uint8_t> pack_fast(const Header& h, const uint16_t* tokens, std::size_t count, const Limits& limits)
{
    validate_header(h, limits);
    require(h.method == 0, "fast framing needs method 0");
    require(count == h.symbols(), "token count differs from frames x groups x codebooks of the header");
    const std::size_t payload = (checked_mul(count, 10) + 7) / 8;
    require(payload + 8 <= limits.file_bytes, "fast stream would exceed Limits::file_bytes");
    std::vector<uint8_t> bytes{'F', 'B', 'A', 'Z', 0, 0, uint8_t(h.groups | ((h.model_channels - 1) << 7)), h.codebooks};
    bytes.reserve(payload + 8);
    uint32_t pending = 0;
    unsigned held = 0;
    for (std::size_t i = 0; i < count; ++i)
    {
        require(tokens[i] < 1024, "token above 1023: outside the 1024-symbol alphabet");
        pending = (pending << 10) | tokens[i];
        held += 10;
        for (; held >= 8; held -= 8)
        {
            bytes.push_back(uint8_t(pending >> (held - 8)));
        }
        pending &= (1u << held) - 1;
    }
    if (held)
    {
        bytes.push_back(uint8_t(pending << (8 - held)));
    }
    return bytes;
}

std::vector<uint16_t> unpack_fast(const uint8_t* bytes, std::size_t length, const Limits& limits)
{
    const Header h = parse_header(bytes, length, limits);
    require(h.method == 0, "a normal stream needs the probability model to decode");
    std::vector<uint16_t> tokens;
    tokens.reserve(h.symbols());
    uint32_t pending = 0;
    unsigned held = 0;
    for (std::size_t i = 8; i < length; ++i)
    {
        pending = (pending << 8) | bytes[i];
        held += 8;
        if (held >= 10)
        {
            held -= 10;
            tokens.push_back(uint16_t((pending >> held) & 1023));
        }
        pending &= (1u << held) - 1;
    }
    require(tokens.size() == h.symbols(), "fast stream symbol count differs from its header");
    return tokens;
}

// ---------------------------------------------------------------- session drivers

namespace
{
struct Chunk
{
    std::size_t begin, count, left, right;
};

// audio_chunk (src/common/audio_analyzer.cpp:172-181).
Chunk chunk_at(std::size_t begin, std::size_t frames, std::size_t size, std::size_t left_context,
               std::size_t right_context)
{
    const std::size_t count = std::min(size, frames - begin), end = begin + count;
    return {begin, count, begin > left_context ? begin - left_context : 0, end + std::min(right_context, frames - end)};
}

} // namespace

// DacAnalysis::apply (src/common/analysis.tpp:150-190) on `samples` frames of
// `input`: the entry convolution, four stages of three residual units and a
// strided downsampling, the final Snake and the exit convolution, whose
// latent [1024][samples/512] goes to `output`. Every convolution's epilogue
// also writes the Snake its consumer needs, so no activation pass of its own
// runs; `slots` are three buffers of 64 * samples floats.
void Session::analysis_graph(const DacModel& dac, Strided input, int samples, Strided output, float* const* slots)
{
    auto* err = errors_.as<uint32_t>();
    int length = samples;
    int x = 0, s = 1, t = 2;
    const auto signal = [&](int slot, int frames) { return Strided{slots[slot], frames, 1}; };
    // The downsampling input in `phases` planes of frames / phases (frame t
    // of a channel at (t % phases) * frames / phases + t / phases): each
    // plane is one residue of the stride, so the downsampling's lanes read
    // consecutive frames. Chunks hold whole latent frames, so every stage's
    // length is a multiple of its stride.
    const auto polyphase = [&](int slot, int frames, int phases)
    {
        require(frames % phases == 0, "analysis: a stage's length is a multiple of its stride");
        return Strided{slots[slot], frames, 1, phases, frames / phases};
    };
    const auto conv = [&](unsigned index, Strided in, Strided out, Strided activated, unsigned alpha, bool residual)
    {
        ConvArgs a;
        a.conv = dac.convolution(false, index);
        a.x = in;
        a.frames = length;
        a.out = out;
        a.activated = activated;
        a.alpha = activated.data ? dac.alpha(false, alpha) : nullptr;
        if (residual)
        {
            a.residual = out;
        }
        a.error = err;
        dac_conv(a, stream_);
        length = a.conv.shape.output_frames(length);
    };
    const int entry = dac.convolution(false, 0).shape.output_frames(samples);
    conv(0, input, signal(x, entry), signal(s, entry), 0, false);
    for (unsigned stage = 0; stage < 4; ++stage)
    {
        const int stride = dac.convolution(false, 1 + stage * 7 + 6).shape.stride;
        for (unsigned unit = 0; unit < 3; ++unit)
        {
            const unsigned act = stage * 7 + unit * 2, index = 1 + stage * 7 + unit * 2;
            conv(index, signal(s, length), Strided{}, signal(t, length), act + 1, false);
            conv(index + 1, signal(t, length), signal(x, length),
                 unit < 2 ? signal(s, length) : polyphase(s, length, stride), unit < 2 ? act + 2 : stage * 7 + 6,
                 true);
        }
        // downsample: its input (the resample Snake) is in s, polyphase; x is free
        const int down = dac.convolution(false, 1 + stage * 7 + 6).shape.output_frames(length);
        conv(1 + stage * 7 + 6, polyphase(s, length, stride), signal(x, down), signal(t, down),
             stage < 3 ? (stage + 1) * 7 : 28, false);
        std::swap(s, t);
    }
    require(dac.convolution(false, 29).shape.output_frames(length) == samples / int(hop),
            "analysis output length mismatch");
    conv(29, signal(s, length), output, Strided{}, 0, false);
}

// DacSynthesis::apply (src/common/synthesis.tpp:140-180) on `frames` latent
// frames: entry convolution, four stages of a transposed upsampling and three
// residual units, the final Snake and the exit convolution, whose output
// frames [first, last) go to `output`; `slots` hold 96 * 512 * frames floats.
void Session::synthesis_graph(const DacModel& dac, Strided input, int frames, Strided output, int first, int last,
                              float* const* slots)
{
    auto* err = errors_.as<uint32_t>();
    int length = frames;
    int x = 0, s = 1, t = 2;
    const auto signal = [&](int slot, int n) { return Strided{slots[slot], n, 1}; };
    const auto conv = [&](unsigned index, Strided in, Strided out, Strided activated, unsigned alpha, bool residual,
                          int from = 0, int to = 1 << 30)
    {
        ConvArgs a;
        a.conv = dac.convolution(true, index);
        a.x = in;
        a.frames = length;
        a.out = out;
        a.activated = activated;
        a.alpha = activated.data ? dac.alpha(true, alpha) : nullptr;
        if (residual)
        {
            a.residual = out;
        }
        a.error = err;
        a.first = from;
        a.last = to;
        dac_conv(a, stream_);
        length = a.conv.shape.output_frames(length);
    };
    const int entry = dac.convolution(true, 0).shape.output_frames(frames);
    conv(0, input, Strided{}, signal(s, entry), 0, false);
    for (unsigned stage = 0; stage < 4; ++stage)
    {
        const int up = dac.convolution(true, 1 + stage * 7).shape.output_frames(length);
        conv(1 + stage * 7, signal(s, length), signal(x, up), signal(t, up), stage * 7 + 1, false);
        std::swap(s, t);
        for (unsigned unit = 0; unit < 3; ++unit)
        {
            const unsigned act = stage * 7 + 1 + unit * 2, index = 1 + stage * 7 + 1 + unit * 2;
            conv(index, signal(s, length), Strided{}, signal(t, length), act + 1, false);
            conv(index + 1, signal(t, length), signal(x, length), signal(s, length),
                 unit < 2 ? act + 2 : (stage < 3 ? (stage + 1) * 7 : 28), true);
        }
    }
    require(dac.convolution(true, 29).shape.output_frames(length) == frames * int(hop),
            "synthesis output length mismatch");
    conv(29, signal(s, length), output, Strided{}, 0, false, first, last);
}

void Session::dac_apply(const DacModel& dac, bool synthesis, const float* input, std::size_t frames, float* output)
{
    check_hip(hipSetDevice(dac.device()), "hipSetDevice");
    require(dac.device() == model_->device(), "the DAC model and the session are on different devices");
    const std::size_t channels = dac.channels();
    require(frames > 0 && frames < (std::size_t(1) << 30) / hop, "DAC input frames out of range");
    require(synthesis || frames % hop == 0, "analysis PCM must be a nonempty multiple of 512 samples");
    const std::size_t in_count = frames * (synthesis ? 1024 : channels);
    const std::size_t out_count = synthesis ? frames * hop * channels : frames / hop * 1024;
    const std::size_t slot = synthesis ? 96 * hop * frames : 64 * frames;
    auto* d_in = arena_.get<float>("d.in", in_count);
    auto* d_out = arena_.get<float>("d.out", out_count);
    float* slots[3] = {arena_.get<float>("d.0", slot), arena_.get<float>("d.1", slot), arena_.get<float>("d.2", slot)};
    reset_errors();
    upload_input(d_in, input, in_count * sizeof(float));
    if (synthesis)
    {
        synthesis_graph(dac, Strided{d_in, 1, 1024}, int(frames), Strided{d_out, 1, (long long)channels}, 0,
                        int(frames * hop), slots);
    }
    else
    {
        analysis_graph(dac, Strided{d_in, 1, (long long)channels}, int(frames), Strided{d_out, 1, 1024}, slots);
    }
    check_hip(hipMemcpyAsync(output, d_out, out_count * sizeof(float), hipMemcpyDeviceToHost, stream_), "read output");
    check_dsp_errors();
}

void Session::analyze(const DacModel& dac, const float* pcm, std::size_t frames, std::size_t groups,
                      unsigned books, uint16_t* tokens)
{
    check_hip(hipSetDevice(dac.device()), "hipSetDevice");
    require(dac.device() == model_->device(), "the DAC model and the session are on different devices");
    require(books >= 1 && books <= dac.books(), "more codebooks than the DAC model holds");
    const std::size_t channels = dac.channels(), stride = groups * channels, samples = frames * hop;
    if (!frames || !groups)
    {
        return;
    }
    const std::size_t chunk = audio_chunk_frames(400, dac.limits());
    const std::size_t widest = std::min(frames, chunk + 17) * hop;
    auto* d_pcm = arena_.get<float>("a.pcm", samples * stride);
    auto* d_tokens = arena_.get<uint16_t>("a.tokens", frames * groups * books);
    auto* latent = arena_.get<float>("a.latent", 1024 * (widest / hop));
    float* slots[3] = {arena_.get<float>("a.0", 64 * widest), arena_.get<float>("a.1", 64 * widest),
                       arena_.get<float>("a.2", 64 * widest)};
    reset_errors();
    upload_input(d_pcm, pcm, samples * stride * sizeof(float));
    for (std::size_t g = 0; g < groups; ++g)
    {
        for (std::size_t begin = 0; begin < frames;)
        {
            const Chunk c = chunk_at(begin, frames, chunk, 8, 9);
            const int n = int(c.right - c.left);
            analysis_graph(dac, Strided{d_pcm + c.left * hop * stride + g * channels, 1, (long long)stride},
                           n * int(hop), Strided{latent, n, 1}, slots);
            rvq_encode(dac.rvq(), int(books), latent + (c.begin - c.left), n, int(c.count),
                       d_tokens + (c.begin * groups + g) * books, int(groups * books), errors_.as<uint32_t>(), stream_);
            begin += c.count;
        }
    }
    check_hip(hipMemcpyAsync(tokens, d_tokens, frames * groups * books * 2, hipMemcpyDeviceToHost, stream_),
              "read tokens");
    check_dsp_errors();
}

void Session::synthesize(const DacModel& dac, const uint16_t* tokens, std::size_t frames, std::size_t groups,
                         unsigned books, float* pcm)
{
    check_hip(hipSetDevice(dac.device()), "hipSetDevice");
    require(dac.device() == model_->device(), "the DAC model and the session are on different devices");
    require(books >= 1 && books <= dac.books(), "more codebooks than the DAC model holds");
    const std::size_t channels = dac.channels(), stride = groups * channels;
    if (!frames || !groups)
    {
        return;
    }
    for (std::size_t i = 0; i < frames * groups * books; ++i)
    {
        require(tokens[i] < 1024, "token above 1023: outside the 1024-symbol alphabet");
    }
    const std::size_t chunk = audio_chunk_frames(400, dac.limits());
    const std::size_t widest = std::min(frames, chunk + 22);
    auto* d_tokens = arena_.get<uint16_t>("y.tokens", frames * groups * books);
    auto* d_pcm = arena_.get<float>("y.pcm", frames * hop * stride);
    auto* latent = arena_.get<float>("y.latent", 1024 * widest);
    float* slots[3] = {arena_.get<float>("y.0", 96 * hop * widest), arena_.get<float>("y.1", 96 * hop * widest),
                       arena_.get<float>("y.2", 96 * hop * widest)};
    reset_errors();
    upload_input(d_tokens, tokens, frames * groups * books * 2);
    for (std::size_t g = 0; g < groups; ++g)
    {
        for (std::size_t begin = 0; begin < frames;)
        {
            const Chunk c = chunk_at(begin, frames, chunk, 11, 11);
            const int n = int(c.right - c.left);
            rvq_decode(dac.rvq(), int(books), d_tokens + (c.left * groups + g) * books, int(groups * books), n, latent,
                       n, errors_.as<uint32_t>(), stream_);
            // the chunk's central samples straight into the interleaved PCM
            const int first = int((c.begin - c.left) * hop);
            synthesis_graph(dac, Strided{latent, n, 1},
                            n, Strided{d_pcm + c.left * hop * stride + g * channels, 1, (long long)stride}, first,
                            first + int(c.count * hop), slots);
            begin += c.count;
        }
    }
    check_hip(hipMemcpyAsync(pcm, d_pcm, frames * hop * stride * sizeof(float), hipMemcpyDeviceToHost, stream_),
              "read PCM");
    check_dsp_errors();
}

std::vector<uint8_t> Session::encode_audio(const DacModel& dac, const float* samples, std::size_t count,
                                           std::size_t channels, const EncodeOptions& options,
                                           const SymbolObserver* observer)
{
    const double t0 = now();
    const Header h = audio_header(count, channels, options, dac.limits());
    require(h.model_channels == dac.channels(), "PCM channels and the DAC model's channels do not match");
    require(h.codebooks <= dac.books(), "more codebooks than the DAC model holds");
    // padded_audio (src/common/audio_analyzer.cpp:119-140): zeros to a whole frame.
    std::vector<float> padded(h.frames * 512 * channels, 0.0f);
    for (std::size_t i = 0; i < count * channels; ++i)
    {
        require(std::isfinite(samples[i]), "nonfinite PCM sample");
        padded[i] = samples[i];
    }
    std::vector<uint16_t> tokens(h.symbols());
    analyze(dac, padded.data(), h.frames, h.groups, h.codebooks, tokens.data());
    const double t1 = now();
    std::vector<uint8_t> bytes = h.method == 0 ? pack_fast(h, tokens.data(), tokens.size(), dac.limits())
                                               : encode(h, tokens.data(), tokens.size(), observer);
    const auto model = timing_;
    timing_ = {t1 - t0 + (h.method ? model[0] : 0.0), h.method ? model[1] : 0.0, now() - t0, model[3], 0.0, 0.0,
               h.method ? model[6] : -1.0, h.method ? model[7] : 0.0};
    return bytes;
}

std::vector<float> Session::decode_audio(const DacModel& dac, const uint8_t* stream, std::size_t length,
                                         const SymbolObserver* observer, std::size_t* channels)
{
    const double t0 = now();
    const Header h = parse_header(stream, length, dac.limits());
    require(h.model_channels == dac.channels(), "stream and DAC model channels do not match");
    require(h.codebooks <= dac.books(), "more codebooks than the DAC model holds");
    std::vector<uint16_t> tokens = h.method == 0 ? unpack_fast(stream, length, dac.limits())
                                                 : decode(stream, length, observer);
    const auto model = timing_;
    const double t1 = now();
    *channels = std::size_t(h.groups) * h.model_channels;
    std::vector<float> pcm(h.frames * 512 * *channels);
    synthesize(dac, tokens.data(), h.frames, h.groups, h.codebooks, pcm.data());
    timing_ = {now() - t1 + (h.method ? model[0] : 0.0), 0.0, now() - t0, 0.0, model[4], model[5],
               h.method ? model[6] : -1.0, h.method ? model[7] : 0.0};
    return pcm;
}

void Session::check_dsp_errors()
{
    check_hip(hipMemcpyAsync(pinned_errors_.as<uint32_t>(), errors_.get(), 12, hipMemcpyDeviceToHost, stream_),
              "read error words");
    check_hip(hipStreamSynchronize(stream_), "hipStreamSynchronize");
    require(!pinned_errors_.as<uint32_t>()[0], "nonfinite DSP value");
}
} // namespace tsac_hip
