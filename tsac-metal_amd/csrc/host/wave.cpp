// Audio files and options of the command-line codec (wave.hpp).
#include "wave.hpp"

#include <charconv>
#include <cmath>
#include <cstring>
#include <limits>

namespace tsac_hip
{
namespace
{
constexpr uint32_t sample_rate = 44100;

bool has_tag(const uint8_t* bytes, std::size_t length, std::size_t offset, const char* tag)
{
    require(offset <= length && length - offset >= 4, "invalid wav file");
    return std::memcmp(bytes + offset, tag, 4) == 0;
}

uint32_t le32_at(const uint8_t* bytes, std::size_t length, std::size_t offset)
{
    require(offset <= length && length - offset >= 4, "invalid wav file");
    return uint32_t(bytes[offset]) | (uint32_t(bytes[offset + 1]) << 8) | (uint32_t(bytes[offset + 2]) << 16) |
           (uint32_t(bytes[offset + 3]) << 24);
}
} // namespace

Pcm pcm16_input(const uint8_t* bytes, std::size_t length, unsigned channels, const Limits& limits)
{
    require(channels >= 1 && channels <= 127, "unsupported number of channels");
    const std::size_t frame_bytes = 2 * std::size_t(channels);
    const std::size_t frames = length / frame_bytes;
    const std::size_t padded = checked_mul(checked_add(frames, 511) / 512, 512);
    const std::size_t count = checked_mul(padded, channels);
    require(checked_mul(count, 2) <= limits.pcm_bytes && count <= limits.tensor_elements,
            "input PCM exceeds the size limits");
    Pcm pcm{channels, padded, std::vector<float>(count, 0.0f)};
    for (std::size_t i = 0; i < frames * channels; ++i)
    {
        const int16_t s = int16_t(uint16_t(bytes[2 * i] | (bytes[2 * i + 1] << 8)));
        pcm.samples[i] = float(s) * (1.0f / 32768.0f);
    }
    return pcm;
}

Pcm wave_input(const uint8_t* bytes, std::size_t length, const Limits& limits)
{
    require(has_tag(bytes, length, 0, "RIFF") && has_tag(bytes, length, 8, "WAVE"), "invalid wav file");
    unsigned channels = 0;
    std::size_t at = 12;
    while (at < length)
    {
        const std::size_t size = le32_at(bytes, length, checked_add(at, 4));
        const std::size_t body = checked_add(at, 8);
        if (has_tag(bytes, length, at, "fmt "))
        {
            require(size <= length - body && size >= 16, "invalid wav file");
            const uint8_t* fmt = bytes + body;
            // PCM (format 1), 16 bits per sample.
            require(fmt[0] == 1 && fmt[1] == 0 && fmt[14] == 16 && fmt[15] == 0, "invalid wav file");
            channels = unsigned(fmt[2]) | (unsigned(fmt[3]) << 8);
            require(channels >= 1 && channels <= 8, "unsupported number of channels");
            require(le32_at(fmt, size, 4) == sample_rate, "the sample rate must be 44100 Hz");
        }
        else if (has_tag(bytes, length, at, "data"))
        {
            require(channels > 0, "invalid wav file");
            require(body <= length, "invalid wav file");
            return pcm16_input(bytes + body, length - body, channels, limits);
        }
        require(size <= length - std::min(body, length) && body <= length, "invalid wav file");
        at = checked_add(body, size);
    }
    throw Error("invalid wav file");
}

std::vector<uint8_t> pcm16_wave(const float* samples, std::size_t frames, unsigned channels, const Limits& limits)
{
    require(channels >= 1, "audio sample shape mismatch");
    const std::size_t count = checked_mul(frames, channels);
    require(count <= limits.tensor_elements, "audio sample shape mismatch");
    const std::size_t block = 2 * std::size_t(channels), rate = checked_mul(block, sample_rate);
    const std::size_t data = checked_mul(count, 2);
    require(data <= limits.pcm_bytes, "PCM exceeds the byte limit");
    require(block <= std::numeric_limits<uint16_t>::max() && rate <= std::numeric_limits<uint32_t>::max() &&
                data <= std::numeric_limits<uint32_t>::max() - 36,
            "audio exceeds the RIFF/WAVE dimensions");
    for (std::size_t i = 0; i < count; ++i)
    {
        require(std::isfinite(samples[i]), "nonfinite audio sample");
    }
    std::vector<uint8_t> out;
    out.reserve(data + 44);
    const auto put = [&](std::size_t value, int bytes)
    {
        for (int i = 0; i < bytes; ++i)
        {
            out.push_back(uint8_t(value >> (8 * i)));
        }
    };
    const auto tag = [&](const char* t) { out.insert(out.end(), t, t + 4); };
    tag("RIFF");
    put(data + 36, 4);
    tag("WAVE");
    tag("fmt ");
    put(16, 4);
    put(1, 2);
    put(channels, 2);
    put(sample_rate, 4);
    put(rate, 4);
    put(block, 2);
    put(16, 2);
    tag("data");
    put(data, 4);
    for (std::size_t i = 0; i < count; ++i)
    {
        // Clamped in double first (no overflow for any finite float), then to
        // the nearest integer with ties to even.
        const double scaled = std::min(std::max(double(samples[i]) * 32768.0, -32768.0), 32767.0);
        double whole = std::floor(scaled);
        const double fraction = scaled - whole;
        if (fraction > 0.5 || (fraction == 0.5 && std::fmod(whole, 2.0) != 0.0))
        {
            whole += 1.0;
        }
        put(uint16_t(int16_t(whole)), 2);
    }
    return out;
}

// ---------------------------------------------------------------- options

CliOptions parse_cli(const std::vector<std::string_view>& arguments)
{
    CliOptions o;
    std::vector<std::string_view> positional;
    for (std::size_t i = 0; i < arguments.size(); ++i)
    {
        const std::string_view arg = arguments[i];
        if (arg == "--")
        {
            positional.insert(positional.end(), arguments.begin() + std::ptrdiff_t(i + 1), arguments.end());
            break;
        }
        if (arg.size() <= 1 || arg[0] != '-')
        {
            positional.push_back(arg);
            continue;
        }
        const auto integer = [&](std::string_view name) -> int
        {
            require(++i < arguments.size(), ("option '" + std::string(name) + "' must have an argument").c_str());
            std::string_view text = arguments[i];
            if (text.starts_with('+'))
            {
                text.remove_prefix(1);
            }
            int value = 0;
            const auto parsed = std::from_chars(text.data(), text.data() + text.size(), value);
            if (text.empty() || parsed.ec != std::errc{} || parsed.ptr != text.data() + text.size())
            {
                const std::string_view shown = name == "-q" ? "--n_codebooks" : name == "-c" ? "--channels" : name;
                throw Error("option " + std::string(shown) + " expects an integer");
            }
            return value;
        };
        const auto option = [&](std::string_view name)
        {
            if (name == "-h" || name == "--help")
            {
                o.help = true;
            }
            else if (name == "-f" || name == "--fast")
            {
                o.fast = true;
            }
            else if (name == "-s" || name == "--separate_channels")
            {
                o.separate = true;
            }
            else if (name == "-v")
            {
                ++o.verbose;
            }
            else if (name == "-T")
            {
                o.threads = integer(name);
            }
            else if (name == "-q" || name == "--n_codebooks")
            {
                o.quality = integer(name);
            }
            else if (name == "-c" || name == "--channels")
            {
                o.channels = integer(name);
            }
            else if (name == "--batch_size")
            {
                o.batch = integer(name);
            }
            else if (name == "--metal")
            {
                o.metal = true;
            }
            else
            {
                throw Error("unknown option: '" + std::string(name) + "'");
            }
        };
        if (arg.starts_with("--"))
        {
            option(arg);
        }
        else
        {
            // A short group is checked whole before any of it takes a value:
            // "-q1" is the unknown option "-1", not "-q 1".
            for (const char c : arg.substr(1))
            {
                require(std::string_view("hfsvTqc").find(c) != std::string_view::npos,
                        ("unknown option: '-" + std::string(1, c) + "'").c_str());
            }
            for (const char c : arg.substr(1))
            {
                option(std::string("-") + c);
            }
        }
        if (o.help)
        {
            return o;
        }
    }
    if (positional.size() != 3)
    {
        o.help = true;
        return o;
    }
    require(positional[0] == "c" || positional[0] == "d" || positional[0] == "t",
            ("unknown command: " + std::string(positional[0])).c_str());
    o.command = positional[0][0];
    o.input = positional[1];
    o.output = positional[2];
    return o;
}

std::string_view cli_help()
{
    return R"(TSAC on AMD Instinct MI355X

Very low bitrate audio compression

usage: tsac-hip [options] c infile outfile     audio compression
                          d infile outfile     audio decompression
                          t infile outfile     audio compression then decompression to outfile
Uncompressed wave (.wav) and raw audio (.sw) are natively supported as input files.
FFmpeg is invoked to support other audio formats. Decompression outputs WAVE.
Weights load from the original model files (tsac_{mono,stereo}_q8.bin and
dac_{mono,stereo}_q8.bin) in $TSAC_HIP_MODELS, or beside the executable.

Available options:
-h --help               show the help
-T n                    number of host threads (accepted; the codec runs on the GPU)
-q --n_codebooks n      quality (1-12 for joint stereo, 1-9 otherwise; 0=max)
-s --separate_channels  encode stereo as separate channels
-c --channels n         force input channels through FFmpeg
-f --fast               disable the transformer model
--batch_size n          force the entropy batch size (default=auto)
-v                      display statistics
--metal                 accepted for compatibility (the GPU is always used)
)";
}
} // namespace tsac_hip
