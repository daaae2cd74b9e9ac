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

namespace
{
// One command-line option: its single-letter spelling (0 if none), its long
// spelling (empty if none), whether it consumes the next argument as an
// integer, and what it sets. The accepted spellings and their meanings are the
// reference command line's (src/cli.cpp:50-90).
struct OptionSpec
{
    char letter;
    std::string_view word;
    bool integer;
    void (*apply)(CliOptions&, int);
};

constexpr OptionSpec option_table[] = {
    {'h', "--help", false, [](CliOptions& o, int) { o.help = true; }},
    {'f', "--fast", false, [](CliOptions& o, int) { o.fast = true; }},
    {'s', "--separate_channels", false, [](CliOptions& o, int) { o.separate = true; }},
    {'v', "", false, [](CliOptions& o, int) { ++o.verbose; }},
    {'T', "", true, [](CliOptions& o, int v) { o.threads = v; }},
    {'q', "--n_codebooks", true, [](CliOptions& o, int v) { o.quality = v; }},
    {'c', "--channels", true, [](CliOptions& o, int v) { o.channels = v; }},
    {0, "--batch_size", true, [](CliOptions& o, int v) { o.batch = v; }},
    {0, "--metal", false, [](CliOptions& o, int) { o.metal = true; }},
};

std::string spelling(const OptionSpec& spec)
{
    return spec.word.empty() ? std::string{'-', spec.letter} : std::string(spec.word);
}

const OptionSpec& by_word(std::string_view word)
{
    for (const auto& spec : option_table)
        if (!spec.word.empty() && spec.word == word)
            return spec;
    throw Error("unrecognised option " + std::string(word));
}

const OptionSpec& by_letter(char letter)
{
    for (const auto& spec : option_table)
        if (spec.letter && spec.letter == letter)
            return spec;
    throw Error(std::string("unrecognised option -") + letter);
}

// A decimal int, optionally written with a leading '+', filling the whole argument.
int integer_value(const OptionSpec& spec, std::string_view text)
{
    const std::string_view digits = text.substr(text.starts_with('+') ? 1 : 0);
    int value = 0;
    const auto [end, status] = std::from_chars(digits.data(), digits.data() + digits.size(), value);
    if (digits.empty() || status != std::errc{} || end != digits.data() + digits.size())
        throw Error(spelling(spec) + " takes an integer; '" + std::string(text) + "' is not one");
    return value;
}
} // namespace

CliOptions parse_cli(const std::vector<std::string_view>& arguments)
{
    CliOptions o;
    std::vector<std::string_view> operands;
    std::size_t cursor = 0;
    while (cursor < arguments.size() && !o.help)
    {
        const std::string_view word = arguments[cursor++];
        if (word == "--")
        {
            operands.insert(operands.end(), arguments.begin() + std::ptrdiff_t(cursor), arguments.end());
            break;
        }
        if (word.size() < 2 || word.front() != '-')
        {
            operands.push_back(word);
            continue;
        }
        // Resolve every spelling in the word before acting on any: a bundle of
        // letters such as "-vq" is valid only if all its letters are options.
        std::vector<const OptionSpec*> selected;
        if (word[1] == '-')
            selected.push_back(&by_word(word));
        else
            for (const char letter : word.substr(1))
                selected.push_back(&by_letter(letter));
        // Options that take a value consume the following arguments in order.
        for (const OptionSpec* spec : selected)
        {
            int value = 0;
            if (spec->integer)
            {
                if (cursor == arguments.size())
                    throw Error(spelling(*spec) + " needs a value");
                value = integer_value(*spec, arguments[cursor++]);
            }
            spec->apply(o, value);
        }
    }
    if (o.help)
        return o;
    if (operands.size() != 3)
    {
        o.help = true; // not a complete command: show the usage
        return o;
    }
    const std::string_view command = operands[0];
    if (command != "c" && command != "d" && command != "t")
        throw Error("the command is c, d or t, not '" + std::string(command) + "'");
    o.command = command[0];
    o.input = operands[1];
    o.output = operands[2];
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
