// tsac-hip: the command-line codec (src/main.cpp, src/codec.cpp) on the
// MI355X, over the library's C ABI (include/tsac_hip.h).
//
//   tsac-hip [options] c infile outfile   compress
//   tsac-hip [options] d infile outfile   decompress to WAVE
//   tsac-hip [options] t infile outfile   compress, then decompress to WAVE
//
// The weights are the original model files of the stream's variant,
// tsac_{mono,stereo}_q8.bin and dac_{mono,stereo}_q8.bin, found in
// $TSAC_HIP_MODELS or beside the executable. The input is read before the
// weights are loaded, since the input's channels pick the variant.
#include "../../include/tsac_hip.h"

#include <cerrno>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <filesystem>
#include <fstream>
#include <iostream>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

#include <spawn.h>
#include <sys/resource.h>
#include <sys/wait.h>
#include <unistd.h>

extern char** environ;

namespace
{
namespace fs = std::filesystem;

struct Failure : std::runtime_error
{
    using std::runtime_error::runtime_error;
};

void check(int status)
{
    if (status != TSAC_HIP_OK)
    {
        throw Failure(tsac_hip_last_error());
    }
}

void require(bool condition, const std::string& message)
{
    if (!condition)
    {
        throw Failure(message);
    }
}

// Library-allocated buffers and handles, released on scope exit.
template <class T> struct Freed
{
    T* p = nullptr;
    ~Freed()
    {
        tsac_hip_free(p);
    }
};
template <class T, void (*Destroy)(T*)> struct Handle
{
    T* p = nullptr;
    Handle() = default;
    Handle(const Handle&) = delete;
    ~Handle()
    {
        if (p)
        {
            Destroy(p);
        }
    }
};
using Source = Handle<tsac_hip_source, tsac_hip_source_destroy>;
using Model = Handle<tsac_hip_model, tsac_hip_model_destroy>;
using Session = Handle<tsac_hip_session, tsac_hip_session_destroy>;
using Dac = Handle<tsac_hip_dac, tsac_hip_dac_destroy>;

const tsac_hip_limits limits{}; // the reference defaults

std::vector<uint8_t> read_file(const fs::path& path)
{
    std::ifstream in(path, std::ios::binary | std::ios::ate);
    require(bool(in), "cannot open input: " + path.string());
    const auto size = in.tellg();
    require(size >= 0 && uint64_t(size) <= (uint64_t{512} << 20), "input exceeds the file size limit");
    std::vector<uint8_t> bytes(static_cast<std::size_t>(size));
    in.seekg(0);
    require(bytes.empty() || bool(in.read(reinterpret_cast<char*>(bytes.data()), std::streamsize(bytes.size()))),
            "cannot read complete input: " + path.string());
    return bytes;
}

void write_file(const fs::path& path, const uint8_t* bytes, std::size_t length)
{
    std::ofstream out(path, std::ios::binary | std::ios::trunc);
    require(bool(out), "cannot create output: " + path.string());
    out.write(reinterpret_cast<const char*>(bytes), std::streamsize(length));
    out.flush();
    require(bool(out), "cannot write complete output: " + path.string());
}

struct Pcm
{
    std::vector<float> samples; // [frames][channels]
    std::size_t frames = 0;
    uint32_t channels = 0;
};

Pcm from_library(float* samples, std::size_t frames, uint32_t channels)
{
    Freed<float> owned{samples};
    return {std::vector<float>(samples, samples + frames * channels), frames, channels};
}

Pcm wave(const std::vector<uint8_t>& bytes)
{
    float* samples = nullptr;
    std::size_t frames = 0;
    uint32_t channels = 0;
    check(tsac_hip_wave_read(bytes.data(), bytes.size(), &limits, &samples, &frames, &channels));
    return from_library(samples, frames, channels);
}

// A temporary directory for FFmpeg's output, removed with its contents.
struct TemporaryDirectory
{
    fs::path path;
    TemporaryDirectory()
    {
        std::string pattern = (fs::temp_directory_path() / "tsac-hip-audio-XXXXXX").string();
        require(mkdtemp(pattern.data()) != nullptr, "cannot create the audio conversion directory");
        path = pattern;
    }
    ~TemporaryDirectory()
    {
        std::error_code ignored;
        fs::remove_all(path, ignored);
    }
};

// read_audio (src/audio.cpp:103-158): raw 16-bit PCM for .sw, the native
// reader for .wav, otherwise FFmpeg converting to 44100 Hz 16-bit WAVE
// (with -c, forced to that many channels).
Pcm read_audio(const fs::path& path, int requested_channels)
{
    require(requested_channels >= 0 && requested_channels <= 127, "unsupported number of channels");
    if (path.extension() == ".sw")
    {
        const auto bytes = read_file(path);
        float* samples = nullptr;
        std::size_t frames = 0;
        const uint32_t channels = requested_channels ? uint32_t(requested_channels) : 1u;
        check(tsac_hip_pcm16_read(bytes.data(), bytes.size(), channels, &limits, &samples, &frames));
        return from_library(samples, frames, channels);
    }
    if (path.extension() == ".wav" && requested_channels == 0)
    {
        try
        {
            return wave(read_file(path));
        }
        catch (const Failure& e)
        {
            throw Failure(path.string() + ": " + e.what());
        }
    }
    TemporaryDirectory directory;
    const fs::path converted = directory.path / "converted.wav";
    // An absolute input path cannot be taken for an FFmpeg option.
    std::vector<std::string> arguments{"ffmpeg", "-i", fs::absolute(path).string(), "-y", "-loglevel", "error",
                                       "-ar", "44100", "-acodec", "pcm_s16le"};
    if (requested_channels)
    {
        arguments.insert(arguments.end(), {"-ac", std::to_string(requested_channels)});
    }
    arguments.push_back(converted.string());
    std::vector<char*> argv;
    for (auto& a : arguments)
    {
        argv.push_back(a.data());
    }
    argv.push_back(nullptr);
    pid_t child = 0;
    const int error = posix_spawnp(&child, "ffmpeg", nullptr, nullptr, argv.data(), environ);
    require(error == 0, std::string("cannot run FFmpeg: ") + std::strerror(error));
    int status = 0;
    pid_t waited = 0;
    do
    {
        waited = waitpid(child, &status, 0);
    } while (waited == -1 && errno == EINTR);
    require(waited == child && WIFEXITED(status) && WEXITSTATUS(status) == 0, "FFmpeg failed to convert the input");
    return wave(read_file(converted));
}

fs::path models_directory()
{
    if (const char* dir = std::getenv("TSAC_HIP_MODELS"); dir && *dir)
    {
        return dir;
    }
    std::error_code e;
    const fs::path exe = fs::read_symlink("/proc/self/exe", e);
    require(!e, "cannot locate the executable's directory");
    return exe.parent_path();
}

// The device models of one variant (stereo or mono), from the original files.
struct Codec
{
    Model model;
    Dac dac;
    Session session;

    explicit Codec(unsigned model_channels)
    {
        require(model_channels == 1 || model_channels == 2, "unsupported model channel count");
        const std::string variant = model_channels == 1 ? "mono" : "stereo";
        const fs::path dir = models_directory();
        Source transformer, codec;
        check(tsac_hip_source_load((dir / ("tsac_" + variant + "_q8.bin")).c_str(), nullptr, &transformer.p));
        check(tsac_hip_source_load((dir / ("dac_" + variant + "_q8.bin")).c_str(), nullptr, &codec.p));
        check(tsac_hip_model_create_from_source(transformer.p, codec.p, &limits, &model.p));
        check(tsac_hip_dac_create_from_source(codec.p, &limits, &dac.p));
        check(tsac_hip_session_create(model.p, &session.p));
    }
};

// EntropyProgress (src/codec.cpp:39-106): with -v the header line and a
// percentage per entropy step; with -vv the average bits of every codebook.
struct Progress
{
    tsac_hip_header header{};
    unsigned verbosity = 0;
    std::vector<std::size_t> bits;
    std::size_t committed = 0, symbols = 0;
    int percent = -1;

    Progress(const tsac_hip_header& h, unsigned v) : header(h), verbosity(v), bits(h.codebooks, 0)
    {
        symbols = std::size_t(h.frames) * h.groups * h.codebooks;
        if (verbosity)
        {
            std::printf("batch_size=%u bs=%u n_cb=%u block_len=%llu\n", unsigned(h.batch), unsigned(h.groups),
                        unsigned(h.codebooks), static_cast<unsigned long long>(steps()));
            if (symbols == 0)
            {
                std::printf("\n");
            }
        }
    }
    uint64_t steps() const
    {
        return header.batch ? header.frames / header.batch + (header.frames % header.batch != 0) : 0;
    }
    static int before(void* context, const tsac_hip_position* p)
    {
        auto* self = static_cast<Progress*>(context);
        const int now = static_cast<int>((p->step + 1) * 100 / self->steps());
        if (now != self->percent)
        {
            std::printf("%3d%%\r", now);
            std::fflush(stdout);
            self->percent = now;
        }
        return 0;
    }
    static int after(void* context, const tsac_hip_position* p, uint64_t bits)
    {
        auto* self = static_cast<Progress*>(context);
        self->bits[p->codebook] += bits;
        if (++self->committed == self->symbols)
        {
            std::printf("\n");
        }
        return 0;
    }
    tsac_hip_observer observer()
    {
        return tsac_hip_observer{this, verbosity ? before : nullptr, verbosity ? after : nullptr};
    }
    void averages() const
    {
        if (verbosity < 2)
        {
            return;
        }
        std::printf("CB AVG_BITS\n");
        const double count = double(header.frames) * header.groups;
        for (std::size_t book = 0; book < bits.size(); ++book)
        {
            std::printf("%2zu %7.3f\n", book, count ? double(bits[book]) / count : 0.0);
        }
    }
};

struct Statistics
{
    uint64_t frames = 0;
    std::size_t stream_bytes = 0;
    double bitrate_kbps() const
    {
        return frames ? double(stream_bytes) * 8.0 * 44100.0 / (double(frames) * 512.0 * 1000.0) : 0.0;
    }
};

double peak_memory_gb()
{
    rusage usage{};
    return getrusage(RUSAGE_SELF, &usage) == 0 ? double(usage.ru_maxrss) * 1024.0 / 1e9 : 0.0;
}

tsac_hip_encode_options encode_options(const tsac_hip_cli_options& o)
{
    require(o.quality >= 0 && o.quality <= 255, "invalid number of codebooks");
    tsac_hip_encode_options e{};
    e.method = o.fast ? 0 : 1;
    e.codebooks = uint8_t(o.quality);
    e.separate_channels = o.separate;
    if (!o.fast && o.batch)
    {
        require(o.batch > 0 && o.batch <= 65535, "invalid entropy batch size");
        e.entropy_batch = uint16_t(o.batch);
    }
    return e;
}

std::vector<uint8_t> compress(const tsac_hip_cli_options& o, std::unique_ptr<Codec>& codec, Statistics& stats)
{
    const Pcm pcm = read_audio(o.input, o.channels);
    const tsac_hip_encode_options options = encode_options(o);
    tsac_hip_header header{};
    check(tsac_hip_audio_header(pcm.frames, pcm.channels, &options, &limits, &header));
    if (!codec)
    {
        codec = std::make_unique<Codec>(header.model_channels);
    }
    Progress progress(header, o.fast ? 0 : o.verbose);
    const tsac_hip_observer observer = progress.observer();
    Freed<uint8_t> stream;
    std::size_t length = 0;
    check(tsac_hip_audio_encode(codec->session.p, codec->dac.p, pcm.samples.data(), pcm.frames, pcm.channels,
                                &options, &observer, &stream.p, &length));
    progress.averages();
    stats.frames = header.frames;
    stats.stream_bytes = length;
    return std::vector<uint8_t>(stream.p, stream.p + length);
}

std::vector<uint8_t> decompress(const std::vector<uint8_t>& stream, const tsac_hip_cli_options& o,
                                std::unique_ptr<Codec>& codec, Statistics& stats)
{
    tsac_hip_header header{};
    check(tsac_hip_parse_header(stream.data(), stream.size(), &limits, &header));
    if (!codec)
    {
        codec = std::make_unique<Codec>(header.model_channels);
    }
    Progress progress(header, header.method == 1 ? o.verbose : 0);
    const tsac_hip_observer observer = progress.observer();
    Freed<float> samples;
    std::size_t frames = 0;
    uint32_t channels = 0;
    check(tsac_hip_audio_decode(codec->session.p, codec->dac.p, stream.data(), stream.size(), &observer, &samples.p,
                                &frames, &channels));
    stats.frames = header.frames;
    stats.stream_bytes = stream.size();
    Freed<uint8_t> wave;
    std::size_t length = 0;
    check(tsac_hip_wave_write(samples.p, frames, channels, &limits, &wave.p, &length));
    return std::vector<uint8_t>(wave.p, wave.p + length);
}

// run_codec (src/codec.cpp:211-245).
void run(const tsac_hip_cli_options& o)
{
    std::unique_ptr<Codec> codec;
    Statistics stats;
    std::vector<uint8_t> output;
    if (o.command == 'c' || o.command == 't')
    {
        output = compress(o, codec, stats);
        if (o.verbose)
        {
            std::printf("bitrate=%.2f kb/s, max_memory=%.2f GB\n", stats.bitrate_kbps(), peak_memory_gb());
        }
        if (o.command == 't')
        {
            output = decompress(output, o, codec, stats);
        }
    }
    else if (o.command == 'd')
    {
        output = decompress(read_file(o.input), o, codec, stats);
    }
    else
    {
        throw Failure("invalid codec command");
    }
    write_file(o.output, output.data(), output.size());
}
} // namespace

int main(int argc, char** argv)
{
    try
    {
        tsac_hip_cli_options options{};
        check(tsac_hip_cli_parse(std::size_t(argc > 0 ? argc - 1 : 0), argv + 1, &options));
        if (options.help)
        {
            std::fputs(tsac_hip_cli_help(), stdout);
            return 1;
        }
        run(options);
        return 0;
    }
    catch (const std::exception& e)
    {
        std::fflush(stdout);
        std::fprintf(stderr, "tsac-hip: %s\n", e.what());
        return 1;
    }
}
