// Audio files of the command-line codec (src/audio.cpp): raw 16-bit PCM and
// RIFF/WAVE input, WAVE output, all at 44100 Hz.
#pragma once

#include "format.hpp"

#include <string_view>

namespace tsac_hip
{
// Interleaved float PCM [frames][channels], frames padded with zeros to a
// multiple of 512.
struct Pcm
{
    unsigned channels = 0;
    std::size_t frames = 0;
    std::vector<float> samples;
};

// pcm16_input (src/audio.cpp:19-38): little-endian signed 16-bit samples
// scaled by 1/32768; an incomplete last interleaved frame is dropped.
Pcm pcm16_input(const uint8_t* bytes, std::size_t length, unsigned channels, const Limits& limits);
// wave_input (src/audio.cpp:40-72): chunks walked from offset 12; "fmt " must
// be PCM (1), 16-bit, 1..8 channels, 44100 Hz; the "data" samples are read to
// the end of the file whatever the chunk and RIFF sizes say.
Pcm wave_input(const uint8_t* bytes, std::size_t length, const Limits& limits);
// pcm16_wave (src/audio.cpp:176-246): a 44-byte canonical WAVE header, then
// every sample clamped to [-32768, 32767] after scaling by 32768 and rounded
// half to even.
std::vector<uint8_t> pcm16_wave(const float* samples, std::size_t frames, unsigned channels, const Limits& limits);

// parse_cli (src/cli.cpp:7-129) and cli_help (:131-155).
struct CliOptions
{
    char command = 0;
    std::string_view input, output; // views into the arguments
    int threads = 0, quality = 0, channels = 0, batch = 0;
    unsigned verbose = 0;
    bool fast = false, separate = false, help = false, metal = false;
};
CliOptions parse_cli(const std::vector<std::string_view>& arguments);
std::string_view cli_help();
} // namespace tsac_hip
