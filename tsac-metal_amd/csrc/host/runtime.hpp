// Device model, sessions and the encode/decode drivers of the probability model.
#pragma once

#include "../kernels/attention.hpp"
#include "../kernels/codec.hpp"
#include "../kernels/dac.hpp"
#include "../kernels/frame.hpp"
#include "../kernels/kernels.hpp"
#include "format.hpp"

#include <array>
#include <chrono>
#include <map>
#include <memory>
#include <string>
#include <vector>

namespace tsac_hip
{
class DacModel;
struct EncodeOptions;

// Monotonic wall clock, seconds.
inline double now()
{
    return std::chrono::duration<double>(std::chrono::steady_clock::now().time_since_epoch()).count();
}

struct Geometry
{
    uint32_t width = 512, heads = 4, head_width = 128, ffn = 2048;
    uint32_t temporal_layers = 12, codebook_layers = 3;
    uint32_t latent = 1024, alphabet = 1024, books = 12, channels = 2, context = 1024;
    float attention_scale = 0.0883883461356163f;

    std::size_t projections() const
    {
        return 4 * std::size_t(temporal_layers + codebook_layers) + 3;
    }
    std::size_t norms() const
    {
        return 2 * std::size_t(temporal_layers + codebook_layers) + 2;
    }
    // (K, N) of projection `index` (src/models/contract.cpp:88-110).
    std::pair<std::size_t, std::size_t> projection_shape(std::size_t index) const;
};

// Owning device allocation.
class DeviceBuffer
{
public:
    DeviceBuffer() = default;
    explicit DeviceBuffer(std::size_t bytes);
    ~DeviceBuffer();
    DeviceBuffer(DeviceBuffer&& other) noexcept;
    DeviceBuffer& operator=(DeviceBuffer&& other) noexcept;
    DeviceBuffer(const DeviceBuffer&) = delete;
    DeviceBuffer& operator=(const DeviceBuffer&) = delete;

    void* get() const
    {
        return data_;
    }
    template <class T> T* as() const
    {
        return static_cast<T*>(data_);
    }
    std::size_t bytes() const
    {
        return bytes_;
    }

private:
    void* data_ = nullptr;
    std::size_t bytes_ = 0;
};

// Page-locked host staging.
class PinnedBuffer
{
public:
    PinnedBuffer() = default;
    ~PinnedBuffer();
    void reserve(std::size_t bytes);
    template <class T> T* as() const
    {
        return static_cast<T*>(data_);
    }

private:
    void* data_ = nullptr;
    std::size_t bytes_ = 0;
};

// Named scratch that grows on demand and is released by clear().
class Arena
{
public:
    void* get(const std::string& name, std::size_t bytes);
    template <class T> T* get(const std::string& name, std::size_t count)
    {
        return static_cast<T*>(get(name, count * sizeof(T)));
    }
    void clear()
    {
        buffers_.clear();
    }

private:
    std::map<std::string, DeviceBuffer> buffers_;
};

struct LinearHost
{
    const int8_t* values;
    const float* scales;
    const float* bias;
};

class Model
{
public:
    Model(const Geometry& g, const LinearHost* projections, const uint16_t* const* gain,
          const uint16_t* const* bias, const uint16_t* positions, const uint16_t* rotations,
          const uint16_t* embeddings, const Limits& limits);

    const Geometry& geometry() const
    {
        return g_;
    }
    const Limits& limits() const
    {
        return limits_;
    }
    int device() const
    {
        return device_;
    }
    const DeviceLinear& projection(std::size_t index) const
    {
        return projections_.at(index);
    }
    // Stack projections: op 0 qkv, 1 attn_out, 2 mlp_in, 3 mlp_out.
    const DeviceLinear& layer(bool temporal, std::size_t layer, int op) const;
    const DeviceLinear& temporal_projection() const;
    const DeviceLinear& codebook_projection() const;
    const DeviceLinear& output_projection() const;
    const uint16_t* norm_gain(std::size_t index) const
    {
        return gain_.at(index);
    }
    const uint16_t* norm_bias(std::size_t index) const
    {
        return bias_.at(index);
    }
    std::size_t norm_index(bool temporal, std::size_t layer, bool mlp) const;
    std::size_t final_norm_index(bool temporal) const;
    const uint16_t* positions() const
    {
        return positions_;
    }
    const uint16_t* rotations() const
    {
        return rotations_;
    }
    const uint16_t* embeddings() const
    {
        return embeddings_;
    }
    // The model's projections and norms for the frame kernel's job table.
    const FrameModel& frame_tables() const
    {
        return frame_;
    }

private:
    Geometry g_;
    Limits limits_;
    int device_ = 0;
    DeviceBuffer values_, constants_;
    FrameModel frame_;
    std::vector<DeviceLinear> projections_;
    std::vector<const uint16_t*> gain_, bias_;
    const uint16_t *positions_ = nullptr, *rotations_ = nullptr, *embeddings_ = nullptr;
};

class Session
{
public:
    explicit Session(std::shared_ptr<const Model> model);
    ~Session();
    Session(const Session&) = delete;
    Session& operator=(const Session&) = delete;

    void clear();
    // pack_normal / unpack_normal on the GPU; an observer, when given, sees every
    // symbol in stream order once the GPU work is done (encode: with its bits).
    std::vector<uint8_t> encode(Header header, const uint16_t* tokens, std::size_t count,
                                const SymbolObserver* observer = nullptr);
    std::vector<uint16_t> decode(const uint8_t* stream, std::size_t length,
                                 const SymbolObserver* observer = nullptr);
    // The DAC side (audio.cpp). analyze: padded PCM interleaved
    // [frames*512][groups*channels] -> tokens [frame][group][book]
    // (analyze_audio, src/common/audio_pipeline.hpp:37-58); synthesize: the
    // inverse (synthesize_audio, :60-79), float PCM without rounding.
    void analyze(const DacModel& dac, const float* pcm, std::size_t frames, std::size_t groups, unsigned books,
                 uint16_t* tokens);
    void synthesize(const DacModel& dac, const uint16_t* tokens, std::size_t frames, std::size_t groups,
                    unsigned books, float* pcm);
    // DacAnalysis::apply / DacSynthesis::apply on one window, reference Signal
    // layout [frame][channel]: analysis PCM of `frames` samples (a multiple of
    // 512) -> latent [frames/512][1024]; synthesis latent [frames][1024] ->
    // [frames*512][channels].
    void dac_apply(const DacModel& dac, bool synthesis, const float* input, std::size_t frames, float* output);
    // AudioAnalyzer::encode / decode (include/tsac/audio_analyzer.hpp:31-36):
    // interleaved float PCM of `count` frames <-> an FBAZ stream, fast or normal
    // framing; decoded PCM keeps the padding to whole frames.
    std::vector<uint8_t> encode_audio(const DacModel& dac, const float* samples, std::size_t count,
                                      std::size_t channels, const EncodeOptions& options,
                                      const SymbolObserver* observer = nullptr);
    std::vector<float> decode_audio(const DacModel& dac, const uint8_t* stream, std::size_t length,
                                    const SymbolObserver* observer, std::size_t* channels);
    // Teacher-forced distributions [count][alphabet]; decode_pass selects the
    // stepwise (GEMV) driver instead of the batched (GEMM) one.
    void distributions(Header header, const uint16_t* tokens, std::size_t count, bool decode_pass,
                       uint16_t* out);
    // Seconds of the last call: GPU model work, host range coding, total, the
    // host-to-device copy of the call's input (tokens or payload), which the
    // first and third include, then (decode-side passes) the GPU time of the
    // frame-step loop between two events on the session stream, the number of
    // frame steps in it, and how its frame steps were launched (FrameLaunch:
    // 0 cooperative, 1 plain on request, 2 plain because another process held
    // the cooperative-launch resources; -1 when the call ran none), and 1 when
    // the call's model work ran step by step (decode; an encode whose batched
    // pass would not fit Limits::cache_bytes), else 0.
    std::array<double, 8> timing() const
    {
        return timing_;
    }

private:
    struct Stepwise;
    void check_errors();
    void check_dsp_errors();
    void analysis_graph(const DacModel& dac, Strided input, int samples, Strided output, float* const* slots);
    void synthesis_graph(const DacModel& dac, Strided input, int frames, Strided output, int first, int last,
                         float* const* slots);
    void reset_errors();
    // Copies the call's input to the device between two events; input_seconds()
    // (after the stream has drained) is that copy's duration.
    void upload_input(void* device, const void* host, std::size_t bytes);
    double input_seconds();
    // GPU seconds between the events around the last stepwise loop.
    double steps_seconds();
    void validate(const Header& h, const uint16_t* tokens, std::size_t count) const;
    // Bytes of the persistent key/value caches the header's lanes need
    // (src/common/cpu_transformer.tpp:285-305), which Limits::cache_bytes bounds.
    std::size_t persistent_cache_bytes(const Header& h) const;
    // How a known-token pass runs within Limits::cache_bytes: the batched pass
    // computes whole sequences and many frames of codebook rows ahead, and its
    // scratch (with the persistent caches) must fit the limit, as the lookahead
    // of the reference's Metal encoder must (src/metal/transformer/encoding.mm:139-150);
    // it shrinks its batches to fit, and where not even one sequence and one
    // step fit, the pass runs step by step on the frame-step path instead.
    struct KnownPlan
    {
        bool stepwise = false;
        std::size_t temporal_rows = 0; // rows per temporal batch (whole sequences)
        std::size_t codebook_steps = 0; // frame steps per codebook chunk
    };
    KnownPlan plan_known(const Header& h) const;
    // Batched known-token pass. Writes either the BF16 distributions of every
    // token (distributions != null) or its ten Q15 splits (splits != null).
    void batched(const Header& h, const uint16_t* tokens, uint16_t* distributions,
                 uint16_t* splits, const KnownPlan& plan);
    void temporal_rows(const Header& h, const uint16_t* tokens, uint16_t* conditioning, std::size_t batch_rows);
    void stack_rows(bool temporal, uint16_t* x, std::size_t rows, const int* starts,
                    const int* lengths, const int* replays, std::size_t sequences,
                    std::size_t max_length, const std::string& tag);
    // Stepwise pass, enqueued without host round trips. `known` tokens are
    // teacher-forced when non-null; otherwise symbols are range-decoded on the
    // GPU from `payload`. Writes tokens (and, if requested, the BF16
    // distributions, or with known tokens each token's ten Q15 splits,
    // [symbols][16]) in token order.
    void stepwise(const Header& h, const uint16_t* known, const uint8_t* payload,
                  std::size_t payload_bytes, uint16_t* tokens_out, uint16_t* distributions,
                  uint16_t* splits = nullptr);
    // position: host value, or read from device_position when that is non-null.
    void layer_step(bool temporal, std::size_t layer, uint16_t* x, std::size_t rows,
                    std::size_t first_lane, std::size_t position, const int* device_position,
                    bool replay, std::size_t extent);

    std::shared_ptr<const Model> model_;
    hipStream_t stream_ = nullptr;
    Arena arena_;
    DeviceBuffer errors_;
    PinnedBuffer pinned_errors_, staging_, staging_nodes_, staging_tokens_;
    std::array<double, 8> timing_{};
    // TSAC_HIP_FRAME_LAUNCH=plain in the environment when the session was
    // created: frame steps go out as plain launches (see FrameArgs::plain_launch).
    bool plain_frame_launch_ = false;
    int frame_launch_ = -1; // FrameLaunch of the last stepwise pass, -1 if none
    hipEvent_t upload_start_ = nullptr, upload_stop_ = nullptr;
    hipEvent_t steps_start_ = nullptr, steps_stop_ = nullptr;
    bool stepped_ = false;
    bool uploaded_ = false;
};
} // namespace tsac_hip
