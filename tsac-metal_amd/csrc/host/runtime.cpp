#include "runtime.hpp"

#include <cstdlib>
#include <string_view>

#include <algorithm>
#include <chrono>
#include <cstring>

namespace tsac_hip
{
namespace
{
constexpr std::size_t replay_frames = 256;
// Rows processed per batched launch sequence; bounds scratch at roughly
// rows * (3*width + ffn) * 2 bytes.
constexpr std::size_t batch_rows = 65536;

std::size_t align_up(std::size_t n, std::size_t a)
{
    return (n + a - 1) / a * a;
}

bool supported_width(std::size_t k)
{
    return k == 256 || k == 512 || k == 1024 || k == 2048 || k == 4096;
}

// Quantised activations feed the MFMA GEMM in operand tiles; a handful of
// rows stays row-major for the GEMV.
Layout activation_layout(std::size_t rows)
{
    return rows > small_gemm_max_rows() ? Layout::tiles : Layout::rows;
}
} // namespace

// ---------------------------------------------------------------- geometry

std::pair<std::size_t, std::size_t> Geometry::projection_shape(std::size_t index) const
{
    const std::size_t stacked = 4 * std::size_t(temporal_layers + codebook_layers);
    if (index == stacked || index == stacked + 1)
    {
        return {latent, width};
    }
    if (index == stacked + 2)
    {
        return {width, alphabet};
    }
    switch (index % 4)
    {
    case 0:
        return {width, 3 * std::size_t(width)};
    case 1:
        return {width, width};
    case 2:
        return {width, ffn};
    default:
        return {ffn, width};
    }
}

// ---------------------------------------------------------------- memory

DeviceBuffer::DeviceBuffer(std::size_t bytes) : bytes_(bytes)
{
    if (bytes)
    {
        check_hip(hipMalloc(&data_, bytes), "hipMalloc");
    }
}

DeviceBuffer::~DeviceBuffer()
{
    if (data_)
    {
        (void)hipFree(data_);
    }
}

DeviceBuffer::DeviceBuffer(DeviceBuffer&& other) noexcept : data_(other.data_), bytes_(other.bytes_)
{
    other.data_ = nullptr;
    other.bytes_ = 0;
}

DeviceBuffer& DeviceBuffer::operator=(DeviceBuffer&& other) noexcept
{
    if (this != &other)
    {
        if (data_)
        {
            (void)hipFree(data_);
        }
        data_ = other.data_;
        bytes_ = other.bytes_;
        other.data_ = nullptr;
        other.bytes_ = 0;
    }
    return *this;
}

PinnedBuffer::~PinnedBuffer()
{
    if (data_)
    {
        (void)hipHostFree(data_);
    }
}

void PinnedBuffer::reserve(std::size_t bytes)
{
    if (bytes <= bytes_)
    {
        return;
    }
    if (data_)
    {
        (void)hipHostFree(data_);
        data_ = nullptr;
    }
    check_hip(hipHostMalloc(&data_, bytes, hipHostMallocDefault), "hipHostMalloc");
    bytes_ = bytes;
}

void* Arena::get(const std::string& name, std::size_t bytes)
{
    auto& buffer = buffers_[name];
    if (buffer.bytes() < bytes)
    {
        buffer = DeviceBuffer();
        buffer = DeviceBuffer(align_up(std::max<std::size_t>(bytes, 256), 256));
    }
    return buffer.get();
}

// ---------------------------------------------------------------- model

Model::Model(const Geometry& g, const LinearHost* projections, const uint16_t* const* gain,
             const uint16_t* const* bias, const uint16_t* positions, const uint16_t* rotations,
             const uint16_t* embeddings, const Limits& limits)
    : g_(g), limits_(limits)
{
    require(g.width >= 256 && g.width <= 2048 && supported_width(g.width), "model width must be 256..2048, a power of two");
    require(g.heads * g.head_width == g.width && (g.head_width == 64 || g.head_width == 128),
            "heads x head width must equal width with 64- or 128-wide heads");
    require(supported_width(g.ffn) && supported_width(g.latent), "ffn and latent widths must be 256..4096, powers of two");
    require(g.alphabet == 1024, "the alphabet must hold 1024 symbols");
    require(g.books >= 1 && g.books <= 12, "model codebooks must be 1..12");
    require(g.channels == 1 || g.channels == 2, "model channels must be 1 or 2");
    require(g.context >= replay_frames, "context must hold the 256-frame replay");
    require(g.temporal_layers >= 1 && g.codebook_layers >= 1, "empty transformer stack");
    require(projections && gain && bias && positions && rotations && embeddings, "missing model tensor");
    check_hip(hipGetDevice(&device_), "hipGetDevice");

    const std::size_t count = g.projections();
    std::vector<std::size_t> value_offset(count), scale_offset(count), bias_offset(count);
    std::size_t values_bytes = 0, constants_bytes = 0;
    for (std::size_t i = 0; i < count; ++i)
    {
        const auto [k, n] = g.projection_shape(i);
        require(projections[i].values && projections[i].scales && projections[i].bias,
                "missing projection tensor");
        value_offset[i] = values_bytes;
        values_bytes += align_up(k * n, 256);
        scale_offset[i] = constants_bytes;
        constants_bytes += align_up(k / 256 * n * 4, 256);
        bias_offset[i] = constants_bytes;
        constants_bytes += align_up(n * 4, 256);
    }
    const std::size_t norm_bytes = align_up(std::size_t(g.width) * 2, 256);
    const std::size_t norms_offset = constants_bytes;
    constants_bytes += 2 * g.norms() * norm_bytes;
    const std::size_t positions_offset = constants_bytes;
    constants_bytes += align_up(std::size_t(g.books) * g.width * 2, 256);
    const std::size_t rotations_offset = constants_bytes;
    constants_bytes += align_up(std::size_t(g.context) * g.head_width * 2, 256);
    const std::size_t embeddings_offset = constants_bytes;
    constants_bytes += align_up(std::size_t(g.books) * g.alphabet * g.latent * 2, 256);

    values_ = DeviceBuffer(values_bytes);
    constants_ = DeviceBuffer(constants_bytes);
    auto* values = values_.as<uint8_t>();
    auto* constants = constants_.as<uint8_t>();
    for (std::size_t i = 0; i < count; ++i)
    {
        const auto [k, n] = g.projection_shape(i);
        std::vector<int8_t> tiled(k * n);
        tile_weights(projections[i].values, k, n, tiled.data());
        check_hip(hipMemcpy(values + value_offset[i], tiled.data(), k * n, hipMemcpyHostToDevice),
                  "upload weights");
        check_hip(hipMemcpy(constants + scale_offset[i], projections[i].scales, k / 256 * n * 4,
                            hipMemcpyHostToDevice),
                  "upload scales");
        check_hip(hipMemcpy(constants + bias_offset[i], projections[i].bias, n * 4, hipMemcpyHostToDevice),
                  "upload bias");
        projections_.push_back({reinterpret_cast<const int8_t*>(values + value_offset[i]),
                                reinterpret_cast<const float*>(constants + scale_offset[i]),
                                reinterpret_cast<const float*>(constants + bias_offset[i]), k, n});
    }
    for (std::size_t i = 0; i < g.norms(); ++i)
    {
        require(gain[i] && bias[i], "missing norm tensor");
        uint8_t* gp = constants + norms_offset + 2 * i * norm_bytes;
        uint8_t* bp = gp + norm_bytes;
        check_hip(hipMemcpy(gp, gain[i], g.width * 2, hipMemcpyHostToDevice), "upload norm");
        check_hip(hipMemcpy(bp, bias[i], g.width * 2, hipMemcpyHostToDevice), "upload norm");
        gain_.push_back(reinterpret_cast<const uint16_t*>(gp));
        bias_.push_back(reinterpret_cast<const uint16_t*>(bp));
    }
    check_hip(hipMemcpy(constants + positions_offset, positions, std::size_t(g.books) * g.width * 2,
                        hipMemcpyHostToDevice),
              "upload positions");
    check_hip(hipMemcpy(constants + rotations_offset, rotations,
                        std::size_t(g.context) * g.head_width * 2, hipMemcpyHostToDevice),
              "upload rotations");
    check_hip(hipMemcpy(constants + embeddings_offset, embeddings,
                        std::size_t(g.books) * g.alphabet * g.latent * 2, hipMemcpyHostToDevice),
              "upload embeddings");
    positions_ = reinterpret_cast<const uint16_t*>(constants + positions_offset);
    rotations_ = reinterpret_cast<const uint16_t*>(constants + rotations_offset);
    embeddings_ = reinterpret_cast<const uint16_t*>(constants + embeddings_offset);

    // The frame kernel's job descriptors are built per pass from these host
    // arrays of device pointers (frame_job_table).
    frame_.linears = projections_.data();
    frame_.gain = gain_.data();
    frame_.bias = bias_.data();
    frame_.positions = positions_;
    frame_.rotations = rotations_;
    frame_.embeddings = embeddings_;
}

const DeviceLinear& Model::layer(bool temporal, std::size_t layer, int op) const
{
    return projections_.at((temporal ? 0 : 4 * std::size_t(g_.temporal_layers)) + 4 * layer + op);
}

const DeviceLinear& Model::temporal_projection() const
{
    return projections_.at(4 * std::size_t(g_.temporal_layers + g_.codebook_layers));
}

const DeviceLinear& Model::codebook_projection() const
{
    return projections_.at(4 * std::size_t(g_.temporal_layers + g_.codebook_layers) + 1);
}

const DeviceLinear& Model::output_projection() const
{
    return projections_.at(4 * std::size_t(g_.temporal_layers + g_.codebook_layers) + 2);
}

std::size_t Model::norm_index(bool temporal, std::size_t layer, bool mlp) const
{
    return (temporal ? 0 : 2 * std::size_t(g_.temporal_layers) + 1) + 2 * layer + (mlp ? 1 : 0);
}

std::size_t Model::final_norm_index(bool temporal) const
{
    return temporal ? 2 * std::size_t(g_.temporal_layers)
                    : 2 * std::size_t(g_.temporal_layers) + 1 + 2 * std::size_t(g_.codebook_layers);
}

// ---------------------------------------------------------------- session

Session::Session(std::shared_ptr<const Model> model) : model_(std::move(model))
{
    check_hip(hipSetDevice(model_->device()), "hipSetDevice");
    check_hip(hipStreamCreateWithFlags(&stream_, hipStreamNonBlocking), "hipStreamCreate");
    check_hip(hipEventCreate(&upload_start_), "hipEventCreate");
    check_hip(hipEventCreate(&upload_stop_), "hipEventCreate");
    check_hip(hipEventCreate(&steps_start_), "hipEventCreate");
    check_hip(hipEventCreate(&steps_stop_), "hipEventCreate");
    errors_ = DeviceBuffer(256);
    pinned_errors_.reserve(256);
    const char* launch = std::getenv("TSAC_HIP_FRAME_LAUNCH");
    plain_frame_launch_ = launch && std::string_view(launch) == "plain";
}

Session::~Session()
{
    if (stream_)
    {
        (void)hipStreamSynchronize(stream_);
        (void)hipStreamDestroy(stream_);
    }
    if (upload_start_)
    {
        (void)hipEventDestroy(upload_start_);
    }
    for (hipEvent_t e : {upload_stop_, steps_start_, steps_stop_})
    {
        if (e)
        {
            (void)hipEventDestroy(e);
        }
    }
}

double Session::steps_seconds()
{
    if (!stepped_)
    {
        return 0.0;
    }
    stepped_ = false;
    float ms = 0.0f;
    check_hip(hipEventSynchronize(steps_stop_), "hipEventSynchronize");
    check_hip(hipEventElapsedTime(&ms, steps_start_, steps_stop_), "hipEventElapsedTime");
    return ms / 1000.0;
}

void Session::upload_input(void* device, const void* host, std::size_t bytes)
{
    check_hip(hipEventRecord(upload_start_, stream_), "hipEventRecord");
    check_hip(hipMemcpyAsync(device, host, bytes, hipMemcpyHostToDevice, stream_), "upload input");
    check_hip(hipEventRecord(upload_stop_, stream_), "hipEventRecord");
    uploaded_ = true;
}

double Session::input_seconds()
{
    if (!uploaded_)
    {
        return 0.0;
    }
    uploaded_ = false;
    float ms = 0.0f;
    check_hip(hipEventSynchronize(upload_stop_), "hipEventSynchronize");
    check_hip(hipEventElapsedTime(&ms, upload_start_, upload_stop_), "hipEventElapsedTime");
    return ms / 1000.0;
}

void Session::clear()
{
    check_hip(hipStreamSynchronize(stream_), "hipStreamSynchronize");
    arena_.clear();
}

void Session::reset_errors()
{
    check_hip(hipMemsetAsync(errors_.get(), 0, 12, stream_), "hipMemsetAsync");
}

void Session::check_errors()
{
    check_hip(hipMemcpyAsync(pinned_errors_.as<uint32_t>(), errors_.get(), 12, hipMemcpyDeviceToHost, stream_),
              "read error words");
    check_hip(hipStreamSynchronize(stream_), "hipStreamSynchronize");
    const uint32_t* e = pinned_errors_.as<uint32_t>();
    require(!e[2], "decode frame step stalled");
    require(!(e[0] & error_nonfinite), "probability model activation is not finite");
    require(!e[1], "invalid range decoder state");
}

// src/format/entropy.cpp:60-66, src/common/transformer.cpp:104-118 and
// src/common/cpu_transformer.tpp:285-305.
void Session::validate(const Header& h, const uint16_t* tokens, std::size_t count) const
{
    const Geometry& g = model_->geometry();
    const Limits& limits = model_->limits();
    validate_header(h, limits);
    require(h.method == 1, "the probability model codes normal (method 1) streams only");
    require(h.frames <= 0xffffffffu, "normal stream frame count does not fit 32 bits");
    require(count == h.symbols(), "token count differs from frames x groups x codebooks of the header");
    require(h.model_channels == g.channels && h.codebooks <= g.books,
            "header channels or codebooks do not match the model");
    if (tokens)
    {
        for (std::size_t i = 0; i < count; ++i)
        {
            require(tokens[i] < 1024, "token above 1023: outside the 1024-symbol alphabet");
        }
    }
    const std::size_t independent = checked_mul(std::min<std::size_t>(h.batch, h.frames), h.groups);
    require(independent <= limits.tensor_elements, "independent lane count is above Limits::tensor_elements");
    require(persistent_cache_bytes(h) <= limits.cache_bytes,
            "key/value caches would exceed Limits::cache_bytes: lower the entropy batch or the channel count");
}

std::size_t Session::persistent_cache_bytes(const Header& h) const
{
    const Geometry& g = model_->geometry();
    const std::size_t independent = checked_mul(std::min<std::size_t>(h.batch, h.frames), h.groups);
    const std::size_t base = h.frames / h.batch, extra = h.frames % h.batch;
    const std::size_t contexts = checked_mul(
        h.groups, checked_add(checked_mul(h.batch - extra, std::min<std::size_t>(base, g.context)),
                              checked_mul(extra, std::min<std::size_t>(base + 1, g.context))));
    const std::size_t temporal_bytes =
        checked_mul(contexts, std::size_t(g.temporal_layers) * g.width * 2 * sizeof(uint16_t));
    const std::size_t codebook_bytes = checked_mul(
        checked_mul(independent, h.codebooks), std::size_t(g.codebook_layers) * g.width * 2 * sizeof(uint16_t));
    return checked_add(temporal_bytes, codebook_bytes);
}

Session::KnownPlan Session::plan_known(const Header& h) const
{
    const Geometry& g = model_->geometry();
    const std::size_t C = h.codebooks, w = g.width, steps = h.frames * h.groups;
    const std::size_t widest = std::max<std::size_t>({w, g.ffn, g.latent});
    // Device scratch of the batched pass (the arena entries of temporal_rows,
    // batched and stack_rows), per batch of `rows` rows.
    const auto quantised = [&](std::size_t rows) { return tile_padded_rows(rows) * (widest + widest / 64); };
    const auto temporal = [&](std::size_t rows)
    { return rows * (2 * C + 2 * g.latent + 10 * w + 2 * g.ffn + 8) + quantised(rows); };
    const auto codebook = [&](std::size_t rows)
    { return rows * (2 * g.latent + 10 * w + 4 * g.alphabet + 2 * g.ffn + 32) + quantised(rows); };
    const std::size_t limit = model_->limits().cache_bytes;
    const std::size_t used = checked_add(persistent_cache_bytes(h), steps * (2 * w + 2 * C)); // + conditioning, tokens
    const Lanes lanes(h);
    const std::size_t longest = std::min<std::size_t>(lanes.length(0), g.context); // longest sequence
    // Temporal rows of the whole pass: every (frame, group), plus 256 replayed
    // frames per rollover.
    std::size_t all_rows = 0;
    for (std::size_t lane = 0; lane < lanes.count; ++lane)
    {
        const std::size_t length = lanes.length(lane);
        const std::size_t rollovers = length > g.context ? (length - g.context - 1) / (g.context - replay_frames) + 1 : 0;
        all_rows += h.groups * (length + rollovers * replay_frames);
    }
    KnownPlan plan;
    for (const std::size_t t : {std::min(all_rows, std::max(batch_rows, longest)), longest})
    {
        std::size_t n = std::min(steps, std::max<std::size_t>(1, batch_rows / C));
        const auto fits = [&](std::size_t chunk) { return used + temporal(t) + codebook(chunk * C) <= limit; };
        if (!fits(1))
        {
            continue;
        }
        std::size_t lo = 1, hi = n; // the largest chunk that fits
        while (lo < hi)
        {
            const std::size_t mid = (lo + hi + 1) / 2;
            if (fits(mid))
            {
                lo = mid;
            }
            else
            {
                hi = mid - 1;
            }
        }
        plan.temporal_rows = t;
        plan.codebook_steps = lo;
        return plan;
    }
    plan.stepwise = true;
    return plan;
}

// One transformer stack over rows with causal prefill attention
// (src/common/cpu_transformer.tpp:133-175, final norm left to the caller).
void Session::stack_rows(bool temporal, uint16_t* x, std::size_t rows, const int* starts,
                         const int* lengths, const int* replays, std::size_t sequences,
                         std::size_t max_length, const std::string& tag)
{
    const Geometry& g = model_->geometry();
    const Model& m = *model_;
    const std::size_t w = g.width;
    const std::size_t widest = std::max<std::size_t>({w, g.ffn, g.latent});
    const Layout layout = activation_layout(rows);
    auto* q8 = arena_.get<int8_t>(tag + ".q8", tile_padded_rows(rows) * widest);
    auto* s8 = arena_.get<float>(tag + ".s8", tile_padded_rows(rows) * widest / 256);
    auto* qkv = arena_.get<uint16_t>(tag + ".qkv", rows * 3 * w);
    auto* att = arena_.get<uint16_t>(tag + ".att", rows * w);
    auto* hidden = arena_.get<uint16_t>(tag + ".hidden", rows * g.ffn);
    auto* err = errors_.as<uint32_t>();
    const std::size_t layers = temporal ? g.temporal_layers : g.codebook_layers;
    for (std::size_t l = 0; l < layers; ++l)
    {
        const std::size_t n1 = m.norm_index(temporal, l, false), n2 = m.norm_index(temporal, l, true);
        quantize_rows(x, rows, w, Prologue::layer_norm, m.norm_gain(n1), m.norm_bias(n1), q8, s8,
                      nullptr, err, stream_, layout);
        linear(m.layer(temporal, l, 0), q8, s8, rows, qkv, nullptr, LinearPath::automatic, stream_, layout);
        attention_prefill(qkv, w, g.heads, g.head_width, starts, lengths, replays, sequences,
                          max_length, temporal ? m.rotations() : nullptr, g.attention_scale, att,
                          stream_);
        quantize_rows(att, rows, w, Prologue::none, nullptr, nullptr, q8, s8, nullptr, err, stream_, layout);
        linear(m.layer(temporal, l, 1), q8, s8, rows, x, x, LinearPath::automatic, stream_, layout);
        quantize_rows(x, rows, w, Prologue::layer_norm, m.norm_gain(n2), m.norm_bias(n2), q8, s8,
                      nullptr, err, stream_, layout);
        linear(m.layer(temporal, l, 2), q8, s8, rows, hidden, nullptr, LinearPath::automatic, stream_, layout);
        quantize_rows(hidden, rows, g.ffn, Prologue::gelu, nullptr, nullptr, q8, s8, nullptr, err, stream_, layout);
        linear(m.layer(temporal, l, 3), q8, s8, rows, x, x, LinearPath::automatic, stream_, layout);
    }
}

// Temporal conditioning of every (frame, group) for known tokens: each lane's
// context positions form causal sequences; a rollover starts a new sequence
// with the last 256 complete frames replayed (src/common/transformer.cpp:184-211).
void Session::temporal_rows(const Header& h, const uint16_t* tokens, uint16_t* conditioning,
                            std::size_t batch_rows)
{
    const Geometry& g = model_->geometry();
    const Model& m = *model_;
    const std::size_t C = h.codebooks, G = h.groups, w = g.width;
    const Lanes lanes(h);
    struct Sequence
    {
        std::size_t row, length, replay;
    };
    std::vector<uint16_t> feedback;
    std::vector<Sequence> sequences;
    std::vector<std::size_t> source_row(h.frames * G);
    std::size_t rows = 0;
    const auto add_row = [&](std::size_t frame_plus_one, std::size_t group)
    {
        // frame_plus_one == 0 feeds the all-zero indices of the first frame.
        for (std::size_t b = 0; b < C; ++b)
        {
            feedback.push_back(frame_plus_one ? tokens[((frame_plus_one - 1) * G + group) * C + b] : 0);
        }
        return rows++;
    };
    for (std::size_t lane = 0; lane < lanes.count; ++lane)
    {
        for (std::size_t group = 0; group < G; ++group)
        {
            const std::size_t start = lanes.start(lane), length = lanes.length(lane);
            Sequence current{rows, 0, 0};
            std::size_t context_used = 0;
            for (std::size_t s = 0; s < length; ++s)
            {
                if (context_used == g.context)
                {
                    sequences.push_back(current);
                    current = {rows, 0, replay_frames};
                    for (std::size_t k = 0; k < replay_frames; ++k)
                    {
                        add_row(start + s - replay_frames + k + 1, group);
                    }
                    current.length = replay_frames;
                    context_used = replay_frames;
                    source_row[(start + s) * G + group] = rows - 1;
                }
                else
                {
                    const std::size_t r = add_row(s == 0 ? 0 : start + s, group);
                    ++current.length;
                    ++context_used;
                    source_row[(start + s) * G + group] = r;
                }
            }
            sequences.push_back(current);
        }
    }
    // Process whole sequences in batches of at most batch_rows rows.
    auto* err = errors_.as<uint32_t>();
    std::size_t first = 0;
    while (first < sequences.size())
    {
        std::size_t last = first, batch = 0;
        while (last < sequences.size() && (last == first || batch + sequences[last].length <= batch_rows))
        {
            batch += sequences[last].length;
            ++last;
        }
        const std::size_t row0 = sequences[first].row;
        const std::size_t count = last - first;
        std::vector<int> info(3 * count);
        std::size_t max_length = 0;
        for (std::size_t i = 0; i < count; ++i)
        {
            info[i] = int(sequences[first + i].row - row0);
            info[count + i] = int(sequences[first + i].length);
            info[2 * count + i] = int(sequences[first + i].replay);
            max_length = std::max(max_length, sequences[first + i].length);
        }
        std::vector<int> out_rows, out_index;
        for (std::size_t step = 0; step < source_row.size(); ++step)
        {
            if (source_row[step] >= row0 && source_row[step] < row0 + batch)
            {
                out_rows.push_back(int(source_row[step] - row0));
                out_index.push_back(int(step));
            }
        }
        auto* d_feedback = arena_.get<uint16_t>("t.feedback", batch * C);
        auto* d_info = arena_.get<int>("t.info", 3 * count);
        auto* d_rows = arena_.get<int>("t.rows", std::max<std::size_t>(out_rows.size(), 1));
        auto* d_index = arena_.get<int>("t.index", std::max<std::size_t>(out_index.size(), 1));
        check_hip(hipMemcpyAsync(d_feedback, feedback.data() + row0 * C, batch * C * 2,
                                 hipMemcpyHostToDevice, stream_),
                  "upload feedback");
        check_hip(hipMemcpyAsync(d_info, info.data(), info.size() * 4, hipMemcpyHostToDevice, stream_),
                  "upload sequences");
        check_hip(hipMemcpyAsync(d_rows, out_rows.data(), out_rows.size() * 4, hipMemcpyHostToDevice, stream_),
                  "upload rows");
        check_hip(hipMemcpyAsync(d_index, out_index.data(), out_index.size() * 4, hipMemcpyHostToDevice,
                                 stream_),
                  "upload rows");
        auto* embedded = arena_.get<uint16_t>("t.embedded", batch * g.latent);
        auto* x = arena_.get<uint16_t>("t.x", batch * w);
        const Layout layout = activation_layout(batch);
        auto* q8 = arena_.get<int8_t>("t.q8", tile_padded_rows(batch) * std::max<std::size_t>({w, g.ffn, g.latent}));
        auto* s8 = arena_.get<float>("t.s8", tile_padded_rows(batch) * std::max<std::size_t>({w, g.ffn, g.latent}) / 256);
        embed_sum(m.embeddings(), g.alphabet, g.latent, d_feedback, C, batch, embedded, stream_);
        quantize_rows(embedded, batch, g.latent, Prologue::none, nullptr, nullptr, q8, s8, nullptr, err,
                      stream_, layout);
        linear(m.temporal_projection(), q8, s8, batch, x, nullptr, LinearPath::automatic, stream_, layout);
        stack_rows(true, x, batch, d_info, d_info + count, d_info + 2 * count, count, max_length, "t");
        const std::size_t f = m.final_norm_index(true);
        layer_norm_rows(x, batch, w, m.norm_gain(f), m.norm_bias(f), x, stream_);
        copy_rows(x, d_rows, conditioning, d_index, out_rows.size(), w, stream_);
        // Host vectors above must outlive the asynchronous uploads.
        check_hip(hipStreamSynchronize(stream_), "hipStreamSynchronize");
        first = last;
    }
}

void Session::batched(const Header& h, const uint16_t* tokens, uint16_t* distributions,
                      uint16_t* splits, const KnownPlan& plan)
{
    const Geometry& g = model_->geometry();
    const Model& m = *model_;
    const std::size_t C = h.codebooks, w = g.width;
    const std::size_t steps = h.frames * h.groups;
    if (!steps)
    {
        return;
    }
    auto* err = errors_.as<uint32_t>();
    auto* conditioning = arena_.get<uint16_t>("cond", steps * w);
    temporal_rows(h, tokens, conditioning, plan.temporal_rows);
    auto* d_tokens = arena_.get<uint16_t>("tokens", steps * C);
    upload_input(d_tokens, tokens, steps * C * 2);
    const std::size_t chunk_steps = plan.codebook_steps;
    // Codebook sequences: step i of a chunk is rows i*C .. i*C+C-1.
    {
        std::vector<int> info(3 * chunk_steps);
        for (std::size_t i = 0; i < chunk_steps; ++i)
        {
            info[i] = int(i * C);
            info[chunk_steps + i] = int(C);
            info[2 * chunk_steps + i] = 0;
        }
        auto* d_info = arena_.get<int>("c.info", info.size());
        check_hip(hipMemcpyAsync(d_info, info.data(), info.size() * 4, hipMemcpyHostToDevice, stream_),
                  "upload sequences");
        check_hip(hipStreamSynchronize(stream_), "hipStreamSynchronize");
    }
    const int* d_info = arena_.get<int>("c.info", 3 * chunk_steps);
    const std::size_t widest = std::max<std::size_t>({w, g.ffn, g.latent});
    for (std::size_t s0 = 0; s0 < steps; s0 += chunk_steps)
    {
        const std::size_t n = std::min(chunk_steps, steps - s0), rows = n * C;
        auto* prefix = arena_.get<uint16_t>("c.prefix", rows * g.latent);
        auto* y = arena_.get<uint16_t>("c.y", rows * w);
        const Layout layout = activation_layout(rows);
        auto* q8 = arena_.get<int8_t>("c.q8", tile_padded_rows(rows) * widest);
        auto* s8 = arena_.get<float>("c.s8", tile_padded_rows(rows) * widest / 256);
        auto* logits = arena_.get<uint16_t>("c.logits", rows * g.alphabet);
        embed_prefixes(m.embeddings(), g.alphabet, g.latent, d_tokens + s0 * C, C, n, prefix, stream_);
        quantize_rows(prefix, rows, g.latent, Prologue::none, nullptr, nullptr, q8, s8, nullptr, err, stream_, layout);
        linear(m.codebook_projection(), q8, s8, rows, y, nullptr, LinearPath::automatic, stream_, layout);
        scatter_rows(conditioning + s0 * w, n, w, C, 0, y, stream_);
        add_rows(y, m.positions(), rows, w, C, y, stream_);
        stack_rows(false, y, rows, d_info, d_info + chunk_steps, d_info + 2 * chunk_steps, n, C, "c");
        const std::size_t f = m.final_norm_index(false);
        quantize_rows(y, rows, w, Prologue::layer_norm, m.norm_gain(f), m.norm_bias(f), q8, s8, nullptr,
                      err, stream_, layout);
        linear(m.output_projection(), q8, s8, rows, logits, nullptr, LinearPath::automatic, stream_, layout);
        auto* probs = arena_.get<uint16_t>("c.probs", rows * g.alphabet);
        softmax_rows(logits, rows, g.alphabet, probs, err, stream_);
        if (distributions)
        {
            check_hip(hipMemcpyAsync(distributions + s0 * C * g.alphabet, probs, rows * g.alphabet * 2,
                                     hipMemcpyDeviceToHost, stream_),
                      "read distributions");
        }
        if (splits)
        {
            auto* d_splits = arena_.get<uint16_t>("c.splits", rows * 16);
            categorical_paths(probs, rows, g.alphabet, d_tokens + s0 * C, d_splits, err, stream_);
            check_hip(hipMemcpyAsync(splits + s0 * C * 16, d_splits, rows * 16 * 2, hipMemcpyDeviceToHost,
                                     stream_),
                      "read splits");
        }
        check_hip(hipStreamSynchronize(stream_), "hipStreamSynchronize");
    }
}

std::vector<uint8_t> Session::encode(Header h, const uint16_t* tokens, std::size_t count,
                                     const SymbolObserver* observer)
{
    check_hip(hipSetDevice(model_->device()), "hipSetDevice");
    const double t0 = now();
    h.method = 1;
    validate(h, tokens, count);
    require(model_->limits().file_bytes >= 19, "the stream limit is below the 19-byte FBAZ framing");
    const uint32_t crc = token_crc32(tokens, count);
    std::vector<uint16_t> splits(count * 16);
    reset_errors();
    const KnownPlan plan = plan_known(h);
    frame_launch_ = -1;
    if (plan.stepwise)
    {
        stepwise(h, tokens, nullptr, 0, nullptr, nullptr, splits.data());
    }
    else
    {
        batched(h, tokens, nullptr, splits.data(), plan);
    }
    check_errors();
    const double t1 = now();
    // Host range coding in stream order (src/format/entropy.cpp:57-100): the ten
    // Q15 splits along each symbol's bisection path, computed on the GPU.
    RangeEncoder encoder(model_->limits().file_bytes - 18);
    const bool before = observer && observer->before, after = observer && observer->after;
    for_each_position(h, [&](const Position& p)
    {
        if (before)
        {
            observer->before(p);
        }
        const std::size_t start = after ? encoder.bit_position() : 0;
        const uint16_t symbol = tokens[p.offset];
        const uint16_t* s = splits.data() + p.offset * 16;
        std::size_t base = 0, n = 1024;
        for (int level = 0; n > 1; ++level)
        {
            const std::size_t half = n / 2;
            const bool one = symbol >= base + half;
            encoder.put(s[level], one);
            if (one)
            {
                base += half;
                n -= half;
            }
            else
            {
                n = half;
            }
        }
        if (after)
        {
            observer->after(p, encoder.bit_position() - start);
        }
    });
    const auto bytes = frame_normal(h, crc, encoder.finish());
    const double t2 = now();
    timing_ = {t1 - t0, t2 - t1, t2 - t0, input_seconds(), 0.0, 0.0, double(frame_launch_),
               plan.stepwise ? 1.0 : 0.0};
    return bytes;
}

std::vector<uint16_t> Session::decode(const uint8_t* stream, std::size_t length, const SymbolObserver* observer)
{
    check_hip(hipSetDevice(model_->device()), "hipSetDevice");
    const double t0 = now();
    const Header h = parse_header(stream, length, model_->limits());
    require(h.method == 1, "the probability model decodes normal (method 1) streams only");
    validate(h, nullptr, h.symbols());
    std::vector<uint16_t> tokens(h.symbols());
    // The initial interval is validated on the host (src/format/range.cpp:122-129).
    RangeDecoder initial(stream + h.payload_offset, h.payload_bytes);
    reset_errors();
    stepwise(h, nullptr, stream + h.payload_offset, h.payload_bytes, tokens.data(), nullptr);
    check_errors();
    const double t1 = now();
    // Every symbol was decoded on the GPU; observers see them in stream order
    // with 0 bits, as unpack_normal reports them (src/format/entropy.cpp:137-149),
    // before the CRC check.
    if (observer && (observer->before || observer->after))
    {
        for_each_position(h, [&](const Position& p)
        {
            if (observer->before)
            {
                observer->before(p);
            }
            if (observer->after)
            {
                observer->after(p, 0);
            }
        });
    }
    require(token_crc32(tokens.data(), tokens.size()) == h.token_crc,
            "decoded tokens fail the stream's CRC-32 check");
    const double t2 = now();
    const double steps = double(Lanes(h).steps());
    timing_ = {t1 - t0, t2 - t1, t2 - t0, input_seconds(), steps_seconds(), steps, double(frame_launch_), 1.0};
    return tokens;
}

void Session::distributions(Header h, const uint16_t* tokens, std::size_t count, bool decode_pass,
                            uint16_t* out)
{
    check_hip(hipSetDevice(model_->device()), "hipSetDevice");
    const double t0 = now();
    h.method = 1;
    validate(h, tokens, count);
    reset_errors();
    if (decode_pass)
    {
        stepwise(h, tokens, nullptr, 0, nullptr, out);
    }
    else if (const KnownPlan plan = plan_known(h); plan.stepwise)
    {
        stepwise(h, tokens, nullptr, 0, nullptr, out);
        decode_pass = true;
    }
    else
    {
        batched(h, tokens, out, nullptr, plan);
    }
    check_errors();
    const double t1 = now();
    const double steps = decode_pass ? double(Lanes(h).steps()) : 0.0;
    timing_ = {t1 - t0, 0.0, t1 - t0, input_seconds(), decode_pass ? steps_seconds() : 0.0, steps,
               decode_pass ? double(frame_launch_) : -1.0, decode_pass ? 1.0 : 0.0};
}
} // namespace tsac_hip
