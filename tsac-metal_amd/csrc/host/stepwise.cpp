// Decode-side driver: frame by frame, book by book, all ready lanes batched as
// the columns of each projection (src/common/transformer.cpp:137-244 schedule).
// Every kernel of the pass is enqueued up front on the session's stream; the
// range decoder runs on the GPU, so nothing returns to the host until the end.
// Ordinary frame steps (every lane active, no context rollover) replay one
// captured HIP graph whose kernels read the context position and step index
// from device counters.
#include "../kernels/decode.hpp"
#include "../kernels/frame.hpp"
#include "runtime.hpp"

#include <algorithm>
#include <cstring>

namespace tsac_hip
{
namespace
{
constexpr std::size_t replay_frames = 256;
// Frame steps per persistent launch: the launches in between cost ~20 us each,
// and a launch of this many steps holds the device for ~50 ms.
constexpr std::size_t frame_launch_steps = 64;
// Projections batch up to `chunk` lanes as their columns; larger lane sets run
// chunk by chunk, which keeps each (step, book)'s lanes in stream order.
constexpr std::size_t chunk = 8;

struct Graph
{
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    ~Graph()
    {
        if (exec)
        {
            (void)hipGraphExecDestroy(exec);
        }
        if (graph)
        {
            (void)hipGraphDestroy(graph);
        }
    }
};
} // namespace

// One decode-shaped layer (src/common/cpu_transformer.tpp:139-173) over lanes
// first_lane .. first_lane + rows - 1: five launches.
void Session::layer_step(bool temporal, std::size_t layer, uint16_t* x, std::size_t rows,
                         std::size_t first_lane, std::size_t position, const int* device_position,
                         bool replay, std::size_t extent)
{
    const Geometry& g = model_->geometry();
    const Model& m = *model_;
    const std::size_t w = g.width;
    const std::size_t layers = temporal ? g.temporal_layers : g.codebook_layers;
    auto* query = arena_.get<uint16_t>("s.query", chunk * w);
    auto* att = arena_.get<uint16_t>("s.att", chunk * w);
    auto* hidden = arena_.get<uint16_t>("s.hidden", chunk * g.ffn);
    auto* keys = arena_.get<uint16_t>(temporal ? "s.tk" : "s.ck", 0);
    auto* values = arena_.get<uint16_t>(temporal ? "s.tv" : "s.cv", 0);
    auto* err = errors_.as<uint32_t>();
    const long long lane_stride = static_cast<long long>(layers * extent * w);
    uint16_t* layer_keys = keys + first_lane * lane_stride + layer * extent * w;
    uint16_t* layer_values = values + first_lane * lane_stride + layer * extent * w;
    const std::size_t n1 = m.norm_index(temporal, layer, false), n2 = m.norm_index(temporal, layer, true);

    FusedLinear qkv;
    qkv.w = m.layer(temporal, layer, 0);
    qkv.M = int(rows);
    qkv.input = Input::layer_norm;
    qkv.x = x;
    qkv.x_stride = int(w);
    qkv.gain = m.norm_gain(n1);
    qkv.beta = m.norm_bias(n1);
    qkv.error = err;
    qkv.output = Output::qkv;
    qkv.query = query;
    qkv.keys = layer_keys;
    qkv.values = layer_values;
    qkv.lane_stride = lane_stride;
    qkv.width = int(w);
    qkv.head_width = int(g.head_width);
    qkv.rotations = temporal ? m.rotations() : nullptr;
    qkv.position = device_position;
    qkv.fixed_position = int(position);
    fused_linear(qkv, stream_);

    attention_step(query, layer_keys, layer_values, lane_stride, rows, w, g.heads, g.head_width,
                   g.attention_scale, device_position, int(position), extent, replay, att, stream_);

    FusedLinear out;
    out.w = m.layer(temporal, layer, 1);
    out.M = int(rows);
    out.input = Input::bf16;
    out.x = att;
    out.x_stride = int(w);
    out.error = err;
    out.output = Output::residual;
    out.residual = x;
    out.residual_stride = int(w);
    out.y = x;
    out.y_stride = int(w);
    fused_linear(out, stream_);

    FusedLinear up;
    up.w = m.layer(temporal, layer, 2);
    up.M = int(rows);
    up.input = Input::layer_norm;
    up.x = x;
    up.x_stride = int(w);
    up.gain = m.norm_gain(n2);
    up.beta = m.norm_bias(n2);
    up.error = err;
    up.output = Output::gelu;
    up.y = hidden;
    up.y_stride = int(g.ffn);
    fused_linear(up, stream_);

    FusedLinear down;
    down.w = m.layer(temporal, layer, 3);
    down.M = int(rows);
    down.input = Input::bf16;
    down.x = hidden;
    down.x_stride = int(g.ffn);
    down.error = err;
    down.output = Output::residual;
    down.residual = x;
    down.residual_stride = int(w);
    down.y = x;
    down.y_stride = int(w);
    fused_linear(down, stream_);
}

void Session::stepwise(const Header& h, const uint16_t* known, const uint8_t* payload,
                       std::size_t payload_bytes, uint16_t* tokens_out, uint16_t* distributions,
                       uint16_t* splits)
{
    frame_launch_ = -1;
    const Geometry& g = model_->geometry();
    const Model& m = *model_;
    const std::size_t C = h.codebooks, G = h.groups, w = g.width;
    const Lanes lanes(h);
    const std::size_t independent = lanes.count * G;
    const std::size_t symbols = h.symbols();
    if (!independent)
    {
        return;
    }
    const std::size_t extent = std::min<std::size_t>(lanes.length(0), g.context);
    arena_.get<uint16_t>("s.tk", independent * g.temporal_layers * extent * w);
    arena_.get<uint16_t>("s.tv", independent * g.temporal_layers * extent * w);
    arena_.get<uint16_t>("s.ck", independent * g.codebook_layers * C * w);
    arena_.get<uint16_t>("s.cv", independent * g.codebook_layers * C * w);
    arena_.get<uint16_t>("s.query", chunk * w);
    arena_.get<uint16_t>("s.att", chunk * w);
    arena_.get<uint16_t>("s.hidden", chunk * g.ffn);
    auto* current = arena_.get<uint16_t>("s.current", independent * C);
    auto* feedback = arena_.get<uint16_t>("s.feedback", independent * C);
    auto* tokens = arena_.get<uint16_t>("s.tokens", symbols);
    auto* prefix_a = arena_.get<uint16_t>("s.prefix_a", independent * g.latent);
    auto* prefix_b = arena_.get<uint16_t>("s.prefix_b", independent * g.latent);
    auto* x = arena_.get<uint16_t>("s.x", independent * w);
    auto* book0 = arena_.get<uint16_t>("s.book0", independent * w);
    auto* y = arena_.get<uint16_t>("s.y", independent * w);
    auto* logits = arena_.get<uint16_t>("s.logits", independent * g.alphabet);
    auto* row_base = arena_.get<int>("s.row_base", independent);
    auto* counters = arena_.get<int>("s.counters", 2);
    auto* state = arena_.get<DecoderState>("s.state", 1);
    uint16_t* d_known = nullptr;
    uint16_t* d_distributions = nullptr;
    uint8_t* d_payload = nullptr;
    auto* err = errors_.as<uint32_t>();

    std::vector<int> bases(independent);
    for (std::size_t i = 0; i < independent; ++i)
    {
        bases[i] = int((lanes.start(i / G) * G + i % G) * C);
    }
    check_hip(hipMemcpyAsync(row_base, bases.data(), independent * sizeof(int), hipMemcpyHostToDevice,
                             stream_),
              "upload lanes");
    check_hip(hipMemsetAsync(current, 0, independent * C * 2, stream_), "clear tokens");
    if (known)
    {
        d_known = arena_.get<uint16_t>("s.known", symbols);
        check_hip(hipMemcpyAsync(d_known, known, symbols * 2, hipMemcpyHostToDevice, stream_), "upload tokens");
    }
    else
    {
        d_payload = arena_.get<uint8_t>("s.payload", std::max<std::size_t>(payload_bytes, 1));
        if (payload_bytes)
        {
            upload_input(d_payload, payload, payload_bytes);
        }
        // RangeDecoder construction (src/format/range.cpp:122-129): three bytes, zero-extended.
        DecoderState s{0xff0000u, 0, 0, 0, 0};
        for (int i = 0; i < 3; ++i)
        {
            const uint32_t byte = s.offset < payload_bytes ? payload[s.offset] : 0u;
            s.offset += s.offset < payload_bytes ? 1 : 0;
            s.code = (s.code << 8) | byte;
        }
        check_hip(hipMemcpyAsync(state, &s, sizeof s, hipMemcpyHostToDevice, stream_), "upload decoder");
    }
    if (distributions)
    {
        d_distributions = arena_.get<uint16_t>("s.distributions", symbols * g.alphabet);
    }
    require(!splits || known, "stepwise: splits need known tokens");
    uint16_t* d_splits = splits ? arena_.get<uint16_t>("s.splits", symbols * 16) : nullptr;
    // Host data above must reach the device before the host buffers go away.
    check_hip(hipStreamSynchronize(stream_), "hipStreamSynchronize");

    // Temporal stack for lanes [first, first + count) fed by `fed` token rows.
    const auto temporal_step = [&](std::size_t first, std::size_t count, std::size_t position,
                                   const int* device_position, bool replay, const uint16_t* fed)
    {
        FusedLinear project;
        project.w = m.temporal_projection();
        project.M = int(count);
        project.input = Input::embed_sum;
        project.embeddings = m.embeddings();
        project.alphabet = int(g.alphabet);
        project.books = int(C);
        project.tokens = fed + first * C;
        project.token_stride = int(C);
        project.error = err;
        project.output = Output::plain;
        project.y = x + first * w;
        project.y_stride = int(w);
        fused_linear(project, stream_);
        for (std::size_t l = 0; l < g.temporal_layers; ++l)
        {
            layer_step(true, l, x + first * w, count, first, position, device_position, replay, extent);
        }
    };

    // Conditioning + every codebook of one frame step for `active` lanes.
    const auto codebooks = [&](std::size_t active, std::size_t step, const int* device_step)
    {
        layer_norm_add(x, active, w, m.norm_gain(m.final_norm_index(true)),
                       m.norm_bias(m.final_norm_index(true)), m.positions(), book0, stream_);
        uint16_t* prefix_in = nullptr;
        uint16_t* prefix_out = prefix_a;
        for (std::size_t book = 0; book < C; ++book)
        {
            for (std::size_t first = 0; first < active; first += chunk)
            {
                const std::size_t count = std::min(chunk, active - first);
                uint16_t* input = book0 + first * w;
                if (book > 0)
                {
                    FusedLinear project;
                    project.w = m.codebook_projection();
                    project.M = int(count);
                    project.input = Input::embed_accumulate;
                    project.embeddings = m.embeddings();
                    project.alphabet = int(g.alphabet);
                    project.book = int(book - 1);
                    project.x = prefix_in ? prefix_in + first * g.latent : nullptr;
                    project.tokens = current + first * C;
                    project.token_stride = int(C);
                    project.token_offset = int(book - 1);
                    project.prefix_out = prefix_out + first * g.latent;
                    project.error = err;
                    project.output = Output::residual;
                    project.residual = m.positions() + book * w;
                    project.residual_stride = 0;
                    project.y = y + first * w;
                    project.y_stride = int(w);
                    fused_linear(project, stream_);
                    input = y + first * w;
                }
                for (std::size_t l = 0; l < g.codebook_layers; ++l)
                {
                    layer_step(false, l, input, count, first, book, nullptr, false, C);
                }
                FusedLinear head;
                head.w = m.output_projection();
                head.M = int(count);
                head.input = Input::layer_norm;
                head.x = input;
                head.x_stride = int(w);
                head.gain = m.norm_gain(m.final_norm_index(false));
                head.beta = m.norm_bias(m.final_norm_index(false));
                head.error = err;
                head.output = Output::plain;
                head.y = logits + first * g.alphabet;
                head.y_stride = int(g.alphabet);
                fused_linear(head, stream_);

                Sample sample;
                sample.logits = logits + first * g.alphabet;
                sample.lanes = int(count);
                sample.book = int(book);
                sample.books = int(C);
                sample.current = current + first * C;
                sample.tokens = tokens;
                sample.row_base = row_base + first;
                sample.step = device_step;
                sample.fixed_step = int(step);
                sample.step_stride = int(G * C);
                sample.known = d_known;
                sample.distributions = d_distributions;
                sample.splits = d_splits;
                sample.state = known ? nullptr : state;
                sample.payload = d_payload;
                sample.payload_bytes = payload_bytes;
                sample.error = err;
                sample_step(sample, stream_);
            }
            if (book > 0)
            {
                prefix_in = prefix_out;
                prefix_out = prefix_out == prefix_a ? prefix_b : prefix_a;
            }
        }
    };

    // An ordinary step: feedback = the previous complete frame (all-zero
    // indices first), context position from counters[0], step from counters[1].
    const auto ordinary_step = [&](std::size_t active, std::size_t position, std::size_t step,
                                   bool device)
    {
        for (std::size_t first = 0; first < active; first += chunk)
        {
            temporal_step(first, std::min(chunk, active - first), position, device ? counters : nullptr,
                          false, current);
        }
        codebooks(active, step, device ? counters + 1 : nullptr);
    };

    // Frame steps without a context rollover run as one persistent launch each
    // when the geometry has a frame kernel and all lanes fit one launch.
    const bool framed = frame_supported(int(w), int(g.heads), int(g.head_width), int(g.ffn), int(g.latent),
                                        int(g.alphabet), int(independent)) &&
                        extent <= 1024;
    FrameArgs frame;
    if (framed)
    {
        const std::size_t count = frame_exchange_words(int(w), int(g.ffn), int(g.latent), int(g.alphabet), int(C),
                                                       int(g.temporal_layers), int(g.codebook_layers));
        auto* exchange = arena_.get<unsigned long long>("s.exchange", count);
        check_hip(hipMemsetAsync(exchange, 0, count * 8, stream_), "clear exchange words");
        frame.model = m.frame_tables();
        frame.books = int(C);
        frame.temporal_layers = int(g.temporal_layers);
        frame.codebook_layers = int(g.codebook_layers);
        frame.width = int(w);
        frame.heads = int(g.heads);
        frame.head_width = int(g.head_width);
        frame.ffn = int(g.ffn);
        frame.latent = int(g.latent);
        frame.alphabet = int(g.alphabet);
        frame.scale = g.attention_scale;
        frame.keys = arena_.get<uint16_t>("s.tk", 0);
        frame.values = arena_.get<uint16_t>("s.tv", 0);
        frame.lane_stride = static_cast<long long>(g.temporal_layers * extent * w);
        frame.extent = int(extent);
        frame.current = current;
        frame.row_base = row_base;
        frame.step_stride = int(G * C);
        frame.tokens = tokens;
        frame.known = d_known;
        frame.distributions = d_distributions;
        frame.splits = d_splits;
        frame.state = known ? nullptr : state;
        frame.payload = d_payload;
        frame.payload_bytes = payload_bytes;
        frame.error = err;
        frame.words = exchange;
        frame.abort = err + 2;
        const std::vector<uint8_t> table = frame_job_table(frame);
        auto* jobs = arena_.get<uint8_t>("s.jobs", table.size());
        check_hip(hipMemcpyAsync(jobs, table.data(), table.size(), hipMemcpyHostToDevice, stream_), "upload jobs");
        check_hip(hipStreamSynchronize(stream_), "hipStreamSynchronize");
        frame.jobs = jobs;
    }

    Graph graph;
    std::size_t context_used = 0;
    check_hip(hipEventRecord(steps_start_, stream_), "hipEventRecord");
    for (std::size_t step = 0; step < lanes.steps(); ++step)
    {
        const std::size_t active = step < lanes.base ? independent : lanes.extra * G;
        if (framed && context_used != g.context)
        {
            // Consecutive steps with the same lanes and no rollover in one
            // launch, at most frame_launch_steps of them.
            std::size_t n = 1;
            while (n < frame_launch_steps && step + n < lanes.steps() && context_used + n < g.context &&
                   (step + n < lanes.base) == (step < lanes.base))
            {
                ++n;
            }
            frame.lanes = int(active);
            frame.position = int(context_used);
            frame.step = int(step);
            frame.steps = int(n);
            frame.epoch = uint32_t(step + 1); // exchange words are cleared for every pass
            frame.plain_launch = plain_frame_launch_;
            frame_launch_ = std::max(frame_launch_, int(frame_step(frame, stream_)));
            context_used += n;
            step += n - 1;
        }
        else if (context_used == g.context)
        {
            // Context rollover: reset and replay the last 256 complete frames
            // (src/common/transformer.cpp:187-203).
            context_used = 0;
            for (std::size_t k = 0; k < replay_frames; ++k)
            {
                gather_frame(tokens, row_base, int(step - replay_frames + k), int(G * C), int(C), int(active),
                             feedback, stream_);
                for (std::size_t first = 0; first < active; first += chunk)
                {
                    temporal_step(first, std::min(chunk, active - first), context_used, nullptr, true, feedback);
                }
                ++context_used;
            }
            codebooks(active, step, nullptr);
        }
        else if (active == independent && step > 0)
        {
            if (!graph.exec)
            {
                set_counters(counters, int(context_used), int(step), stream_);
                check_hip(hipStreamBeginCapture(stream_, hipStreamCaptureModeThreadLocal), "begin capture");
                try
                {
                    ordinary_step(active, 0, 0, true);
                    advance_counters(counters, stream_);
                }
                catch (...)
                {
                    hipGraph_t broken = nullptr;
                    (void)hipStreamEndCapture(stream_, &broken);
                    if (broken)
                    {
                        (void)hipGraphDestroy(broken);
                    }
                    throw;
                }
                check_hip(hipStreamEndCapture(stream_, &graph.graph), "end capture");
                check_hip(hipGraphInstantiate(&graph.exec, graph.graph, nullptr, nullptr, 0),
                          "instantiate graph");
            }
            else
            {
                set_counters(counters, int(context_used), int(step), stream_);
            }
            check_hip(hipGraphLaunch(graph.exec, stream_), "launch graph");
            ++context_used;
        }
        else
        {
            ordinary_step(active, context_used, step, false);
            ++context_used;
        }
    }
    check_hip(hipEventRecord(steps_stop_, stream_), "hipEventRecord");
    stepped_ = true;
    if (tokens_out)
    {
        check_hip(hipMemcpyAsync(tokens_out, tokens, symbols * 2, hipMemcpyDeviceToHost, stream_),
                  "read tokens");
    }
    if (distributions)
    {
        check_hip(hipMemcpyAsync(distributions, d_distributions, symbols * g.alphabet * 2,
                                 hipMemcpyDeviceToHost, stream_),
                  "read distributions");
    }
    if (splits)
    {
        check_hip(hipMemcpyAsync(splits, d_splits, symbols * 16 * 2, hipMemcpyDeviceToHost, stream_), "read splits");
    }
    check_hip(hipStreamSynchronize(stream_), "hipStreamSynchronize");
}
} // namespace tsac_hip
