// C ABI of the probability model (include/tsac_hip.h). Exceptions stop here and
// become a nonzero status plus a thread-local message.
#include "../../../include/tsac_hip.h"
#include "audio.hpp"
#include "runtime.hpp"
#include "source.hpp"
#include "wave.hpp"

#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <new>
#include <utility>

using namespace tsac_hip;

struct tsac_hip_model
{
    std::shared_ptr<const Model> model;
};

struct tsac_hip_session
{
    std::unique_ptr<Session> session;
};

struct tsac_hip_dac
{
    std::unique_ptr<DacModel> dac;
};

struct tsac_hip_source
{
    SourceModel model;
};

struct tsac_hip_prepared_transformer
{
    PreparedTransformer prepared;
};

struct tsac_hip_prepared_dac
{
    PreparedDac prepared;
};

struct tsac_hip_device_linear
{
    DeviceBuffer values, constants;
    DeviceLinear linear;
};

namespace
{
thread_local std::string last_error;

template <class F> int guarded(F&& f)
{
    try
    {
        f();
        last_error.clear();
        return TSAC_HIP_OK;
    }
    catch (const std::bad_alloc&)
    {
        last_error = "out of host memory";
    }
    catch (const std::exception& e)
    {
        last_error = e.what();
    }
    return TSAC_HIP_ERROR;
}

hipStream_t as_stream(void* stream)
{
    return static_cast<hipStream_t>(stream);
}

Limits limits_of(const tsac_hip_limits* l)
{
    Limits r;
    if (l)
    {
        r.file_bytes = l->file_bytes ? l->file_bytes : r.file_bytes;
        r.symbols = l->symbols ? l->symbols : r.symbols;
        r.pcm_bytes = l->pcm_bytes ? l->pcm_bytes : r.pcm_bytes;
        r.cache_bytes = l->cache_bytes ? l->cache_bytes : r.cache_bytes;
        r.tensor_elements = l->tensor_elements ? l->tensor_elements : r.tensor_elements;
    }
    return r;
}

Header header_of(const tsac_hip_header* h)
{
    require(h != nullptr, "missing header");
    Header r;
    r.method = h->method;
    r.groups = h->groups;
    r.model_channels = h->model_channels;
    r.codebooks = h->codebooks;
    r.frames = h->frames;
    r.batch = h->batch;
    return r;
}

template <class T> T* copy_out(const std::vector<T>& v)
{
    T* p = static_cast<T*>(std::malloc(v.empty() ? 1 : v.size() * sizeof(T)));
    if (!p)
    {
        throw std::bad_alloc();
    }
    if (!v.empty())
    {
        std::memcpy(p, v.data(), v.size() * sizeof(T));
    }
    return p;
}

// Stream-ordered scratch for the operator entry points.
struct AsyncScratch
{
    void* pointer = nullptr;
    hipStream_t stream;
    AsyncScratch(std::size_t bytes, hipStream_t s) : stream(s)
    {
        check_hip(hipMallocAsync(&pointer, bytes ? bytes : 256, s), "hipMallocAsync");
    }
    ~AsyncScratch()
    {
        (void)hipFreeAsync(pointer, stream);
    }
};

// Decode-attention scratch kept per (device, stream): arrival counters at
// the start, block records after them. The kernel leaves its counters at
// zero, so they are cleared when allocated and then serve every later call on
// that stream, which runs after the earlier ones. Allocation, clearing and
// the release of an outgrown buffer are all ordered on the stream.
class DecodeScratch
{
  public:
    struct View
    {
        unsigned* arrivals;
        float* partial;
    };

    View get(hipStream_t stream, std::size_t counters, std::size_t floats)
    {
        int device = 0;
        check_hip(hipGetDevice(&device), "hipGetDevice");
        const std::lock_guard<std::mutex> lock(mutex_);
        Entry& e = entries_[{device, stream}];
        if (e.counters < counters || e.floats < floats)
        {
            const Entry grown{nullptr, std::max(e.counters, (counters + 63) / 64 * 64), std::max(e.floats, floats)};
            if (e.pointer)
            {
                check_hip(hipFreeAsync(e.pointer, stream), "hipFreeAsync");
                e = Entry{};
            }
            check_hip(hipMallocAsync(&e.pointer, grown.counters * 4 + grown.floats * 4, stream), "hipMallocAsync");
            e.counters = grown.counters;
            e.floats = grown.floats;
            clear_arrival_counters(static_cast<unsigned*>(e.pointer), e.counters, stream);
        }
        return {static_cast<unsigned*>(e.pointer), reinterpret_cast<float*>(static_cast<unsigned*>(e.pointer) + e.counters)};
    }

  private:
    struct Entry
    {
        void* pointer = nullptr;
        std::size_t counters = 0;
        std::size_t floats = 0;
    };
    std::mutex mutex_;
    std::map<std::pair<int, hipStream_t>, Entry> entries_;
};

DecodeScratch& decode_scratch()
{
    static DecodeScratch* cache = new DecodeScratch; // outlives every static destructor
    return *cache;
}

tsac_hip_position position_of(const Position& p)
{
    return {p.frame, p.group, p.book, p.lane, p.step, p.offset};
}

// The C callbacks as the session's observer; a nonzero return becomes an
// exception that ends the call.
SymbolObserver observer_of(const tsac_hip_observer* o)
{
    SymbolObserver r;
    if (o && o->before_symbol)
    {
        r.before = [o](const Position& p)
        {
            const tsac_hip_position c = position_of(p);
            require(o->before_symbol(o->context, &c) == 0, "stopped by the observer (before_symbol)");
        };
    }
    if (o && o->after_symbol)
    {
        r.after = [o](const Position& p, std::size_t bits)
        {
            const tsac_hip_position c = position_of(p);
            require(o->after_symbol(o->context, &c, bits) == 0, "stopped by the observer (after_symbol)");
        };
    }
    return r;
}

SourceLimits source_limits_of(const tsac_hip_source_limits* l)
{
    SourceLimits r;
    if (l)
    {
        r.file_bytes = l->file_bytes ? l->file_bytes : r.file_bytes;
        r.tensor_elements = l->tensor_elements ? l->tensor_elements : r.tensor_elements;
        r.tensors = l->tensors ? l->tensors : r.tensors;
        r.metadata_bytes = l->metadata_bytes ? l->metadata_bytes : r.metadata_bytes;
        r.name_bytes = l->name_bytes ? l->name_bytes : r.name_bytes;
    }
    return r;
}

void fill_model_desc(const ModelDesc& m, tsac_hip_model_desc* desc)
{
    const Geometry& g = m.geometry;
    desc->geometry = tsac_hip_geometry{g.width,  g.heads,    g.head_width, g.ffn,   g.temporal_layers,
                                       g.codebook_layers, g.latent, g.alphabet, g.books, g.channels,
                                       g.context, g.attention_scale};
    static_assert(sizeof(LinearHost) == sizeof(tsac_hip_linear));
    desc->projections = reinterpret_cast<const tsac_hip_linear*>(m.projections);
    desc->norm_gain = m.gain;
    desc->norm_bias = m.bias;
    desc->positions = m.positions;
    desc->rotations = m.rotations;
    desc->embeddings = m.embeddings;
}

void fill_dac_desc(const PreparedDac& d, tsac_hip_dac_desc* desc)
{
    static_assert(sizeof(DacConvolutionSource) == sizeof(tsac_hip_dac_convolution));
    static_assert(sizeof(RvqSource) == sizeof(tsac_hip_rvq_book));
    *desc = tsac_hip_dac_desc{};
    desc->channels = d.channels();
    desc->books = d.books();
    std::memcpy(desc->analysis, d.analysis(), sizeof desc->analysis);
    std::memcpy(desc->synthesis, d.synthesis(), sizeof desc->synthesis);
    std::memcpy(desc->analysis_alpha, d.analysis_alpha(), sizeof desc->analysis_alpha);
    std::memcpy(desc->synthesis_alpha, d.synthesis_alpha(), sizeof desc->synthesis_alpha);
    std::memcpy(desc->rvq, d.rvq(), d.books() * sizeof(tsac_hip_rvq_book));
}

LinearPath path_of(int path)
{
    require(path >= 0 && path <= 4 && path != TSAC_HIP_PATH_GEMM_TILES, "invalid linear path");
    return path == TSAC_HIP_PATH_GEMV    ? LinearPath::gemv
           : path == TSAC_HIP_PATH_GEMM  ? LinearPath::gemm
           : path == TSAC_HIP_PATH_SMALL ? LinearPath::small
                                         : LinearPath::automatic;
}
} // namespace

extern "C"
{
const char* tsac_hip_last_error(void)
{
    return last_error.c_str();
}

int tsac_hip_model_create(const tsac_hip_model_desc* desc, const tsac_hip_limits* limits,
                          tsac_hip_model** model)
{
    return guarded(
        [&]
        {
            require(desc && model, "missing argument");
            const auto& d = desc->geometry;
            Geometry g;
            g.width = d.width;
            g.heads = d.heads;
            g.head_width = d.head_width;
            g.ffn = d.ffn;
            g.temporal_layers = d.temporal_layers;
            g.codebook_layers = d.codebook_layers;
            g.latent = d.latent;
            g.alphabet = d.alphabet;
            g.books = d.books;
            g.channels = d.channels;
            g.context = d.context;
            g.attention_scale = d.attention_scale;
            static_assert(sizeof(LinearHost) == sizeof(tsac_hip_linear));
            auto m = std::make_shared<const Model>(
                g, reinterpret_cast<const LinearHost*>(desc->projections), desc->norm_gain,
                desc->norm_bias, desc->positions, desc->rotations, desc->embeddings, limits_of(limits));
            *model = new tsac_hip_model{std::move(m)};
        });
}

void tsac_hip_model_destroy(tsac_hip_model* model)
{
    delete model;
}

int tsac_hip_session_create(tsac_hip_model* model, tsac_hip_session** session)
{
    return guarded(
        [&]
        {
            require(model && session, "missing argument");
            *session = new tsac_hip_session{std::make_unique<Session>(model->model)};
        });
}

void tsac_hip_session_destroy(tsac_hip_session* session)
{
    delete session;
}

int tsac_hip_session_clear(tsac_hip_session* session)
{
    return guarded(
        [&]
        {
            require(session, "missing session");
            session->session->clear();
        });
}

int tsac_hip_encode(tsac_hip_session* session, const tsac_hip_header* header,
                    const uint16_t* tokens, size_t count, uint8_t** stream, size_t* length)
{
    return tsac_hip_encode_observed(session, header, tokens, count, nullptr, stream, length);
}

int tsac_hip_encode_observed(tsac_hip_session* session, const tsac_hip_header* header,
                             const uint16_t* tokens, size_t count, const tsac_hip_observer* observer,
                             uint8_t** stream, size_t* length)
{
    return guarded(
        [&]
        {
            require(session && stream && length && (tokens || !count), "missing argument");
            const SymbolObserver o = observer_of(observer);
            const auto bytes = session->session->encode(header_of(header), tokens, count, observer ? &o : nullptr);
            *stream = copy_out(bytes);
            *length = bytes.size();
        });
}

int tsac_hip_decode(tsac_hip_session* session, const uint8_t* stream, size_t length,
                    uint16_t** tokens, size_t* count)
{
    return tsac_hip_decode_observed(session, stream, length, nullptr, tokens, count);
}

int tsac_hip_decode_observed(tsac_hip_session* session, const uint8_t* stream, size_t length,
                             const tsac_hip_observer* observer, uint16_t** tokens, size_t* count)
{
    return guarded(
        [&]
        {
            require(session && stream && tokens && count, "missing argument");
            const SymbolObserver o = observer_of(observer);
            const auto t = session->session->decode(stream, length, observer ? &o : nullptr);
            *tokens = copy_out(t);
            *count = t.size();
        });
}

void tsac_hip_free(void* pointer)
{
    std::free(pointer);
}

int tsac_hip_dac_create(const tsac_hip_dac_desc* desc, const tsac_hip_limits* limits, tsac_hip_dac** dac)
{
    return guarded(
        [&]
        {
            require(desc && dac, "missing argument");
            static_assert(sizeof(DacConvolutionSource) == sizeof(tsac_hip_dac_convolution));
            static_assert(sizeof(RvqSource) == sizeof(tsac_hip_rvq_book));
            require(desc->books >= 1 && desc->books <= 12, "DAC model codebooks out of range");
            *dac = new tsac_hip_dac{std::make_unique<DacModel>(
                desc->channels, desc->books, reinterpret_cast<const DacConvolutionSource*>(desc->analysis),
                desc->analysis_alpha, reinterpret_cast<const DacConvolutionSource*>(desc->synthesis),
                desc->synthesis_alpha, reinterpret_cast<const RvqSource*>(desc->rvq), limits_of(limits))};
        });
}

void tsac_hip_dac_destroy(tsac_hip_dac* dac)
{
    delete dac;
}


int tsac_hip_source_load(const char* path, const tsac_hip_source_limits* limits, tsac_hip_source** source)
{
    return guarded(
        [&]
        {
            require(path && source, "missing argument");
            *source = new tsac_hip_source{SourceModel::load(path, source_limits_of(limits))};
        });
}

int tsac_hip_source_parse(const uint8_t* bytes, size_t length, const tsac_hip_source_limits* limits,
                          tsac_hip_source** source)
{
    return guarded(
        [&]
        {
            require((bytes || !length) && source, "missing argument");
            *source = new tsac_hip_source{
                SourceModel::parse(std::vector<uint8_t>(bytes, bytes + length), source_limits_of(limits))};
        });
}

void tsac_hip_source_destroy(tsac_hip_source* source)
{
    delete source;
}

int tsac_hip_source_tensor_count(const tsac_hip_source* source, size_t* count)
{
    return guarded(
        [&]
        {
            require(source && count, "missing argument");
            *count = source->model.tensors().size();
        });
}

int tsac_hip_source_tensor_info(const tsac_hip_source* source, size_t index, tsac_hip_source_tensor* info)
{
    return guarded(
        [&]
        {
            require(source && info, "missing argument");
            require(index < source->model.tensors().size(), "tensor index out of range");
            const SourceTensor& t = source->model.tensors()[index];
            *info = tsac_hip_source_tensor{};
            info->name = t.name.c_str();
            info->storage = uint32_t(t.storage);
            info->rank = uint32_t(t.dims.size());
            for (std::size_t a = 0; a < t.dims.size(); ++a)
            {
                info->dims[a] = t.dims[a];
            }
            info->elements = t.elements;
        });
}

int tsac_hip_source_metadata(const tsac_hip_source* source, const char** json, size_t* length)
{
    return guarded(
        [&]
        {
            require(source && json && length, "missing argument");
            *json = source->model.metadata().data();
            *length = source->model.metadata().size();
        });
}

int tsac_hip_source_dequantize(const tsac_hip_source* source, const char* name, float* out, size_t capacity)
{
    return guarded(
        [&]
        {
            require(source && name && out, "missing argument");
            const auto values = source->model.dequantize(name);
            require(values.size() <= capacity, "output buffer too small for the tensor");
            std::memcpy(out, values.data(), values.size() * sizeof(float));
        });
}

int tsac_hip_source_dac_config(const tsac_hip_source* source, uint32_t* channels, uint32_t* books)
{
    return guarded(
        [&]
        {
            require(source && channels && books, "missing argument");
            const SourceDacConfig c = source_dac_config(source->model);
            *channels = c.channels;
            *books = c.books;
        });
}

int tsac_hip_source_transformer_config(const tsac_hip_source* source, uint32_t* books)
{
    return guarded(
        [&]
        {
            require(source && books, "missing argument");
            *books = source_transformer_books(source->model);
        });
}

int tsac_hip_prepare_transformer(const tsac_hip_source* transformer, const tsac_hip_source* dac,
                                 tsac_hip_prepared_transformer** prepared, tsac_hip_model_desc* desc)
{
    return guarded(
        [&]
        {
            require(transformer && dac && prepared && desc, "missing argument");
            auto p = std::make_unique<tsac_hip_prepared_transformer>(
                tsac_hip_prepared_transformer{PreparedTransformer(transformer->model, dac->model)});
            fill_model_desc(p->prepared.desc(), desc);
            *prepared = p.release();
        });
}

void tsac_hip_prepared_transformer_destroy(tsac_hip_prepared_transformer* prepared)
{
    delete prepared;
}

int tsac_hip_prepare_dac(const tsac_hip_source* dac, tsac_hip_prepared_dac** prepared, tsac_hip_dac_desc* desc)
{
    return guarded(
        [&]
        {
            require(dac && prepared && desc, "missing argument");
            auto p = std::make_unique<tsac_hip_prepared_dac>(tsac_hip_prepared_dac{PreparedDac(dac->model)});
            fill_dac_desc(p->prepared, desc);
            *prepared = p.release();
        });
}

void tsac_hip_prepared_dac_destroy(tsac_hip_prepared_dac* prepared)
{
    delete prepared;
}

int tsac_hip_model_create_from_source(const tsac_hip_source* transformer, const tsac_hip_source* dac,
                                      const tsac_hip_limits* limits, tsac_hip_model** model)
{
    tsac_hip_prepared_transformer* prepared = nullptr;
    tsac_hip_model_desc desc{};
    if (const int status = tsac_hip_prepare_transformer(transformer, dac, &prepared, &desc); status != TSAC_HIP_OK)
    {
        return status;
    }
    const int status = model ? tsac_hip_model_create(&desc, limits, model) : TSAC_HIP_ERROR;
    if (!model)
    {
        last_error = "missing argument";
    }
    tsac_hip_prepared_transformer_destroy(prepared);
    return status;
}

int tsac_hip_dac_create_from_source(const tsac_hip_source* dac, const tsac_hip_limits* limits, tsac_hip_dac** model)
{
    tsac_hip_prepared_dac* prepared = nullptr;
    tsac_hip_dac_desc desc{};
    if (const int status = tsac_hip_prepare_dac(dac, &prepared, &desc); status != TSAC_HIP_OK)
    {
        return status;
    }
    const int status = model ? tsac_hip_dac_create(&desc, limits, model) : TSAC_HIP_ERROR;
    if (!model)
    {
        last_error = "missing argument";
    }
    tsac_hip_prepared_dac_destroy(prepared);
    return status;
}

int tsac_hip_pcm16_read(const uint8_t* bytes, size_t length, uint32_t channels, const tsac_hip_limits* limits,
                        float** samples, size_t* frames)
{
    return guarded(
        [&]
        {
            require((bytes || !length) && samples && frames, "missing argument");
            const Pcm pcm = pcm16_input(bytes, length, channels, limits_of(limits));
            *samples = copy_out(pcm.samples);
            *frames = pcm.frames;
        });
}

int tsac_hip_wave_read(const uint8_t* bytes, size_t length, const tsac_hip_limits* limits, float** samples,
                       size_t* frames, uint32_t* channels)
{
    return guarded(
        [&]
        {
            require((bytes || !length) && samples && frames && channels, "missing argument");
            const Pcm pcm = wave_input(bytes, length, limits_of(limits));
            *samples = copy_out(pcm.samples);
            *frames = pcm.frames;
            *channels = pcm.channels;
        });
}

int tsac_hip_wave_write(const float* samples, size_t frames, uint32_t channels, const tsac_hip_limits* limits,
                        uint8_t** bytes, size_t* length)
{
    return guarded(
        [&]
        {
            require((samples || !frames) && bytes && length, "missing argument");
            const auto wave = pcm16_wave(samples, frames, channels, limits_of(limits));
            *bytes = copy_out(wave);
            *length = wave.size();
        });
}

int tsac_hip_audio_header(size_t frames, uint32_t channels, const tsac_hip_encode_options* options,
                          const tsac_hip_limits* limits, tsac_hip_header* header)
{
    return guarded(
        [&]
        {
            require(header, "missing argument");
            EncodeOptions o;
            if (options)
            {
                o.method = options->method;
                o.codebooks = options->codebooks;
                o.separate_channels = options->separate_channels != 0;
                if (options->entropy_batch)
                {
                    o.entropy_batch = options->entropy_batch;
                }
            }
            const Header h = audio_header(frames, channels, o, limits_of(limits));
            *header = tsac_hip_header{h.method, h.groups, h.model_channels, h.codebooks, h.frames, h.batch};
        });
}

int tsac_hip_parse_header(const uint8_t* stream, size_t length, const tsac_hip_limits* limits,
                          tsac_hip_header* header)
{
    return guarded(
        [&]
        {
            require((stream || !length) && header, "missing argument");
            const Header h = parse_header(stream, length, limits_of(limits));
            *header = tsac_hip_header{h.method, h.groups, h.model_channels, h.codebooks, h.frames, h.batch};
        });
}

int tsac_hip_cli_parse(size_t count, const char* const* arguments, tsac_hip_cli_options* options)
{
    return guarded(
        [&]
        {
            require((arguments || !count) && options, "missing argument");
            std::vector<std::string_view> args;
            for (size_t i = 0; i < count; ++i)
            {
                require(arguments[i] != nullptr, "missing argument");
                args.emplace_back(arguments[i]);
            }
            const CliOptions o = parse_cli(args);
            *options = tsac_hip_cli_options{};
            options->command = o.command;
            // Views of whole arguments, so their data is NUL-terminated.
            options->input = o.input.empty() ? nullptr : o.input.data();
            options->output = o.output.empty() ? nullptr : o.output.data();
            options->threads = o.threads;
            options->quality = o.quality;
            options->channels = o.channels;
            options->batch = o.batch;
            options->verbose = o.verbose;
            options->fast = o.fast;
            options->separate = o.separate;
            options->help = o.help;
            options->metal = o.metal;
        });
}

const char* tsac_hip_cli_help(void)
{
    return cli_help().data();
}

int tsac_hip_prepare_rvq(const float* codebook, const float* in_v, const float* in_g, const float* out_v,
                         const float* out_g, float* search, float* input_weights, float* output_weights)
{
    return guarded(
        [&]
        {
            require(codebook && in_v && in_g && out_v && out_g && search && input_weights && output_weights,
                    "missing argument");
            prepare_rvq(codebook, in_v, in_g, out_v, out_g, search, input_weights, output_weights);
        });
}

int tsac_hip_dac_analyze(tsac_hip_session* session, const tsac_hip_dac* dac, const float* pcm, size_t frames,
                         size_t groups, uint32_t codebooks, uint16_t* tokens)
{
    return guarded(
        [&]
        {
            require(session && dac && (pcm || !frames) && (tokens || !frames), "missing argument");
            session->session->analyze(*dac->dac, pcm, frames, groups, codebooks, tokens);
        });
}

int tsac_hip_dac_synthesize(tsac_hip_session* session, const tsac_hip_dac* dac, const uint16_t* tokens,
                            size_t frames, size_t groups, uint32_t codebooks, float* pcm)
{
    return guarded(
        [&]
        {
            require(session && dac && (pcm || !frames) && (tokens || !frames), "missing argument");
            session->session->synthesize(*dac->dac, tokens, frames, groups, codebooks, pcm);
        });
}

int tsac_hip_dac_apply(tsac_hip_session* session, const tsac_hip_dac* dac, int synthesis, const float* input,
                       size_t frames, float* output)
{
    return guarded(
        [&]
        {
            require(session && dac && input && output, "missing argument");
            session->session->dac_apply(*dac->dac, synthesis != 0, input, frames, output);
        });
}

int tsac_hip_audio_encode(tsac_hip_session* session, const tsac_hip_dac* dac, const float* samples, size_t frames,
                          uint32_t channels, const tsac_hip_encode_options* options,
                          const tsac_hip_observer* observer, uint8_t** stream, size_t* length)
{
    return guarded(
        [&]
        {
            require(session && dac && (samples || !frames) && stream && length, "missing argument");
            EncodeOptions o;
            if (options)
            {
                o.method = options->method;
                o.codebooks = options->codebooks;
                o.separate_channels = options->separate_channels != 0;
                if (options->entropy_batch)
                {
                    o.entropy_batch = options->entropy_batch;
                }
            }
            const SymbolObserver obs = observer_of(observer);
            const auto bytes =
                session->session->encode_audio(*dac->dac, samples, frames, channels, o, observer ? &obs : nullptr);
            *stream = copy_out(bytes);
            *length = bytes.size();
        });
}

int tsac_hip_audio_decode(tsac_hip_session* session, const tsac_hip_dac* dac, const uint8_t* stream, size_t length,
                          const tsac_hip_observer* observer, float** samples, size_t* frames, uint32_t* channels)
{
    return guarded(
        [&]
        {
            require(session && dac && stream && samples && frames && channels, "missing argument");
            const SymbolObserver obs = observer_of(observer);
            std::size_t c = 0;
            const auto pcm = session->session->decode_audio(*dac->dac, stream, length, observer ? &obs : nullptr, &c);
            *samples = copy_out(pcm);
            *channels = uint32_t(c);
            *frames = c ? pcm.size() / c : 0;
        });
}

int tsac_hip_distributions(tsac_hip_session* session, const tsac_hip_header* header,
                           const uint16_t* tokens, size_t count, int mode, uint16_t* out)
{
    return guarded(
        [&]
        {
            require(session && out && (tokens || !count), "missing argument");
            require(mode == TSAC_HIP_PASS_ENCODE || mode == TSAC_HIP_PASS_DECODE, "invalid pass");
            session->session->distributions(header_of(header), tokens, count,
                                            mode == TSAC_HIP_PASS_DECODE, out);
        });
}

int tsac_hip_session_timing(const tsac_hip_session* session, double* seconds, size_t count)
{
    return guarded(
        [&]
        {
            require(session && seconds, "missing argument");
            const auto t = session->session->timing();
            for (size_t i = 0; i < count && i < t.size(); ++i)
            {
                seconds[i] = t[i];
            }
        });
}

int tsac_hip_linear_create(const tsac_hip_linear* weights, size_t K, size_t N,
                           tsac_hip_device_linear** linear)
{
    return guarded(
        [&]
        {
            require(weights && linear && weights->values && weights->scales && weights->bias,
                    "missing argument");
            require(K >= 256 && K % 256 == 0 && N > 0, "invalid generated linear shape");
            auto l = std::make_unique<tsac_hip_device_linear>();
            l->values = DeviceBuffer(K * N);
            const std::size_t scale_bytes = K / 256 * N * 4;
            l->constants = DeviceBuffer((scale_bytes + 255) / 256 * 256 + N * 4);
            auto* c = l->constants.as<uint8_t>();
            std::vector<int8_t> tiled(K * N);
            tile_weights(weights->values, K, N, tiled.data());
            check_hip(hipMemcpy(l->values.get(), tiled.data(), K * N, hipMemcpyHostToDevice), "upload");
            check_hip(hipMemcpy(c, weights->scales, scale_bytes, hipMemcpyHostToDevice), "upload");
            check_hip(hipMemcpy(c + (scale_bytes + 255) / 256 * 256, weights->bias, N * 4,
                                hipMemcpyHostToDevice),
                      "upload");
            l->linear = {l->values.as<int8_t>(), reinterpret_cast<const float*>(c),
                         reinterpret_cast<const float*>(c + (scale_bytes + 255) / 256 * 256), K, N};
            *linear = l.release();
        });
}

void tsac_hip_linear_destroy(tsac_hip_device_linear* linear)
{
    delete linear;
}

int tsac_hip_linear_apply(const tsac_hip_device_linear* linear, const uint16_t* x, size_t M,
                          uint16_t* y, int path, void* stream)
{
    return guarded(
        [&]
        {
            require(linear && (x || !M) && (y || !M), "missing argument");
            const auto s = as_stream(stream);
            const std::size_t K = linear->linear.K;
            const LinearPath chosen = path_of(path);
            // The GEMM reads MFMA operand tiles; the GEMV and the small-M GEMM read rows.
            const bool tiles = chosen == LinearPath::gemm ||
                               (chosen == LinearPath::automatic && M > small_gemm_max_rows() &&
                                !small_gemm_chosen(M, linear->linear.N, K));
            const Layout layout = tiles ? Layout::tiles : Layout::rows;
            const std::size_t rows = tiles ? tile_padded_rows(M) : M;
            AsyncScratch scratch(rows * K + rows * (K / 256) * 4 + 256 + 8, s);
            auto* q = static_cast<int8_t*>(scratch.pointer);
            auto* scales =
                reinterpret_cast<float*>(static_cast<uint8_t*>(scratch.pointer) + (rows * K + 255) / 256 * 256);
            auto* error = reinterpret_cast<uint32_t*>(scales + rows * (K / 256));
            check_hip(hipMemsetAsync(error, 0, 8, s), "hipMemsetAsync");
            quantize_rows(x, M, K, Prologue::none, nullptr, nullptr, q, scales, nullptr, error, s, layout);
            tsac_hip::linear(linear->linear, q, scales, M, y, nullptr, chosen, s, layout);
            uint32_t flags[2];
            check_hip(hipMemcpyAsync(flags, error, 8, hipMemcpyDeviceToHost, s), "read error words");
            check_hip(hipStreamSynchronize(s), "hipStreamSynchronize");
            require(!flags[0], "BF8L activations must be finite");
        });
}

int tsac_hip_linear_apply_static(const tsac_hip_device_linear* linear, const uint16_t* x, size_t M,
                                 uint16_t* y, int path, void* stream)
{
    return guarded(
        [&]
        {
            require(linear && (x || !M) && (y || !M), "missing argument");
            linear_apply_static(linear->linear, x, M, y, path_of(path), as_stream(stream));
        });
}

int tsac_hip_linear_apply_quantized(const tsac_hip_device_linear* linear, const int8_t* q,
                                    const float* scales, size_t M, uint16_t* y,
                                    const uint16_t* residual, int path, void* stream)
{
    return guarded(
        [&]
        {
            require(linear && (q || !M) && (scales || !M) && (y || !M), "missing argument");
            if (path == TSAC_HIP_PATH_GEMM_TILES)
            {
                tsac_hip::linear(linear->linear, q, scales, M, y, residual, LinearPath::gemm, as_stream(stream),
                                 Layout::tiles);
                return;
            }
            tsac_hip::linear(linear->linear, q, scales, M, y, residual, path_of(path), as_stream(stream));
        });
}

int tsac_hip_bf8l(const uint16_t* x, size_t rows, size_t K, int8_t* q, float* scales, void* stream)
{
    return guarded(
        [&]
        {
            const auto s = as_stream(stream);
            AsyncScratch scratch(8, s);
            auto* error = static_cast<uint32_t*>(scratch.pointer);
            check_hip(hipMemsetAsync(error, 0, 8, s), "hipMemsetAsync");
            quantize_rows(x, rows, K, Prologue::none, nullptr, nullptr, q, scales, nullptr, error, s);
            uint32_t flags[2];
            check_hip(hipMemcpyAsync(flags, error, 8, hipMemcpyDeviceToHost, s), "read error words");
            check_hip(hipStreamSynchronize(s), "hipStreamSynchronize");
            require(!flags[0], "BF8L activations must be finite");
        });
}

int tsac_hip_bf8l_tiles(const uint16_t* x, size_t rows, size_t K, int8_t* q, float* scales, void* stream)
{
    return guarded(
        [&]
        {
            const auto s = as_stream(stream);
            AsyncScratch scratch(8, s);
            auto* error = static_cast<uint32_t*>(scratch.pointer);
            check_hip(hipMemsetAsync(error, 0, 8, s), "hipMemsetAsync");
            quantize_rows(x, rows, K, Prologue::none, nullptr, nullptr, q, scales, nullptr, error, s,
                          Layout::tiles);
            uint32_t flags[2];
            check_hip(hipMemcpyAsync(flags, error, 8, hipMemcpyDeviceToHost, s), "read error words");
            check_hip(hipStreamSynchronize(s), "hipStreamSynchronize");
            require(!flags[0], "BF8L activations must be finite");
        });
}

size_t tsac_hip_tile_rows(size_t rows)
{
    return tile_padded_rows(rows);
}

int tsac_hip_layer_norm(const uint16_t* x, size_t rows, size_t width, const uint16_t* gain,
                        const uint16_t* bias, uint16_t* out, void* stream)
{
    return guarded([&] { layer_norm_rows(x, rows, width, gain, bias, out, as_stream(stream)); });
}

int tsac_hip_softmax(const uint16_t* x, size_t rows, size_t width, uint16_t* out, void* stream)
{
    return guarded(
        [&]
        {
            const auto s = as_stream(stream);
            AsyncScratch scratch(8, s);
            auto* error = static_cast<uint32_t*>(scratch.pointer);
            check_hip(hipMemsetAsync(error, 0, 8, s), "hipMemsetAsync");
            softmax_rows(x, rows, width, out, error, s);
            uint32_t flags[2];
            check_hip(hipMemcpyAsync(flags, error, 8, hipMemcpyDeviceToHost, s), "read error words");
            check_hip(hipStreamSynchronize(s), "hipStreamSynchronize");
            require(!flags[0], "softmax input must be finite");
        });
}

int tsac_hip_gelu(const uint16_t* x, size_t count, uint16_t* out, void* stream)
{
    return guarded([&] { gelu_values(x, count, out, as_stream(stream)); });
}

int tsac_hip_rotary(const uint16_t* x, const uint16_t* coefficients, size_t count, uint16_t* out,
                    void* stream)
{
    return guarded([&] { rotary_values(x, coefficients, count, out, as_stream(stream)); });
}

int tsac_hip_add(const uint16_t* a, const uint16_t* b, size_t rows, size_t width, size_t period,
                 uint16_t* out, void* stream)
{
    return guarded([&] { add_rows(a, b, rows, width, period, out, as_stream(stream)); });
}

int tsac_hip_attention(const uint16_t* query, const uint16_t* keys, const uint16_t* values,
                       size_t sequence_stride, size_t sequences, size_t time, size_t heads,
                       size_t head_width, float scale, int prefill, uint16_t* out, void* stream)
{
    return guarded(
        [&]
        {
            const auto s = as_stream(stream);
            const std::size_t floats = decode_partial_floats(sequences, heads, head_width, time);
            const std::size_t counters = decode_arrival_counters(sequences, heads, time);
            if (floats == 0)
            {
                attention_decode(query, keys, values, sequence_stride, sequences, time, heads, head_width, scale,
                                 prefill != 0, nullptr, nullptr, out, s);
                return;
            }
            hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
            check_hip(hipStreamIsCapturing(s, &capture), "hipStreamIsCapturing");
            if (capture != hipStreamCaptureStatusNone)
            {
                // A captured call gets scratch of its own, cleared by a kernel
                // inside the graph.
                AsyncScratch scratch(counters * 4 + floats * 4, s);
                const auto arrivals = static_cast<unsigned*>(scratch.pointer);
                clear_arrival_counters(arrivals, counters, s);
                attention_decode(query, keys, values, sequence_stride, sequences, time, heads, head_width,
                                 scale, prefill != 0, reinterpret_cast<float*>(arrivals + counters), arrivals, out, s);
                return;
            }
            const DecodeScratch::View scratch = decode_scratch().get(s, counters, floats);
            attention_decode(query, keys, values, sequence_stride, sequences, time, heads, head_width, scale,
                             prefill != 0, scratch.partial, scratch.arrivals, out, s);
        });
}

int tsac_hip_attention_causal(const uint16_t* qkv, size_t heads, size_t head_width, const int* start,
                              const int* length, const int* replay, size_t sequences,
                              size_t max_length, const uint16_t* rotations, float scale,
                              uint16_t* out, void* stream)
{
    return guarded(
        [&]
        {
            attention_prefill(qkv, heads * head_width, heads, head_width, start, length, replay,
                              sequences, max_length, rotations, scale, out, as_stream(stream));
        });
}

int tsac_hip_probe_read(const void* data, size_t bytes, void* stream)
{
    return guarded([&] { probe_read(data, bytes, as_stream(stream)); });
}

int tsac_hip_probe_mfma(size_t workgroups, int iterations, double* ops, void* stream)
{
    return guarded(
        [&]
        {
            require(ops != nullptr, "probe_mfma: ops must not be null");
            *ops = probe_mfma(workgroups, iterations, as_stream(stream));
        });
}
}
