// TEST INFRASTRUCTURE ONLY. A C-ABI over the reference's own composition
// classes, compiled where they lie under the reference tree by oracle/Makefile
// into oracle/_ref/libtsacmodel.so, against the adapter_offsets.hpp that the
// reference's own packer (src/weights/pack_main.cpp, built from source by the
// same recipe) generates from seeded original-format model files. Tests use it
// to pin the C oracle's layer sequence, predictor schedule, DAC graphs and
// quantizer; nothing else loads it.
//
// What runs here is the reference's code end to end:
// * ModelDirectory (src/weights/model_directory.cpp) maps the packed files;
// * TransformerModel / DacAnalysisModel / DacSynthesisModel / RvqEncoderModel /
//   RvqDecoderModel (src/models/*.cpp) read them through the generated offsets;
// * CpuTransformer<scalar::Kernels>, DacAnalysis, DacSynthesis, RvqEncoder
//   (instantiated by src/scalar/pipeline.cpp) and RvqDecoder (src/common/rvq.cpp);
// * TransformerPredictor (src/common/transformer.cpp) with
//   pack_normal / unpack_normal (src/format/entropy.cpp).
// The glue below only copies arrays across the C boundary.
#include "common/transformer.hpp"
#include "format/container.hpp"
#include "format/entropy.hpp"
#include "models/contract.hpp"
#include "models/dac_analysis_model.hpp"
#include "models/dac_synthesis_model.hpp"
#include "models/rvq_decoder_model.hpp"
#include "models/rvq_encoder_model.hpp"
#include "models/transformer_model.hpp"
#include "scalar/pipeline.hpp"
#include "tsac/model_directory.hpp"

#include "tsac_oracle.h"

#include <algorithm>
#include <cstring>
#include <optional>
#include <string>
#include <thread>

using namespace tsac;

namespace
{
thread_local std::string last_error;

template <class F> int guarded(F&& f)
{
    try
    {
        f();
        return 0;
    }
    catch (const std::exception& e)
    {
        last_error = e.what();
        return 1;
    }
}

Header header_of(const orc_header& h)
{
    Header r;
    r.method = h.method;
    r.groups = h.groups;
    r.model_channels = h.model_channels;
    r.codebooks = h.codebooks;
    r.frames = h.frames;
    r.batch = h.batch;
    return r;
}

ModelVariant variant_of(unsigned channels)
{
    detail::require(channels == 1 || channels == 2, "model channels must be 1 or 2");
    return channels == 1 ? ModelVariant::mono : ModelVariant::stereo;
}

// The lane executor the reference's CPU analyzers hand to TransformerPredictor
// (src/common/transformer.cpp:70-90): independent lanes prepared concurrently,
// entropy commits serial. Plain threads, `threads` at a time.
class Threads final : public ParallelExecutor
{
public:
    explicit Threads(unsigned n) : n_(std::max(1u, n))
    {
    }
    bool parallel() const override
    {
        return n_ > 1;
    }
    void parallel_for(std::size_t count, const std::function<void(std::size_t)>& task) const override
    {
        for (std::size_t base = 0; base < count; base += n_)
        {
            const auto end = std::min<std::size_t>(count, base + n_);
            std::vector<std::thread> pool;
            std::vector<std::exception_ptr> errors(end - base);
            for (std::size_t i = base; i < end; ++i)
                pool.emplace_back(
                    [&, i]
                    {
                        try
                        {
                            task(i);
                        }
                        catch (...)
                        {
                            errors[i - base] = std::current_exception();
                        }
                    });
            for (auto& t : pool)
                t.join();
            for (auto& e : errors)
                if (e)
                    std::rethrow_exception(e);
        }
    }

private:
    unsigned n_;
};

struct Transformer
{
    TransformerModel model;
    Limits limits;
    scalar::CpuTransformer backend;

    Transformer(const char* dir, unsigned channels, unsigned books, const Limits& l)
        : model(ModelDirectory(dir), variant_of(channels), books), limits(l),
          backend(scalar::CpuTransformer::from_model(model, l))
    {
    }
};

struct Dac
{
    ModelDirectory directory;
    ModelVariant variant;
    unsigned books;
    DacAnalysis<scalar::Kernels> analysis;
    DacSynthesis<scalar::Kernels> synthesis;
    RvqEncoder<scalar::Kernels> encoder;
    RvqDecoder decoder;

    Dac(const char* dir, unsigned channels, unsigned b)
        : directory(dir), variant(variant_of(channels)), books(b),
          analysis(DacAnalysis<scalar::Kernels>::from_model(DacAnalysisModel(directory, variant))),
          synthesis(DacSynthesis<scalar::Kernels>::from_model(DacSynthesisModel(directory, variant))),
          encoder(RvqEncoder<scalar::Kernels>::from_model(
              RvqEncoderModel(directory, variant, RvqInputLayout::input_major, b))),
          decoder(RvqDecoder::from_model(RvqDecoderModel(directory, variant, b)))
    {
    }
};

template <class T> void copy_out(std::span<const T> from, T* to)
{
    if (to)
        std::copy(from.begin(), from.end(), to);
}

// Tensor views hand out their spans only while the view lives.
template <class View, class T> void copy_view(const View& view, T* to)
{
    if (to)
    {
        const auto from = view.values();
        std::copy(from.begin(), from.end(), to);
    }
}
} // namespace

extern "C"
{
const char* refm_last_error()
{
    return last_error.c_str();
}

// ---- the probability model -------------------------------------------------

int refm_transformer_open(const char* dir, unsigned channels, unsigned books, std::size_t cache_bytes,
                          void** handle)
{
    return guarded(
        [&]
        {
            Limits limits;
            if (cache_bytes)
                limits.cache_bytes = cache_bytes;
            *handle = new Transformer(dir, channels, books, limits);
        });
}

void refm_transformer_close(void* handle)
{
    delete static_cast<Transformer*>(handle);
}

// TransformerModel's view of projection `index` (src/models/transformer_model.cpp:48-55):
// int8 values [N][K], fp32 block scales [K/256][N], fp32 bias [N]. Null
// destinations are skipped; `k` and `n` report the shape.
int refm_transformer_projection(void* handle, unsigned index, std::int8_t* values, float* scales,
                                float* bias, std::size_t* k, std::size_t* n)
{
    return guarded(
        [&]
        {
            const auto& m = static_cast<Transformer*>(handle)->model;
            const unsigned per_stack = 4;
            const unsigned stacked = per_stack * (model_contract::temporal_layers + model_contract::codebook_layers);
            LinearWeights w = index == stacked       ? m.temporal_projection()
                              : index == stacked + 1 ? m.codebook_projection()
                              : index == stacked + 2 ? m.output_projection()
                              : [&]
            {
                detail::require(index < stacked, "projection index");
                const bool codebook = index >= per_stack * model_contract::temporal_layers;
                const auto stack = codebook ? TransformerStack::codebook : TransformerStack::temporal;
                const auto local = codebook ? index - per_stack * model_contract::temporal_layers : index;
                const auto layer = local / per_stack;
                switch (local % per_stack)
                {
                case 0:
                    return m.attention_qkv(stack, layer);
                case 1:
                    return m.attention_output(stack, layer);
                case 2:
                    return m.mlp_input(stack, layer);
                default:
                    return m.mlp_output(stack, layer);
                }
            }();
            *k = w.values.shape().axes[0];
            *n = w.values.shape().axes[1];
            copy_view(w.values, values);
            copy_view(w.scales, scales);
            copy_view(w.bias, bias);
        });
}

// Norm `index` in the reference's order: per temporal layer (attention, mlp),
// temporal final, per codebook layer (attention, mlp), codebook final.
int refm_transformer_norm(void* handle, unsigned index, std::uint16_t* gain, std::uint16_t* bias)
{
    return guarded(
        [&]
        {
            const auto& m = static_cast<Transformer*>(handle)->model;
            const unsigned temporal = 2 * model_contract::temporal_layers + 1;
            const bool codebook = index >= temporal;
            const auto stack = codebook ? TransformerStack::codebook : TransformerStack::temporal;
            const auto local = codebook ? index - temporal : index;
            const auto layers = model_contract::layers(stack);
            detail::require(local <= 2 * layers, "norm index");
            const auto w = local == 2 * layers ? m.final_normalization(stack)
                           : local % 2         ? m.mlp_normalization(stack, local / 2)
                                               : m.attention_normalization(stack, local / 2);
            copy_view(w.gain, gain);
            copy_view(w.bias, bias);
        });
}

// positions [books][512], rotary [1024][128], feedback embeddings [books][1024][1024].
int refm_transformer_constants(void* handle, std::uint16_t* positions, std::uint16_t* rotations,
                               std::uint16_t* embeddings)
{
    return guarded(
        [&]
        {
            const auto& m = static_cast<Transformer*>(handle)->model;
            copy_view(m.positions(), positions);
            copy_view(m.rotations(), rotations);
            copy_view(m.feedback_embeddings(), embeddings);
        });
}

int refm_pack_normal(void* handle, const orc_header* header, const std::uint16_t* tokens,
                     std::size_t count, unsigned threads, std::uint8_t* out, std::size_t capacity,
                     std::size_t* written)
{
    return guarded(
        [&]
        {
            auto& t = *static_cast<Transformer*>(handle);
            Threads executor(threads);
            TransformerPredictor predictor(t.backend, t.limits, &executor);
            const auto bytes = pack_normal(header_of(*header), std::span(tokens, count), predictor);
            detail::require(bytes.size() <= capacity, "capacity");
            std::memcpy(out, bytes.data(), bytes.size());
            *written = bytes.size();
        });
}

// pack_normal with an EntropyObserver that records, per symbol in the order the
// observer sees them, before_symbol's position (frame, group, codebook, lane,
// step, token offset) and after_symbol's bit count (src/format/entropy.cpp:86-100).
int refm_pack_normal_observed(void* handle, const orc_header* header, const std::uint16_t* tokens,
                              std::size_t count, std::uint8_t* out, std::size_t capacity, std::size_t* written,
                              std::uint32_t* bits, std::uint64_t* positions)
{
    return guarded(
        [&]
        {
            auto& t = *static_cast<Transformer*>(handle);
            TransformerPredictor predictor(t.backend, t.limits);
            std::size_t before = 0, after = 0;
            EntropyObserver observer{
                [&](const EntropyPosition& p)
                {
                    detail::require(before == after && before < count, "observer order");
                    std::uint64_t* r = positions + 6 * before++;
                    r[0] = p.frame;
                    r[1] = p.group;
                    r[2] = p.codebook;
                    r[3] = p.lane;
                    r[4] = p.step;
                    r[5] = p.token_offset;
                },
                [&](const EntropyPosition& p, std::size_t n)
                {
                    detail::require(after + 1 == before && positions[6 * after + 5] == p.token_offset,
                                    "observer order");
                    bits[after++] = static_cast<std::uint32_t>(n);
                }};
            const auto bytes =
                pack_normal(header_of(*header), std::span(tokens, count), predictor, t.limits, observer);
            detail::require(bytes.size() <= capacity && after == count, "capacity");
            std::memcpy(out, bytes.data(), bytes.size());
            *written = bytes.size();
        });
}

int refm_unpack_normal(void* handle, const std::uint8_t* bytes, std::size_t length, unsigned threads,
                       std::uint16_t* tokens, std::size_t capacity, std::size_t* count)
{
    return guarded(
        [&]
        {
            auto& t = *static_cast<Transformer*>(handle);
            Threads executor(threads);
            TransformerPredictor predictor(t.backend, t.limits, &executor);
            const auto decoded = unpack_normal(ByteView(bytes, length), predictor);
            detail::require(decoded.size() <= capacity, "capacity");
            std::memcpy(tokens, decoded.data(), decoded.size() * 2);
            *count = decoded.size();
        });
}

// Every symbol's distribution, BF16-rounded, at its token offset: the
// predictor driven in entropy order with the known tokens committed.
int refm_distributions(void* handle, const orc_header* header, const std::uint16_t* tokens,
                       std::size_t count, unsigned threads, std::uint16_t* out)
{
    return guarded(
        [&]
        {
            auto& t = *static_cast<Transformer*>(handle);
            Threads executor(threads);
            TransformerPredictor predictor(t.backend, t.limits, &executor);
            auto h = header_of(*header);
            h.method = 1;
            detail::require(count == h.symbol_count(), "token count");
            predictor.reset(h);
            visit_entropy_positions(h,
                                    [&](const EntropyPosition& p)
                                    {
                                        const auto probs = predictor.predict(p);
                                        for (std::size_t i = 0; i < probs.size(); ++i)
                                            out[p.token_offset * probs.size() + i] =
                                                probability_bf16(probs[i]);
                                        predictor.commit(p, tokens[p.token_offset]);
                                    });
        });
}

// ---- the codec ---------------------------------------------------------------

int refm_dac_open(const char* dir, unsigned channels, unsigned books, void** handle)
{
    return guarded(
        [&]
        {
            *handle = new Dac(dir, channels, books);
        });
}

void refm_dac_close(void* handle)
{
    delete static_cast<Dac*>(handle);
}

// DacAnalysis::apply (chunk 0) or apply_chunked (src/common/analysis.tpp:217-257)
// on PCM [groups][samples][channels] -> latent [groups][samples/512][1024].
int refm_dac_analysis(void* handle, const float* pcm, std::size_t samples, std::size_t groups,
                      std::size_t chunk, float* latent)
{
    return guarded(
        [&]
        {
            const auto& d = *static_cast<Dac*>(handle);
            const SignalShape shape{d.analysis.channels(), samples, groups};
            const std::span input(pcm, shape.elements());
            const auto out = chunk ? d.analysis.apply_chunked(input, shape, chunk) : d.analysis.apply(input, shape);
            copy_out<float>(out.values, latent);
        });
}

// DacSynthesis::apply (chunk 0) or apply_chunked on latent [groups][frames][1024]
// -> PCM [groups][frames*512][channels] (no tanh, no PCM rounding).
int refm_dac_synthesis(void* handle, const float* latent, std::size_t frames, std::size_t groups,
                       std::size_t chunk, float* pcm)
{
    return guarded(
        [&]
        {
            const auto& d = *static_cast<Dac*>(handle);
            const SignalShape shape{1024, frames, groups};
            const std::span input(latent, shape.elements());
            const auto out = chunk ? d.synthesis.apply_chunked(input, shape, chunk) : d.synthesis.apply(input, shape);
            copy_out<float>(out.values, pcm);
        });
}

// RvqEncoder::encode: latent [groups][frames][1024] -> tokens [frame][group][book].
int refm_rvq_encode(void* handle, const orc_header* header, const float* latent, std::uint16_t* tokens)
{
    return guarded(
        [&]
        {
            const auto& d = *static_cast<Dac*>(handle);
            const auto h = header_of(*header);
            const auto out = d.encoder.encode(h, std::span(latent, h.frames * h.groups * 1024));
            copy_out<std::uint16_t>(out, tokens);
        });
}

// RvqDecoder::decode: tokens [frame][group][book] (a normal header carries
// their CRC) -> latent [groups][frames][1024].
int refm_rvq_decode(void* handle, const orc_header* header, const std::uint16_t* tokens, float* latent)
{
    return guarded(
        [&]
        {
            const auto& d = *static_cast<Dac*>(handle);
            auto h = header_of(*header);
            const std::span t(tokens, h.symbol_count());
            if (h.method == 1)
                h.token_crc = token_crc32(t);
            const auto out = d.decoder.decode(h, t);
            copy_out<float>(out, latent);
        });
}

// The DAC model's view of convolution `index` of one graph: payload bytes as
// packed (int8 plane and BF16 scale plane, or float32), weight-norm gains per
// stored column and biases.
int refm_dac_convolution(void* handle, int synthesis, unsigned index, std::uint8_t* payload,
                         std::size_t* payload_bytes, std::size_t* data_plane_bytes, float* gain,
                         std::size_t* gains, float* bias, std::size_t* biases)
{
    return guarded(
        [&]
        {
            const auto& d = *static_cast<Dac*>(handle);
            const auto convolution = [&]() -> ConvolutionWeights
            {
                if (synthesis)
                {
                    const DacSynthesisModel m(d.directory, d.variant);
                    if (index == 0)
                        return m.entry_convolution();
                    if (index == 29)
                        return m.exit_convolution();
                    const auto stage = (index - 1) / 7, within = (index - 1) % 7;
                    if (within == 0)
                        return m.resample_convolution(stage);
                    return m.residual_convolution(stage, (within - 1) / 2,
                                                  (within - 1) % 2 ? ResidualConvolution::pointwise
                                                                   : ResidualConvolution::dilated);
                }
                const DacAnalysisModel m(d.directory, d.variant);
                if (index == 0)
                    return m.entry_convolution();
                if (index == 29)
                    return m.exit_convolution();
                const auto stage = (index - 1) / 7, within = (index - 1) % 7;
                if (within == 6)
                    return m.resample_convolution(stage);
                return m.residual_convolution(stage, within / 2,
                                              within % 2 ? ResidualConvolution::pointwise
                                                         : ResidualConvolution::dilated);
            }();
            const auto bytes = convolution.values.payload();
            *payload_bytes = bytes.size();
            *data_plane_bytes = convolution.values.data_plane_bytes();
            *gains = convolution.gain.size();
            *biases = convolution.bias.size();
            copy_out(bytes, payload);
            copy_view(convolution.gain, gain);
            copy_view(convolution.bias, bias);
        });
}

// Snake alpha `index` of one graph in graph order (the contract's
// residual_activation / resample_activation / final activation numbering).
int refm_dac_activation(void* handle, int synthesis, unsigned index, float* alpha, std::size_t* count)
{
    return guarded(
        [&]
        {
            const auto& d = *static_cast<Dac*>(handle);
            const auto stage = index / 7, within = index % 7;
            const auto which = [](unsigned w)
            {
                return w % 2 ? ResidualActivation::before_pointwise : ResidualActivation::before_dilated;
            };
            const auto view = [&]() -> TensorView<float>
            {
                if (synthesis)
                {
                    const DacSynthesisModel m(d.directory, d.variant);
                    if (index == 28)
                        return m.final_activation();
                    if (within == 0)
                        return m.resample_activation(stage);
                    return m.residual_activation(stage, (within - 1) / 2, which(within - 1));
                }
                const DacAnalysisModel m(d.directory, d.variant);
                if (index == 28)
                    return m.final_activation();
                if (within == 6)
                    return m.resample_activation(stage);
                return m.residual_activation(stage, within / 2, which(within));
            }();
            *count = view.size();
            copy_view(view, alpha);
        });
}

// The RVQ models' prepared tensors of one book: codebook [1024][8], search
// vectors [1024][8], input projection (input-major, as the packer folds it),
// input bias [8], output projection [8][1024] folded, output bias [1024].
int refm_rvq_tensors(void* handle, unsigned book, float* codebook, float* search, float* input_weights,
                     float* input_bias, float* output_weights, float* output_bias)
{
    return guarded(
        [&]
        {
            const auto& d = *static_cast<Dac*>(handle);
            const RvqEncoderModel e(d.directory, d.variant, RvqInputLayout::input_major, d.books);
            copy_view(e.codebook(book), codebook);
            copy_view(e.search_vectors(book), search);
            const auto in = e.input_projection(book);
            copy_view(in.values, input_weights);
            copy_view(in.bias, input_bias);
            const auto out = e.output_projection(book);
            copy_view(out.values, output_weights);
            copy_view(out.bias, output_bias);
        });
}
}
