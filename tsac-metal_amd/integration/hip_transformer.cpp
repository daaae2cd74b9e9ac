// HipTransformer over the C ABI of libtsac_hip.so. See hip_transformer.hpp.
#include "hip_transformer.hpp"

#include "models/config.hpp"
#include "models/contract.hpp"
#include "tsac_hip.h"

#include <exception>

namespace tsac
{
namespace
{
void check(int status)
{
    if (status != TSAC_HIP_OK)
    {
        throw Error(tsac_hip_last_error());
    }
}

tsac_hip_linear linear(const LinearWeights& w)
{
    return {w.values.data(), w.scales.data(), w.bias.data()};
}

tsac_hip_header header_of(const Header& h)
{
    return {h.method, h.groups, h.model_channels, h.codebooks, h.frames, h.batch};
}

EntropyPosition position_of(const tsac_hip_position* p)
{
    return {p->frame, p->group, p->codebook, p->lane, p->step, p->token_offset};
}

// The EntropyObserver behind the ABI's C callbacks. An exception from the
// observer is kept, the call is stopped (nonzero return), and the exception is
// rethrown to the caller once the ABI call has returned.
struct ObserverBridge
{
    const EntropyObserver& observer;
    std::exception_ptr failure;

    static int before(void* context, const tsac_hip_position* p)
    {
        auto* self = static_cast<ObserverBridge*>(context);
        try
        {
            self->observer.before_symbol(position_of(p));
            return 0;
        }
        catch (...)
        {
            self->failure = std::current_exception();
            return 1;
        }
    }

    static int after(void* context, const tsac_hip_position* p, std::uint64_t bits)
    {
        auto* self = static_cast<ObserverBridge*>(context);
        try
        {
            self->observer.after_symbol(position_of(p), static_cast<std::size_t>(bits));
            return 0;
        }
        catch (...)
        {
            self->failure = std::current_exception();
            return 1;
        }
    }

    tsac_hip_observer abi()
    {
        return {this, observer.before_symbol ? &before : nullptr, observer.after_symbol ? &after : nullptr};
    }

    void finish(int status)
    {
        if (failure)
        {
            std::rethrow_exception(failure);
        }
        check(status);
    }
};
} // namespace

HipTransformer::~HipTransformer() = default;
HipTransformer::HipTransformer(HipTransformer&&) noexcept = default;
HipTransformer& HipTransformer::operator=(HipTransformer&&) noexcept = default;

HipTransformer HipTransformer::from_model(TransformerModel model, const Limits& limits)
{
    using model_contract::layers;
    // Projection order of src/models/contract.cpp:88-110,195-199; norm order of
    // contract.cpp:201-211. The views stay alive until the device copy is made.
    std::vector<LinearWeights> views;
    std::vector<NormalizationWeights> norms;
    for (const auto stack : {TransformerStack::temporal, TransformerStack::codebook})
    {
        for (unsigned l = 0; l < layers(stack); ++l)
        {
            views.push_back(model.attention_qkv(stack, l));
            views.push_back(model.attention_output(stack, l));
            views.push_back(model.mlp_input(stack, l));
            views.push_back(model.mlp_output(stack, l));
        }
    }
    views.push_back(model.temporal_projection());
    views.push_back(model.codebook_projection());
    views.push_back(model.output_projection());
    for (const auto stack : {TransformerStack::temporal, TransformerStack::codebook})
    {
        for (unsigned l = 0; l < layers(stack); ++l)
        {
            norms.push_back(model.attention_normalization(stack, l));
            norms.push_back(model.mlp_normalization(stack, l));
        }
        norms.push_back(model.final_normalization(stack));
    }
    std::vector<tsac_hip_linear> projections;
    for (const auto& w : views)
    {
        projections.push_back(linear(w));
    }
    std::vector<const std::uint16_t*> gain, bias;
    for (const auto& n : norms)
    {
        gain.push_back(n.gain.data());
        bias.push_back(n.bias.data());
    }
    const auto positions = model.positions();
    const auto rotations = model.rotations();
    const auto embeddings = model.feedback_embeddings();
    const TransformerConfig config{model.codebooks()};
    tsac_hip_model_desc desc{};
    desc.geometry = {config.width,
                     config.heads,
                     config.head_width,
                     4 * config.width,
                     config.temporal_layers,
                     config.codebook_layers,
                     model_contract::latent_width,
                     model_contract::alphabet,
                     model.codebooks(),
                     model_contract::channels(model.variant()),
                     config.context,
                     0.0883883461356163f}; // 1/sqrt(128) as fp32 (src/common/cpu_transformer.tpp:164)
    desc.projections = projections.data();
    desc.norm_gain = gain.data();
    desc.norm_bias = bias.data();
    desc.positions = positions.data();
    desc.rotations = rotations.data();
    desc.embeddings = embeddings.data();
    const tsac_hip_limits l{limits.file_bytes, limits.symbols, limits.pcm_bytes, limits.cache_bytes,
                            limits.tensor_elements};
    tsac_hip_model* m = nullptr;
    check(tsac_hip_model_create(&desc, &l, &m)); // copies and re-lays out; the mappings may go
    HipTransformer t;
    t.model_.reset(m, tsac_hip_model_destroy);
    return t.new_session();
}

HipTransformer HipTransformer::new_session() const
{
    HipTransformer t;
    t.model_ = model_;
    tsac_hip_session* s = nullptr;
    check(tsac_hip_session_create(model_.get(), &s));
    t.session_ = {s, tsac_hip_session_destroy};
    return t;
}

void HipTransformer::clear_session()
{
    check(tsac_hip_session_clear(session_.get()));
}

Bytes HipTransformer::encode(Header h, std::span<const std::uint16_t> tokens, const EntropyObserver& observer)
{
    const tsac_hip_header header = header_of(h);
    ObserverBridge bridge{observer, nullptr};
    const tsac_hip_observer abi = bridge.abi();
    std::uint8_t* bytes = nullptr;
    std::size_t length = 0;
    bridge.finish(tsac_hip_encode_observed(session_.get(), &header, tokens.data(), tokens.size(), &abi, &bytes,
                                           &length));
    Bytes result(bytes, bytes + length);
    tsac_hip_free(bytes);
    return result;
}

std::vector<std::uint16_t> HipTransformer::decode(ByteView stream, const EntropyObserver& observer)
{
    ObserverBridge bridge{observer, nullptr};
    const tsac_hip_observer abi = bridge.abi();
    std::uint16_t* tokens = nullptr;
    std::size_t count = 0;
    bridge.finish(tsac_hip_decode_observed(session_.get(), stream.data(), stream.size(), &abi, &tokens, &count));
    std::vector<std::uint16_t> result(tokens, tokens + count);
    tsac_hip_free(tokens);
    return result;
}
} // namespace tsac
