// HipTransformer: the reference-side drop-in for MetalTransformer
// (src/metal/transformer.hpp:13-39), built inside the skimmilk/tsac-metal tree
// (as src/hip/transformer.{hpp,cpp}) against its headers, linking
// libtsac_hip.so through include/tsac_hip.h. Same operations, ownership,
// error type and bitstream; MetalAnalyzer's two call sites
// (src/metal/audio_analyzer.cpp:157-163,181-187) switch to this class.
#pragma once
#include "format/entropy.hpp"
#include "models/transformer_model.hpp"

#include <memory>
#include <span>
#include <vector>

struct tsac_hip_model;
struct tsac_hip_session;

namespace tsac
{
// One probability-model session on the current HIP device. Sessions made by
// new_session() share the immutable device model and own their caches, scratch
// and stream. Calls are synchronous; observers run on the calling thread in
// entropy order after the call's GPU work completes. A session stays usable
// after a failure; concurrent calls need separate sessions.
class HipTransformer final
{
public:
    static HipTransformer from_model(TransformerModel model, const Limits& limits = {});
    ~HipTransformer();
    HipTransformer(HipTransformer&&) noexcept;
    HipTransformer& operator=(HipTransformer&&) noexcept;
    HipTransformer(const HipTransformer&) = delete;
    HipTransformer& operator=(const HipTransformer&) = delete;

    HipTransformer new_session() const;
    // Releases caches, scratch and graph state; the device weights stay.
    void clear_session();

    Bytes encode(Header header, std::span<const std::uint16_t> tokens,
                 const EntropyObserver& observer = {});
    std::vector<std::uint16_t> decode(ByteView stream, const EntropyObserver& observer = {});

private:
    HipTransformer() = default;
    std::shared_ptr<tsac_hip_model> model_;
    std::unique_ptr<tsac_hip_session, void (*)(tsac_hip_session*)> session_{nullptr, nullptr};
};
} // namespace tsac
