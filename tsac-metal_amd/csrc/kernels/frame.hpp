// One decode frame step (temporal stack, then every codebook with its range
// decoding) in a single persistent launch.
//
// The step's ~240 dependent operations (projections, attention, sampling) run
// as jobs of a fixed set of co-resident workgroups. Activations pass between
// jobs through "exchange words": 8-byte words holding two BF16 values (or a
// token) in the low half and the step's epoch in the high half, written and
// polled with relaxed device-scope atomics. A consumer waits only for the words
// it reads, so no device-wide barrier (and none of its cache write-back and
// invalidation) is needed, and every workgroup issues its next job's weight
// loads before it waits for that job's inputs.
//
// Jobs take the lanes one at a time in lane order, the order in which the range
// decoder produces their tokens, so a lane's next codebook starts as soon as its
// own token is known. A projection normalises and quantises each lane's input
// with all of its waves. When the device holds the extra workgroups, each
// codebook layer's attention (at most one key per book) is computed inside its
// out-projection tiles, one workgroup per (tile, lane), and the qkv/up/down
// tiles alternate between two sets of workgroups from layer to layer.
//
// One launch runs several consecutive steps (epochs advance by one per step),
// so a lane's next step starts as soon as its own tokens are drawn, with no
// launch in between. Key/value rows of earlier steps come from the temporal
// cache: rows stored during the launch with device-coherent stores and read
// back with device-coherent loads; the current step's rows and the whole
// codebook stack come from exchange words, and so do the previous step's
// tokens. Every wait is bounded: a stalled wait raises the abort word, after
// which all waits return at once and the launch ends.
#pragma once

#include "decode.hpp"

#include <vector>

namespace tsac_hip
{
// The model as frame_job_table reads it: host arrays of device pointers.
struct FrameModel
{
    const DeviceLinear* linears = nullptr; // reference projection order
    const uint16_t* const* gain = nullptr; // reference norm order
    const uint16_t* const* bias = nullptr;
    const uint16_t* positions = nullptr;  // [books][width]
    const uint16_t* rotations = nullptr;  // [context][head_width]
    const uint16_t* embeddings = nullptr; // [books][alphabet][latent]
};

struct FrameArgs
{
    FrameModel model;
    int lanes = 0, books = 0, temporal_layers = 0, codebook_layers = 0;
    int width = 0, heads = 0, head_width = 0, ffn = 0, latent = 0, alphabet = 0;
    float scale = 0.0f;
    // temporal cache: lane l, layer k, position p at l*lane_stride + (k*extent + p)*width
    uint16_t* keys = nullptr;
    uint16_t* values = nullptr;
    long long lane_stride = 0;
    int extent = 0;
    int position = 0; // context position of the launch's first step
    int step = 0;     // frame step index of the launch's first step
    int steps = 1;    // consecutive steps of the launch (position, step and epoch advance by one)
    // tokens
    uint16_t* current = nullptr; // [lanes][books]: previous frame in, this frame out
    const int* row_base = nullptr;
    int step_stride = 0;
    uint16_t* tokens = nullptr;
    const uint16_t* known = nullptr;
    uint16_t* distributions = nullptr;
    uint16_t* splits = nullptr; // known tokens, optional: [symbols][16], the ten Q15 splits of each
    DecoderState* state = nullptr;
    const uint8_t* payload = nullptr;
    unsigned long long payload_bytes = 0;
    uint32_t* error = nullptr;
    // exchange
    unsigned long long* words = nullptr; // frame_exchange_words() words, zero before the first step
    uint32_t epoch = 0;                  // first step's; nonzero, different for every step over the same words
    unsigned* abort = nullptr;           // zero before the first step; nonzero after a stalled wait
    const void* jobs = nullptr;          // device copy of frame_job_table(*this), unchanged during a launch
    bool plain_launch = false;           // launch without the cooperative co-residency guarantee
};

// How frame_step launched the kernel.
enum class FrameLaunch
{
    cooperative = 0, // co-residency guaranteed by the runtime
    requested_plain = 1, // plain launch asked for through FrameArgs::plain_launch
    fallback_plain = 2, // plain launch: another process holds the cooperative-launch resources
};

// Geometries the frame kernel is instantiated for, at 1..8 lanes.
bool frame_supported(int width, int heads, int head_width, int ffn, int latent, int alphabet, int lanes);
// Exchange words one step needs.
std::size_t frame_exchange_words(int width, int ffn, int latent, int alphabet, int books, int temporal_layers,
                                 int codebook_layers);
// Every job's descriptor (weights, norms, exchange-word ranges, caches) for the
// launches of one pass, built on the host from the pointers in `args` (all but
// position, step, steps, lanes and epoch, which the launches pass themselves); the
// launches read it from device memory through FrameArgs::jobs.
std::vector<uint8_t> frame_job_table(const FrameArgs& args);
FrameLaunch frame_step(const FrameArgs& args, hipStream_t stream);
} // namespace tsac_hip
