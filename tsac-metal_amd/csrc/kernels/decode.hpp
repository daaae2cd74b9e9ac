// Decode-side (autoregressive) kernels: every projection of a step is one
// launch that quantises its input itself (optionally through LayerNorm or the
// feedback-embedding sums) and applies its own epilogue (residual, GELU, or
// rotary + KV-cache append); attention of a step is one launch; sampling
// (softmax, categorical masses, range decoding) is one launch. Positions and the
// step index are read from device memory so a whole step can be replayed.
#pragma once

#include "kernels.hpp"

namespace tsac_hip
{
enum class Input : int
{
    bf16,             // x rows as they are
    layer_norm,       // LayerNorm(x; gain, beta)
    embed_sum,        // sum over `books` of E[b][tokens[m*token_stride + b]]
    embed_accumulate, // (x ? x + : ) E[book][tokens[m*token_stride + token_offset]]
};

enum class Output : int
{
    plain,    // y = bf16(sum + bias)
    residual, // y = bf16(residual + bf16(sum + bias)); residual_stride 0 broadcasts one row
    gelu,     // y = gelu(bf16(sum + bias))
    qkv,      // Q (rotated) -> query, K (rotated) -> keys, V -> values at the cache position
};

struct FusedLinear
{
    DeviceLinear w;
    int M = 0;
    Input input = Input::bf16;
    Output output = Output::plain;
    // input
    const uint16_t* x = nullptr;
    int x_stride = 0;
    const uint16_t* gain = nullptr;
    const uint16_t* beta = nullptr;
    const uint16_t* embeddings = nullptr;
    int alphabet = 1024, books = 1, book = 0;
    const uint16_t* tokens = nullptr;
    int token_stride = 0, token_offset = 0;
    uint16_t* prefix_out = nullptr; // embed_accumulate: the updated prefix rows
    uint32_t* error = nullptr;
    // output
    uint16_t* y = nullptr;
    int y_stride = 0;
    const uint16_t* residual = nullptr;
    int residual_stride = 0;
    uint16_t* query = nullptr;
    uint16_t* keys = nullptr;   // this layer's cache, row 0
    uint16_t* values = nullptr; // this layer's cache, row 0
    long long lane_stride = 0;  // elements between consecutive lanes' caches
    int width = 0, head_width = 0;
    const uint16_t* rotations = nullptr; // [position][head_width] or null
    const int* position = nullptr;       // device position; fixed_position if null
    int fixed_position = 0;
};

void fused_linear(const FusedLinear& args, hipStream_t stream);

// One query per lane over positions 0..position of that lane's cache, one launch.
void attention_step(const uint16_t* query, const uint16_t* keys, const uint16_t* values,
                    long long lane_stride, std::size_t lanes, std::size_t width,
                    std::size_t heads, std::size_t head_width, float scale, const int* position,
                    int fixed_position, std::size_t max_time, bool replay, uint16_t* out,
                    hipStream_t stream);

// out[r] = bf16(LayerNorm(x[r]) + add_row) (add_row may be null).
void layer_norm_add(const uint16_t* x, std::size_t rows, std::size_t width, const uint16_t* gain,
                    const uint16_t* bias, const uint16_t* add_row, uint16_t* out, hipStream_t stream);

// Range-decoder state resident on the device.
struct DecoderState
{
    uint32_t range, code;
    unsigned long long offset;
    uint32_t failed;
    uint32_t pad;
};

struct Sample
{
    const uint16_t* logits = nullptr; // [lanes][1024]
    int lanes = 0;
    int book = 0, books = 1;
    uint16_t* current = nullptr;      // [lanes][books] tokens of the current frame
    uint16_t* tokens = nullptr;       // [symbols] stream-order destination
    const int* row_base = nullptr;    // per lane: token offset of its first frame, book 0
    const int* step = nullptr;        // device step counter; fixed_step if null
    int fixed_step = 0;
    int step_stride = 0;              // token offset between consecutive frames of a lane
    const uint16_t* known = nullptr;  // teacher forcing: take tokens from here
    uint16_t* distributions = nullptr; // optional [symbols][1024] BF16 output
    uint16_t* splits = nullptr;       // known tokens, optional: [symbols][16], the ten Q15 splits of each
    DecoderState* state = nullptr;    // range decoder (null with known tokens)
    const uint8_t* payload = nullptr;
    unsigned long long payload_bytes = 0;
    uint32_t* error = nullptr;
};

// Softmax -> categorical masses -> range decode (or teacher forcing) for every
// lane in stream order, one launch.
void sample_step(const Sample& args, hipStream_t stream);

// dst[i][b] = tokens[row_base[i] + frame * step_stride + b] for b < books.
void gather_frame(const uint16_t* tokens, const int* row_base, int frame, int step_stride,
                  int books, int lanes, uint16_t* dst, hipStream_t stream);
// counters[0] = position, counters[1] = step (one thread).
void set_counters(int* counters, int position, int step, hipStream_t stream);
// ++counters[0], ++counters[1] (one thread).
void advance_counters(int* counters, hipStream_t stream);
} // namespace tsac_hip
