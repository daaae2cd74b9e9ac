// Attention launchers (src/scalar/attention.cpp:12-131 arithmetic).
#pragma once

#include "kernels.hpp"

namespace tsac_hip
{
// Per row: Q, K, V = thirds of qkv[row][3*width]; Q and K rotated by `rotation`
// ([head_width] coefficients shared by every head) when non-null; K and V
// written to keys/values + row*row_stride, Q to query[row][width].
void append_qkv(const uint16_t* qkv, std::size_t rows, std::size_t width, std::size_t head_width,
                const uint16_t* rotation, uint16_t* query, uint16_t* keys, uint16_t* values,
                std::size_t row_stride, hipStream_t stream);

// Device scratch of attention_decode: floats of block records and arrival
// counters (both 0 when one workgroup per (sequence, head) covers the whole
// history and keeps its records in LDS).
// The counters must be zero when a launch starts, and each launch leaves
// them at zero, so scratch cleared once serves every later launch in order.
std::size_t decode_partial_floats(std::size_t sequences, std::size_t heads, std::size_t head_width,
                                  std::size_t time);
std::size_t decode_arrival_counters(std::size_t sequences, std::size_t heads, std::size_t time);
void clear_arrival_counters(unsigned* counters, std::size_t count, hipStream_t stream);

// One query per sequence over `time` cached rows: keys/values of sequence s start
// at keys + s*sequence_stride, row t at + t*width. `replay` forces BF16 value
// rounding for short histories (src/scalar/attention.cpp:128).
void attention_decode(const uint16_t* query, const uint16_t* keys, const uint16_t* values,
                      std::size_t sequence_stride, std::size_t sequences, std::size_t time,
                      std::size_t heads, std::size_t head_width, float scale, bool replay,
                      float* partial, unsigned* arrivals, uint16_t* out, hipStream_t stream);

// Causal attention over whole sequences held in projection output rows
// qkv[row][3*width]. Sequence s occupies rows sequence_start[s] ..
// + sequence_length[s]-1 at positions 0..; its first sequence_replay[s]
// positions use replay rounding. Rotary (temporal stack) uses rotations
// [position][head_width] when non-null. Output rows match the input rows.
void attention_prefill(const uint16_t* qkv, std::size_t width, std::size_t heads,
                       std::size_t head_width, const int* sequence_start,
                       const int* sequence_length, const int* sequence_replay,
                       std::size_t sequences, std::size_t max_length, const uint16_t* rotations,
                       float scale, uint16_t* out, hipStream_t stream);
} // namespace tsac_hip
