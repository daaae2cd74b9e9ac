// Embedding and categorical-mass launchers.
#pragma once

#include "kernels.hpp"

namespace tsac_hip
{
// out[r] = previous ? bf16(previous[r] + E[book][tokens[r*stride]]) : E[book][tokens[r*stride]].
void embed_accumulate(const uint16_t* embeddings, std::size_t alphabet, std::size_t latent,
                      const uint16_t* tokens, std::size_t token_stride, std::size_t book,
                      std::size_t rows, const uint16_t* previous, uint16_t* out, hipStream_t stream);
// out[r] = ordered BF16 sum of E[b][tokens[r][b]] over b < books.
void embed_sum(const uint16_t* embeddings, std::size_t alphabet, std::size_t latent,
               const uint16_t* tokens, std::size_t books, std::size_t rows, uint16_t* out,
               hipStream_t stream);
// out[s][b] = prefix sum of books 0..b-1 of tokens[s] (zero row for b = 0).
void embed_prefixes(const uint16_t* embeddings, std::size_t alphabet, std::size_t latent,
                    const uint16_t* tokens, std::size_t books, std::size_t steps, uint16_t* out,
                    hipStream_t stream);
// dst[r*stride + offset] = src[r].
void scatter_rows(const uint16_t* src, std::size_t rows, std::size_t width, std::size_t stride,
                  std::size_t offset, uint16_t* dst, hipStream_t stream);
// dst[dst_index[r]] = src[src_index[r]] for r < rows.
void copy_rows(const uint16_t* src, const int* src_index, uint16_t* dst, const int* dst_index,
               std::size_t rows, std::size_t width, hipStream_t stream);
// splits[r][level] = Q15 split of bisection level `level` along symbols[r] (10 levels, stride 16).
void categorical_paths(const uint16_t* probs, std::size_t rows, std::size_t alphabet,
                       const uint16_t* symbols, uint16_t* splits, uint32_t* error, hipStream_t stream);
// nodes[r][1..1023] = heap-ordered subtree masses; nodes[r][0] = 1 if valid.
void categorical_trees(const uint16_t* probs, std::size_t rows, float* nodes, hipStream_t stream);
} // namespace tsac_hip
