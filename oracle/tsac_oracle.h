/*
 * TEST INFRASTRUCTURE ONLY. This is the CPU oracle for the TSAC probability
 * model: a plain-C restatement of the reference's scalar arithmetic, used by
 * tests/ as the checker and by bench.py as the reported CPU baseline. The
 * product library (libtsac_hip.so) never links, loads or calls it.
 *
 * Every function cites the reference file:line it restates (paths relative to
 * the skimmilk/tsac-metal tree). All activations are BF16 bit patterns held in
 * uint16_t; floats are IEEE binary32 with round-to-nearest-even.
 *
 * Pinning (what checks each function against something other than itself):
 *   orc_bf16/orc_float     exhaustive KAT of tests/numeric.cpp:172-188
 *   orc_exp                brute force over every float vs the compiled reference
 *   orc_probability_sum    compiled reference on random spans; closed form
 *   orc_bf8l               KAT tests/scalar.cpp:44-53; compiled reference
 *   orc_qlinear            compiled reference linear_column (R4 layout); brute
 *                          force int64 dot on tiny shapes
 *   orc_layer_norm/softmax/rotary/gelu/add  compiled reference (random + edge bits)
 *   orc_attention          checksum 15737425383056432415 (tests/attention.cpp:103)
 *                          and the compiled reference
 *   range coder/categorical/container  literal streams of tests/sanitation.cpp,
 *                          round trips, compiled reference pack_normal
 *   composition (orc_model_*, predictor)  compiled reference TransformerPredictor
 *                          + pack_normal driving a backend assembled from the
 *                          compiled reference kernels (oracle/ref_shim.cpp)
 */
#ifndef TSAC_ORACLE_H
#define TSAC_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status ---------------------------------------------------------------- */
/* 0 = success, nonzero = failure; orc_last_error() names the failed requirement. */
const char* orc_last_error(void);

/* ---- numerics (src/common/numeric/, src/format/categorical.cpp) ------ */
uint16_t orc_bf16(float value);
float orc_float(uint16_t value);
float orc_flush(float x);
float orc_add(float x, float y);
float orc_subtract(float x, float y);
float orc_multiply(float x, float y);
float orc_divide(float x, float y);
float orc_exp(float z);
float orc_probability_sum(const float* values, size_t count);
uint16_t orc_conditional_q15(float left_mass, float mass);
void orc_exp_batch(const float* z, size_t count, float* out);
void orc_gelu_batch(const uint16_t* x, size_t count, uint16_t* out);
void orc_bf16_batch(const float* x, size_t count, uint16_t* out);

/* ---- kernels --------------------------------------------------------------- */
int orc_bf8l(const float* values, size_t count, int8_t* quantized, uint16_t* scales);
/* y[m][n] for canonical weights w[N][K] (K fastest), block scales [K/256][N]. */
int orc_qlinear(const int8_t* weights, const float* weight_scales, const float* bias, size_t K,
                size_t N, const uint16_t* x, size_t M, uint16_t* y);
int orc_layer_norm(const uint16_t* x, const uint16_t* gain, const uint16_t* bias, size_t n,
                   uint16_t* out);
uint16_t orc_gelu(uint16_t value);
uint16_t orc_add_bf16(uint16_t left, uint16_t right);
int orc_rotary(const uint16_t* values, const uint16_t* coefficients, size_t n, uint16_t* out);
int orc_softmax(const uint16_t* x, size_t n, uint16_t* out);
/* One query over `time` row-major keys/values [time][heads*head_width]. */
int orc_attention(const uint16_t* query, const uint16_t* keys, const uint16_t* values,
                  size_t time, size_t heads, size_t head_width, float scale, int prefill,
                  uint16_t* out);

/* ---- range coder / categorical / container (src/format/) ----------------- */
typedef struct orc_header
{
    uint8_t method, groups, model_channels, codebooks;
    uint64_t frames;
    uint16_t batch;
} orc_header;

uint32_t orc_token_crc32(const uint16_t* tokens, size_t count);
/* Encodes `count` (symbol, probabilities[1024]) pairs into one range stream. */
int orc_range_roundtrip_encode(const float* probabilities, const uint16_t* symbols, size_t count,
                               size_t alphabet, uint8_t* out, size_t capacity, size_t* written);
int orc_range_roundtrip_decode(const float* probabilities, size_t count, size_t alphabet,
                               const uint8_t* bytes, size_t length, uint16_t* symbols);
int orc_parse_header(const uint8_t* bytes, size_t length, orc_header* header,
                     size_t* payload_offset, size_t* payload_bytes, uint32_t* crc);

/* ---- model composition ----------------------------------------------------- */
typedef struct orc_geometry
{
    uint32_t width, heads, head_width, ffn;
    uint32_t temporal_layers, codebook_layers;
    uint32_t latent, alphabet, books, channels, context;
    float attention_scale;
} orc_geometry;

typedef struct orc_linear
{
    const int8_t* values; /* [N][K] */
    const float* scales;  /* [K/256][N] */
    const float* bias;    /* [N] */
} orc_linear;

/* Projection order: temporal 4L+{qkv,attn_out,mlp_in,mlp_out}, codebook
 * 4*Lt+4L+{...}, then temporal cb_proj, codebook cb_proj, proj_f
 * (src/models/contract.cpp:88-110,195-199). Norm order: temporal 2L+{ln_1,ln_2},
 * 2Lt = ln_f, codebook 2Lt+1+2L+{...}, 2Lt+1+2Lc = ln_f (contract.cpp:201-211). */
typedef struct orc_model_desc
{
    orc_geometry geometry;
    const orc_linear* projections;
    const uint16_t* const* norm_gain;
    const uint16_t* const* norm_bias;
    const uint16_t* positions;  /* [books][width] */
    const uint16_t* rotations;  /* [context][head_width] */
    const uint16_t* embeddings; /* [books][alphabet][latent] */
} orc_model_desc;

typedef struct orc_model orc_model;
int orc_model_create(const orc_model_desc* desc, orc_model** out);
void orc_model_destroy(orc_model* model);

/* TransformerBackend operations (src/common/transformer.hpp:14-43). */
int orc_backend_reset(orc_model* model, const orc_header* header, size_t lanes);
int orc_backend_reset_temporal(orc_model* model, size_t lane);
int orc_backend_temporal_step(orc_model* model, size_t lane, size_t position,
                              const uint16_t* feedback, size_t count, int replay);
int orc_backend_reset_codebook(orc_model* model, size_t lane);
/* Writes the BF16 distribution (alphabet entries). */
int orc_backend_codebook_step(orc_model* model, size_t lane, size_t book, const uint16_t* prefix,
                              size_t count, uint16_t* distribution);

/* Predictor-driven whole-stream operations (src/format/entropy.cpp:57-155 with
 * src/common/transformer.cpp:59-166). `threads` > 1 prepares ready lanes
 * concurrently, like the reference's executor. */
int orc_pack_normal(orc_model* model, const orc_header* header, const uint16_t* tokens,
                    size_t count, unsigned threads, uint8_t** out, size_t* length);
/* pack_normal with an EntropyObserver recording, per symbol in stream order,
 * after_symbol's bit count (bits[count], src/format/entropy.cpp:86-100) and the
 * position {frame, group, codebook, lane, step, token_offset} (positions[6*count]);
 * either may be NULL. */
int orc_pack_normal_observed(orc_model* model, const orc_header* header, const uint16_t* tokens,
                             size_t count, unsigned threads, uint8_t** out, size_t* length,
                             uint32_t* bits, uint64_t* positions);
int orc_unpack_normal(orc_model* model, const uint8_t* bytes, size_t length, unsigned threads,
                      uint16_t** tokens, size_t* count);
/* Teacher-forced distributions in token order: out[token_offset][alphabet] BF16. */
int orc_distributions(orc_model* model, const orc_header* header, const uint16_t* tokens,
                      size_t count, unsigned threads, uint16_t* out);
/* Same walk, stopping after `max_symbols` symbols in entropy order (for bounded timing). */
int orc_distributions_prefix(orc_model* model, const orc_header* header, const uint16_t* tokens,
                             size_t count, unsigned threads, size_t max_symbols, uint16_t* out);
void orc_free(void* pointer);

/* ---- DAC analysis/synthesis and RVQ (oracle/dac.c) --------------------------- */
typedef struct orc_conv
{
    size_t in, out, kernel, stride, padding, dilation;
    int transposed;
} orc_conv;

/* A DAC graph: 30 convolutions (prepared fp32 weights in the stored layout,
 * fp32 bias) and 29 Snake alphas, indexed as src/models/contract.cpp numbers them. */
typedef struct orc_dac
{
    int synthesis;
    unsigned channels;
    const float* weights[30];
    const float* bias[30];
    const float* alpha[29];
} orc_dac;

/* Prepared RVQ tensors per book: codebook [1024][8], normalised search vectors
 * [1024][8], input projection [8][1024] (output-major, ordinary conv layout) +
 * bias [8], output projection [1024][8] + bias [1024]. */
typedef struct orc_rvq
{
    unsigned books;
    const float* codebook[12];
    const float* search[12];
    const float* input_weights[12];
    const float* input_bias[12];
    const float* output_weights[12];
    const float* output_bias[12];
} orc_rvq;

float orc_dac_sine_squared(float phase);
int orc_snake(const float* x, size_t count, size_t channels, const float* alpha, float* out);
int orc_fold_dac_weight_norm(const float* v, const float* g, size_t fan_in, size_t columns, float* out);
int orc_expand_bf8(const int8_t* data, const uint16_t* scales, size_t rows, size_t cols, size_t outer, float* out);
size_t orc_conv_output_frames(const orc_conv* c, size_t frames);
int orc_conv1d(const orc_conv* c, const float* w, const float* bias, const float* x, size_t frames, size_t groups,
               float* y, unsigned threads);
int orc_dac_conv_config(int synthesis, unsigned channels, unsigned index, orc_conv* c);
size_t orc_dac_activation_width(int synthesis, unsigned index);
int orc_dac_apply(const orc_dac* m, const float* in, size_t frames, float* out, size_t* out_frames, unsigned threads);
void orc_normalize_search(const float* input, float* output);
uint16_t orc_nearest_rvq(const float* input, const float* vectors);
void orc_project_codebook(uint16_t index, const float* codebook, const float* weights, const float* bias, float* out);
int orc_rvq_encode(const orc_rvq* q, const float* latent, size_t frames, uint16_t* tokens);
int orc_rvq_decode(const orc_rvq* q, const uint16_t* tokens, size_t frames, float* latent);
int orc_analyze_audio(const orc_dac* analysis, const orc_rvq* q, const float* pcm, size_t frames, size_t groups,
                      size_t chunk, unsigned threads, uint16_t* tokens);
int orc_synthesize_audio(const orc_dac* synthesis, const orc_rvq* q, const uint16_t* tokens, size_t frames,
                         size_t groups, size_t chunk, unsigned threads, float* pcm);
int16_t orc_pcm16(float x);

#ifdef __cplusplus
}
#endif
#endif
