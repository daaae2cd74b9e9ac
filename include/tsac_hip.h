/*
 * tsac_hip: the TSAC probability model on AMD Instinct MI355X (gfx950).
 *
 * A C ABI with plain pointers and sizes. Every function returns 0 on success or
 * a nonzero status; tsac_hip_last_error() then names the failed requirement (a
 * thread-local string). No C++ exception crosses this boundary. Sessions stay
 * usable after any failure.
 *
 * Each entry point names the reference interface it replaces (paths relative to
 * the skimmilk/tsac-metal tree).
 */
#ifndef TSAC_HIP_H
#define TSAC_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TSAC_HIP_OK 0
#define TSAC_HIP_ERROR 1

/* Message of the calling thread's last failure ("" after success). */
const char* tsac_hip_last_error(void);

/* ---- model description (host memory, borrowed during creation) -------------
 * Geometry of the two-stack model; the reference fixes width 512, 4x128 heads,
 * FFN 2048, 12 temporal + 3 codebook layers, latent 1024, alphabet 1024,
 * context 1024 (src/models/config.hpp:11-16). */
typedef struct tsac_hip_geometry
{
    uint32_t width, heads, head_width, ffn;
    uint32_t temporal_layers, codebook_layers;
    uint32_t latent, alphabet, books, channels, context;
    float attention_scale; /* 0.0883883461356163f for 128-wide heads */
} tsac_hip_geometry;

/* LinearWeights (src/models/types.hpp:44-48): int8 values [N][K] (input
 * fastest), fp32 block scales [K/256][N], fp32 bias [N]. */
typedef struct tsac_hip_linear
{
    const int8_t* values;
    const float* scales;
    const float* bias;
} tsac_hip_linear;

/* TransformerModel accessors (src/models/transformer_model.hpp:6-29).
 * projections: temporal 4L+{qkv, attn_out, mlp_in, mlp_out}, codebook
 * 4*Lt+4L+{...}, then temporal cb_proj, codebook cb_proj, proj_f
 * (src/models/contract.cpp:88-110,195-199). norms: temporal 2L+{ln_1, ln_2},
 * 2*Lt = ln_f, codebook 2*Lt+1+2L+{...}, 2*Lt+1+2*Lc = ln_f (contract.cpp:201-211). */
typedef struct tsac_hip_model_desc
{
    tsac_hip_geometry geometry;
    const tsac_hip_linear* projections;
    const uint16_t* const* norm_gain; /* BF16 [width] each */
    const uint16_t* const* norm_bias;
    const uint16_t* positions;  /* BF16 [books][width] (codebook_decoder.wpe) */
    const uint16_t* rotations;  /* BF16 [context][head_width] interleaved (cos, sin) */
    const uint16_t* embeddings; /* BF16 [books][alphabet][latent] feedback embeddings */
} tsac_hip_model_desc;

/* Policy limits (include/tsac/types.hpp:21-31); a zero field takes the
 * reference default. */
typedef struct tsac_hip_limits
{
    uint64_t file_bytes, symbols, pcm_bytes, cache_bytes, tensor_elements;
} tsac_hip_limits;

/* Header (src/format/container.hpp:10-25). */
typedef struct tsac_hip_header
{
    uint8_t method, groups, model_channels, codebooks;
    uint64_t frames;
    uint16_t batch;
} tsac_hip_header;

typedef struct tsac_hip_model tsac_hip_model;
typedef struct tsac_hip_session tsac_hip_session;

/* ---- model and sessions (src/metal/transformer.hpp:13-39) ------------------ */

/* MetalTransformer::from_model (src/metal/transformer.hpp:16): validates the
 * description, uploads and re-lays out the weights on the current HIP device.
 * The description's host memory may be released after return. */
int tsac_hip_model_create(const tsac_hip_model_desc* desc, const tsac_hip_limits* limits,
                          tsac_hip_model** model);
/* Destroys the model; every session created from it must be destroyed first. */
void tsac_hip_model_destroy(tsac_hip_model* model);

/* MetalTransformer::new_session (src/metal/transformer.hpp:24): independent
 * mutable state (caches, scratch, stream) sharing the immutable model. One
 * caller at a time per session; separate sessions may run concurrently. The
 * session reads TSAC_HIP_FRAME_LAUNCH from the environment once, here: "plain"
 * launches its decode frame steps without the cooperative co-residency
 * guarantee (for runs under a profiler, on an otherwise idle device); anything
 * else, or unset, launches them cooperatively. */
int tsac_hip_session_create(tsac_hip_model* model, tsac_hip_session** session);
void tsac_hip_session_destroy(tsac_hip_session* session);
/* MetalTransformer::clear_session (src/metal/transformer.hpp:27): releases
 * caches and scratch, keeps the model; the next call recreates them. */
int tsac_hip_session_clear(tsac_hip_session* session);

/* MetalTransformer::encode (src/metal/transformer.hpp:30): normal framing of
 * `count` tokens laid out [frame][group][book] (count must equal
 * frames*groups*codebooks). Writes a library-allocated FBAZ stream; release it
 * with tsac_hip_free. Identical bytes to the reference's pack_normal. */
int tsac_hip_encode(tsac_hip_session* session, const tsac_hip_header* header,
                    const uint16_t* tokens, size_t count, uint8_t** stream, size_t* length);

/* MetalTransformer::decode (src/metal/transformer.hpp:33): decodes an FBAZ
 * normal stream to library-allocated tokens (release with tsac_hip_free);
 * verifies the token CRC before returning (src/format/entropy.cpp:153). */
int tsac_hip_decode(tsac_hip_session* session, const uint8_t* stream, size_t length,
                    uint16_t** tokens, size_t* count);

void tsac_hip_free(void* pointer);

/* EntropyPosition (include/tsac/observer.hpp:7-10): token_offset indexes the
 * [frame][group][book] token array. */
typedef struct tsac_hip_position
{
    uint64_t frame, group, codebook, lane, step, token_offset;
} tsac_hip_position;

/* EntropyObserver (include/tsac/observer.hpp:12-16) as C callbacks; either may
 * be NULL. They run on the calling thread, once per symbol in stream order
 * (step, book, lane, group), after the call's GPU work has completed, as
 * MetalTransformer runs its observers (src/metal/transformer.hpp:9-12).
 * after_symbol receives the bits the range encoder spent on the symbol
 * (RangeEncoder::bit_position() before and after it, src/format/entropy.cpp:86-100)
 * when encoding and 0 when decoding (src/format/entropy.cpp:137-149). A nonzero
 * return stops the call, which then fails with "stopped by the observer". */
typedef struct tsac_hip_observer
{
    void* context;
    int (*before_symbol)(void* context, const tsac_hip_position* position);
    int (*after_symbol)(void* context, const tsac_hip_position* position, uint64_t bits);
} tsac_hip_observer;

/* MetalTransformer::encode / decode with their EntropyObserver argument
 * (src/metal/transformer.hpp:30-33); observer may be NULL. tsac_hip_encode and
 * tsac_hip_decode are these with no observer. */
int tsac_hip_encode_observed(tsac_hip_session* session, const tsac_hip_header* header,
                             const uint16_t* tokens, size_t count, const tsac_hip_observer* observer,
                             uint8_t** stream, size_t* length);
int tsac_hip_decode_observed(tsac_hip_session* session, const uint8_t* stream, size_t length,
                             const tsac_hip_observer* observer, uint16_t** tokens, size_t* count);

/* Teacher-forced probability-model outputs: the BF16 distribution the model
 * assigns to every token position (out: host [count][alphabet]), i.e. what
 * TransformerPredictor::predict returns (src/common/transformer.cpp:137-182).
 * mode 0 = encode-side pass (all frames known; causal GEMM/prefill shapes),
 * mode 1 = decode-side pass (frame by frame, book by book; GEMV shapes). The
 * two modes return identical bits. */
#define TSAC_HIP_PASS_ENCODE 0
#define TSAC_HIP_PASS_DECODE 1
int tsac_hip_distributions(tsac_hip_session* session, const tsac_hip_header* header,
                           const uint16_t* tokens, size_t count, int mode, uint16_t* out);

/* Wall-clock split of the session's last encode/decode/distributions call
 * (seconds): [0] GPU model work, [1] host range coding, [2] total, [3] the
 * host-to-device copy of the call's input (tokens, or the stream's payload),
 * included in [0] and [2]; for decode-side passes [4] the GPU time of the
 * frame-step loop, between two HIP events on the session's stream, [5] the
 * number of frame steps in it (both 0 otherwise) and [6] how those frame steps
 * were launched: 0 cooperatively (co-residency guaranteed), 1 as plain launches
 * because the session was created with TSAC_HIP_FRAME_LAUNCH=plain in the
 * environment (for example to run under a profiler), 2 as plain launches
 * because another process held the device's cooperative-launch resources; -1
 * when the call ran no frame step (an encode runs frame steps only when its
 * batched pass would not fit Limits::cache_bytes), and [7] 1 when the call's
 * model work ran step by step (every decode; an encode whose batched pass
 * would not fit Limits::cache_bytes), else 0. No counterpart in the reference; for callers
 * that report throughput with inputs already in device memory. */
int tsac_hip_session_timing(const tsac_hip_session* session, double* seconds, size_t count);

/* ---- the DAC codec around the model (AudioAnalyzer, include/tsac/audio_analyzer.hpp) ---- */

/* ConvolutionWeights (src/models/types.hpp:33-37) as the DAC source stores a
 * convolution: dims are the stored axes, axis 0 fastest (ordinary [in, kernel,
 * out], transposed [out, kernel, in]); either float32 `values`, or int8
 * `quantized` with BF16 `scales` [dims[2]][dims[0]/32][align8(dims[1])]
 * (src/weights/preparation.cpp:31-56); the weight-norm gain per stored column
 * [dims[2]]; the bias per output channel. */
typedef struct tsac_hip_dac_convolution
{
    uint32_t dims[3];
    const float* values;
    const int8_t* quantized;
    const uint16_t* scales;
    const float* gain;
    const float* bias;
} tsac_hip_dac_convolution;

/* One quantizer codebook as the packed RVQ roles hold it
 * (src/weights/pack_main.cpp:244-300): codebook [1024][8], normalised search
 * vectors [1024][8], folded input projection [8][1024] + bias [8], folded
 * output projection [1024][8] + bias [1024]. */
typedef struct tsac_hip_rvq_book
{
    const float* codebook;
    const float* search;
    const float* input_weights;
    const float* input_bias;
    const float* output_weights;
    const float* output_bias;
} tsac_hip_rvq_book;

/* DacAnalysisModel, DacSynthesisModel (convolutions and Snake alphas numbered
 * as src/models/contract.cpp numbers them) and RvqEncoderModel/RvqDecoderModel. */
typedef struct tsac_hip_dac_desc
{
    uint32_t channels, books;
    tsac_hip_dac_convolution analysis[30];
    const float* analysis_alpha[29];
    tsac_hip_dac_convolution synthesis[30];
    const float* synthesis_alpha[29];
    tsac_hip_rvq_book rvq[12];
} tsac_hip_dac_desc;

typedef struct tsac_hip_dac tsac_hip_dac;

/* DacAnalysis / DacSynthesis / RvqEncoder / RvqDecoder ::from_model
 * (src/common/{analysis,synthesis}.tpp, src/common/rvq.{cpp,tpp}): prepares every
 * convolution (BF8 expansion, DAC weight-norm folding,
 * src/common/dsp.tpp:117-155) and uploads it to the current device. The
 * description's memory may be released after return. */
int tsac_hip_dac_create(const tsac_hip_dac_desc* desc, const tsac_hip_limits* limits, tsac_hip_dac** dac);
void tsac_hip_dac_destroy(tsac_hip_dac* dac);

/* The packer's quantizer preparation for one codebook (src/weights/pack_main.cpp:244-300):
 * search [1024][8] = normalize_search of each codebook row; input_weights
 * [8][1024] and output_weights [1024][8] = DAC weight-norm folds of the source
 * in_proj (v [8][1024], g [8]) and out_proj (v [1024][8], g [1024]). */
int tsac_hip_prepare_rvq(const float* codebook, const float* in_v, const float* in_g, const float* out_v,
                         const float* out_g, float* search, float* input_weights, float* output_weights);

/* analyze_audio (src/common/audio_pipeline.hpp:37-58) on the GPU: padded PCM,
 * interleaved float [frames*512][groups*dac channels], through DAC analysis and
 * the quantizer in chunks of 400 latent frames with 8/9 context frames, to
 * tokens [frame][group][codebook] (frames*groups*codebooks). */
int tsac_hip_dac_analyze(tsac_hip_session* session, const tsac_hip_dac* dac, const float* pcm, size_t frames,
                         size_t groups, uint32_t codebooks, uint16_t* tokens);
/* synthesize_audio (src/common/audio_pipeline.hpp:60-79): tokens through the
 * quantizer's decoder and DAC synthesis in chunks with 11 context frames, to
 * float PCM [frames*512][groups*channels] (no rounding, as the reference). */
int tsac_hip_dac_synthesize(tsac_hip_session* session, const tsac_hip_dac* dac, const uint16_t* tokens,
                            size_t frames, size_t groups, uint32_t codebooks, float* pcm);

/* DacAnalysis::apply / DacSynthesis::apply (src/common/analysis.hpp:31-33,
 * src/common/synthesis.hpp:36-38) on one window without chunking, in the
 * reference's Signal layout (channels fastest): synthesis == 0 takes PCM
 * [frames][channels] (frames a multiple of 512) to latent [frames/512][1024];
 * synthesis == 1 takes latent [frames][1024] to [frames*512][channels]. */
int tsac_hip_dac_apply(tsac_hip_session* session, const tsac_hip_dac* dac, int synthesis, const float* input,
                       size_t frames, float* output);

/* EncodeOptions (include/tsac/audio_analyzer.hpp:16-22): method 0 fast,
 * 1 normal; codebooks 0 = the model's maximum; entropy_batch 0 = automatic. */
typedef struct tsac_hip_encode_options
{
    uint8_t method;
    uint8_t codebooks;
    uint8_t separate_channels;
    uint16_t entropy_batch;
} tsac_hip_encode_options;

/* AudioAnalyzer::encode (include/tsac/audio_analyzer.hpp:33-34, as
 * ScalarAnalyzer::encode composes it, src/scalar/audio_analyzer.cpp:14-38):
 * interleaved float PCM [frames][channels] -> an FBAZ stream (library-allocated,
 * release with tsac_hip_free); normal framing runs the session's model with
 * `observer` (may be NULL). */
int tsac_hip_audio_encode(tsac_hip_session* session, const tsac_hip_dac* dac, const float* samples, size_t frames,
                          uint32_t channels, const tsac_hip_encode_options* options,
                          const tsac_hip_observer* observer, uint8_t** stream, size_t* length);
/* AudioAnalyzer::decode (:35-36, src/scalar/audio_analyzer.cpp:40-63): an
 * FBAZ stream -> interleaved float PCM [frames][channels], padded to whole
 * 512-sample frames (library-allocated, release with tsac_hip_free). */
int tsac_hip_audio_decode(tsac_hip_session* session, const tsac_hip_dac* dac, const uint8_t* stream, size_t length,
                          const tsac_hip_observer* observer, float** samples, size_t* frames, uint32_t* channels);

/* ---- the original model files (tsac_*_q8.bin, dac_*_q8.bin) ---------------- */

typedef struct tsac_hip_source tsac_hip_source;

/* The file-format part of Limits (include/tsac/types.hpp:21-31); a zero field
 * takes the reference default. */
typedef struct tsac_hip_source_limits
{
    uint64_t file_bytes, tensor_elements, tensors, metadata_bytes, name_bytes;
} tsac_hip_source_limits;

/* Tensor (src/weights/source_model.hpp:19-29): storage 0 float32, 1 BF16,
 * 0x8000b BF8, 0x8000e BF8L; dims axis 0 fastest. `name` lives as long as the
 * source. */
typedef struct tsac_hip_source_tensor
{
    const char* name;
    uint32_t storage, rank;
    uint64_t dims[8];
    uint64_t elements;
} tsac_hip_source_tensor;

/* SourceModel::load and ::parse (src/weights/source_model.hpp:33-34,
 * src/weights/source_model.cpp:63-166): the record format with every check of
 * the reference's parser; the bytes are copied. */
int tsac_hip_source_load(const char* path, const tsac_hip_source_limits* limits, tsac_hip_source** source);
int tsac_hip_source_parse(const uint8_t* bytes, size_t length, const tsac_hip_source_limits* limits,
                          tsac_hip_source** source);
void tsac_hip_source_destroy(tsac_hip_source* source);
/* SourceModel::tensors and ::metadata_json (src/weights/source_model.hpp:36-44). */
int tsac_hip_source_tensor_count(const tsac_hip_source* source, size_t* count);
int tsac_hip_source_tensor_info(const tsac_hip_source* source, size_t index, tsac_hip_source_tensor* info);
int tsac_hip_source_metadata(const tsac_hip_source* source, const char** json, size_t* length);
/* SourceModel::dequantize (src/weights/source_model.cpp:284-329) into `out`
 * (capacity in floats, at least the tensor's element count). */
int tsac_hip_source_dequantize(const tsac_hip_source* source, const char* name, float* out, size_t capacity);
/* SourceModel::dac_config and ::transformer_config
 * (src/weights/source_model.cpp:168-266): the shape and inventory checks. */
int tsac_hip_source_dac_config(const tsac_hip_source* source, uint32_t* channels, uint32_t* books);
int tsac_hip_source_transformer_config(const tsac_hip_source* source, uint32_t* books);

/* The packer's preparation of a probability model (src/weights/pack_main.cpp:305-391)
 * from its file and the codec file of the same variant, whose codebook
 * projections are the feedback embeddings: fills `desc` for
 * tsac_hip_model_create with pointers into `prepared` (valid until it is
 * destroyed). */
typedef struct tsac_hip_prepared_transformer tsac_hip_prepared_transformer;
int tsac_hip_prepare_transformer(const tsac_hip_source* transformer, const tsac_hip_source* dac,
                                 tsac_hip_prepared_transformer** prepared, tsac_hip_model_desc* desc);
void tsac_hip_prepared_transformer_destroy(tsac_hip_prepared_transformer* prepared);
/* The packer's preparation of a codec (src/weights/pack_main.cpp:172-300):
 * fills `desc` for tsac_hip_dac_create with pointers into `prepared`. */
typedef struct tsac_hip_prepared_dac tsac_hip_prepared_dac;
int tsac_hip_prepare_dac(const tsac_hip_source* dac, tsac_hip_prepared_dac** prepared, tsac_hip_dac_desc* desc);
void tsac_hip_prepared_dac_destroy(tsac_hip_prepared_dac* prepared);
/* Preparation and creation in one call (ModelDirectory + MetalTransformer::from_model,
 * src/weights/model_directory.hpp, src/metal/transformer.hpp:16; the DAC
 * models' from_model): the prepared host arrays are released on return. */
int tsac_hip_model_create_from_source(const tsac_hip_source* transformer, const tsac_hip_source* dac,
                                      const tsac_hip_limits* limits, tsac_hip_model** model);
int tsac_hip_dac_create_from_source(const tsac_hip_source* dac, const tsac_hip_limits* limits, tsac_hip_dac** model);

/* ---- the command-line codec: audio files, stream headers, options ----------- */

/* pcm16_input (src/audio.cpp:19-38): raw little-endian 16-bit PCM of 1..127
 * interleaved channels to float (1/32768 per step), an incomplete last frame
 * dropped, frames padded with zeros to a multiple of 512. `samples` is
 * library-allocated (release with tsac_hip_free), [frames][channels]. */
int tsac_hip_pcm16_read(const uint8_t* bytes, size_t length, uint32_t channels, const tsac_hip_limits* limits,
                        float** samples, size_t* frames);
/* wave_input (src/audio.cpp:40-72): a RIFF/WAVE file of 16-bit PCM, 1..8
 * channels at 44100 Hz, read like tsac_hip_pcm16_read from the data chunk to
 * the end of the file. */
int tsac_hip_wave_read(const uint8_t* bytes, size_t length, const tsac_hip_limits* limits, float** samples,
                       size_t* frames, uint32_t* channels);
/* pcm16_wave (src/audio.cpp:176-246): interleaved float PCM [frames][channels]
 * to a 44100 Hz 16-bit WAVE file (library-allocated), each sample clamped
 * after scaling by 32768 and rounded half to even; nonfinite samples fail. */
int tsac_hip_wave_write(const float* samples, size_t frames, uint32_t channels, const tsac_hip_limits* limits,
                        uint8_t** bytes, size_t* length);
/* audio_header (src/common/audio_pipeline.hpp:13, src/common/audio_analyzer.cpp:78-108):
 * the stream header tsac_hip_audio_encode writes for `frames` sample frames of
 * `channels`-channel PCM under `options`. */
int tsac_hip_audio_header(size_t frames, uint32_t channels, const tsac_hip_encode_options* options,
                          const tsac_hip_limits* limits, tsac_hip_header* header);
/* parse_header (src/format/container.hpp): the header of a stream. */
int tsac_hip_parse_header(const uint8_t* stream, size_t length, const tsac_hip_limits* limits,
                          tsac_hip_header* header);

/* CliOptions (src/cli.hpp:6-15); input and output point into the arguments. */
typedef struct tsac_hip_cli_options
{
    char command; /* 'c', 'd', 't', or 0 when help is set */
    const char* input;
    const char* output;
    int32_t threads, quality, channels, batch;
    uint32_t verbose;
    uint8_t fast, separate, help, metal;
} tsac_hip_cli_options;
/* parse_cli (src/cli.cpp:7-129) over the arguments after the program name,
 * each a NUL-terminated string. */
int tsac_hip_cli_parse(size_t count, const char* const* arguments, tsac_hip_cli_options* options);
/* cli_help (src/cli.cpp:131-155). */
const char* tsac_hip_cli_help(void);

/* ---- operators on device memory (hipStream_t passed as void*) -------------- */

typedef struct tsac_hip_device_linear tsac_hip_device_linear;

/* PackedLinear::from_weights (src/common/packed_linear.tpp:216-253): copies one
 * projection (host memory) to the current device. */
int tsac_hip_linear_create(const tsac_hip_linear* weights, size_t K, size_t N,
                           tsac_hip_device_linear** linear);
void tsac_hip_linear_destroy(tsac_hip_device_linear* linear);

/* path: 0 automatic (GEMV for M <= 8, the small-M MFMA GEMM for M <= 64 when
 * K <= 2048, and for M <= 1024 when the GEMM's 128 x 128 tiles would occupy at
 * most a quarter of the compute units, else the MFMA GEMM), 1 GEMV, 2 GEMM,
 * 4 small-M MFMA GEMM (row-major activations, M <= 1024, K <= 2048); the GEMM
 * needs y and residual 16-byte aligned.
 * 3 = GEMM on activations in MFMA operand tiles (tsac_hip_bf8l_tiles);
 * accepted by tsac_hip_linear_apply_quantized only. */
#define TSAC_HIP_PATH_AUTO 0
#define TSAC_HIP_PATH_GEMV 1
#define TSAC_HIP_PATH_GEMM 2
#define TSAC_HIP_PATH_GEMM_TILES 3
#define TSAC_HIP_PATH_SMALL 4

/* PackedLinear::apply_into (src/common/packed_linear.tpp:264-302) on device
 * memory: x [M][K] BF16 -> y [M][N] BF16. Quantisation scratch comes from the
 * stream-ordered allocator on `stream`. */
int tsac_hip_linear_apply(const tsac_hip_device_linear* linear, const uint16_t* x, size_t M,
                          uint16_t* y, int path, void* stream);

/* tsac_hip_linear_apply without any device allocation, for callers that cannot
 * allocate (tight serving loops, harnesses that forbid hipMalloc). No
 * counterpart in the reference. The BF8L buffer is a fixed per-device array of
 * 16 MiB (plus its scales), held until the process ends: M x K (M rounded up to
 * a multiple of 128 on the GEMM path) must not exceed 16 MiB, larger calls fail
 * with an error. Every call on a device shares that array, so calls that
 * overlap on one device race. Synchronises `stream` to report a non-finite
 * activation, as tsac_hip_linear_apply does. */
int tsac_hip_linear_apply_static(const tsac_hip_device_linear* linear, const uint16_t* x, size_t M,
                                 uint16_t* y, int path, void* stream);

/* The same product on activations already in BF8L form (q [M][K] int8, scales
 * [M][K/256] fp32 widened from BF16), with an optional BF16 residual [M][N]
 * added after rounding (bf16(residual + y), src/scalar/probability.cpp:6-14);
 * residual may alias y. Launches exactly one kernel and allocates nothing. */
int tsac_hip_linear_apply_quantized(const tsac_hip_device_linear* linear, const int8_t* q,
                                    const float* scales, size_t M, uint16_t* y,
                                    const uint16_t* residual, int path, void* stream);

/* scalar::bf8l (src/scalar/probability.cpp:16-40) on rows of K BF16 values,
 * K in {256, 512, 1024, 2048, 4096}. Fails if any input is not finite. */
int tsac_hip_bf8l(const uint16_t* x, size_t rows, size_t K, int8_t* q, float* scales,
                  void* stream);

/* The same quantisation written as MFMA operand tiles for the encode GEMM
 * (no reference counterpart: the layout is this library's). Rows are padded
 * to P = tsac_hip_tile_rows(rows); byte k of row m is at
 * ((m/32)*(K/32) + k/32)*1024 + ((m%32) + 32*((k/16)%2))*16 + k%16 of q
 * (P*K bytes), and scales are transposed, scales[b*P + m] (P*K/256 floats).
 * Padding rows are left unwritten. */
int tsac_hip_bf8l_tiles(const uint16_t* x, size_t rows, size_t K, int8_t* q, float* scales,
                        void* stream);
size_t tsac_hip_tile_rows(size_t rows);

/* probability_layer_norm_bf16_into (src/common/probability.cpp:138-169), rows
 * of `width` in {256, 512, 1024, 2048}. */
int tsac_hip_layer_norm(const uint16_t* x, size_t rows, size_t width, const uint16_t* gain,
                        const uint16_t* bias, uint16_t* out, void* stream);

/* probability_softmax_bf16_into (src/common/probability.cpp:96-122), rows of
 * `width` in {256, 512, 1024, 2048}. Fails if any input is not finite. */
int tsac_hip_softmax(const uint16_t* x, size_t rows, size_t width, uint16_t* out, void* stream);

/* probability_gelu_bf16 (src/common/probability.cpp:45-85) elementwise. */
int tsac_hip_gelu(const uint16_t* x, size_t count, uint16_t* out, void* stream);

/* probability_rotary_bf16_into (src/common/probability.cpp:24-43). */
int tsac_hip_rotary(const uint16_t* x, const uint16_t* coefficients, size_t count, uint16_t* out,
                    void* stream);

/* scalar::add_bf16 (src/scalar/probability.cpp:6-14): out = bf16(a + b[row % period]). */
int tsac_hip_add(const uint16_t* a, const uint16_t* b, size_t rows, size_t width, size_t period,
                 uint16_t* out, void* stream);

/* scalar::attention_bf16_into (src/scalar/attention.cpp:117-131) for
 * `sequences` independent queries: query [sequences][heads*head_width], keys and
 * values of sequence s at + s*sequence_stride elements, rows of heads*head_width.
 * head_width in {64, 128}. Scratch from the stream-ordered allocator. */
int tsac_hip_attention(const uint16_t* query, const uint16_t* keys, const uint16_t* values,
                       size_t sequence_stride, size_t sequences, size_t time, size_t heads,
                       size_t head_width, float scale, int prefill, uint16_t* out, void* stream);

/* Every query of causal sequences at once (the encode-side shape of the same
 * arithmetic): qkv [rows][3*heads*head_width]; sequence s = rows start[s] ..
 * start[s]+length[s]-1 (device int arrays), its first replay[s] positions use
 * replay rounding; rotations [position][head_width] or NULL. */
int tsac_hip_attention_causal(const uint16_t* qkv, size_t heads, size_t head_width,
                              const int* start, const int* length, const int* replay,
                              size_t sequences, size_t max_length, const uint16_t* rotations,
                              float scale, uint16_t* out, void* stream);

/* ---- calibration (no counterpart in the reference) ------------------------- */

/* The attainable rates roofline fractions are read against, for benchmarks on
 * the device that runs the model. tsac_hip_probe_read launches one pass that
 * streams `bytes` of device memory (a multiple of 64 KiB, 16-byte aligned) with
 * the decode GEMV's load pattern; tsac_hip_probe_mfma launches `workgroups` x 4
 * waves of independent int8 MFMA chains and returns in *ops the int8 operations
 * that launch performs. Time them with events on `stream`. */
int tsac_hip_probe_read(const void* data, size_t bytes, void* stream);
int tsac_hip_probe_mfma(size_t workgroups, int iterations, double* ops, void* stream);

#ifdef __cplusplus
}
#endif
#endif
