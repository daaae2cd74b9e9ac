/*
 * TEST INFRASTRUCTURE ONLY: CPU restatement of the reference's scalar DAC
 * analysis/synthesis and residual vector quantizer, the path the reference's
 * ScalarAnalyzer runs where Apple frameworks are absent. Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline use it.
 *
 * Signals follow the reference layout: values[(group*frames + frame)*channels
 * + channel] (channels fastest). Convolution weights are in the reference's
 * stored layout: ordinary [input, kernel, output], transposed [output, kernel,
 * input], axis 0 fastest.
 *
 * Pinning (tests/test_oracle_dac.py):
 *   orc_dac_sine_squared, orc_snake   compiled reference scalar_snake_frames
 *                                      (src/scalar/dsp.cpp) on random and edge phases
 *   orc_conv1d                        compiled reference scalar::Conv1d, ordinary and
 *                                      transposed, strides/dilations of the DAC
 *   orc_fold_dac_weight_norm          compiled reference fold_dac_weight_norm
 *   orc_expand_bf8                    compiled reference weights::expand_into layout
 *                                      restated; closed form int8 x BF16 scale
 *   orc_normalize_search, orc_nearest_rvq, orc_project_codebook
 *                                      compiled reference (src/weights/preparation.cpp,
 *                                      src/common/rvq.cpp)
 *   composition (orc_dac_apply, analysis/synthesis chunking, RVQ encoder/decoder)
 *                                      restated from src/common/{analysis,synthesis}.tpp,
 *                                      rvq.{cpp,tpp}, audio_pipeline.hpp; the reference's
 *                                      DacAnalysis/DacSynthesis need model adapters that
 *                                      need the packer's generated header, so the layer
 *                                      sequence exists here as a restatement
 */
#include "oracle_internal.h"

#include <math.h>
#include <pthread.h>
#include <string.h>

/* ---- Snake (src/scalar/dsp.cpp:47-111, src/weights/normalization.hpp:9) -------- */

static float from_bits(uint32_t bits)
{
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* dac_sine_squared (src/scalar/dsp.cpp:47-84): sin(phase)^2 by quadrant
 * reduction with a two-term pi/2 and the original minimax polynomials. */
float orc_dac_sine_squared(float phase)
{
    const float reduced = phase * from_bits(0x3f22f983);
    const double lower = floor((double)reduced);
    const double fraction = (double)reduced - lower;
    const double nearest = lower + (fraction > 0.5 || (fraction == 0.5 && fmod(lower, 2.0) != 0));
    const float quadrant = (float)nearest;
    const int32_t q = nearest >= -2147483648.0 && nearest < 2147483648.0 ? (int32_t)nearest : INT32_MIN;
    float x = fmaf(quadrant, from_bits(0xbfc90000), phase);
    x = fmaf(quadrant, from_bits(0xb9fdaa22), x);
    const float x2 = x * x;
    float value;
    if ((q & 1) == 0)
    {
        float polynomial = fmaf(from_bits(0xb94ca1f9), x2, from_bits(0x3c08839e));
        polynomial = fmaf(polynomial, x2, from_bits(0xbe2aaaa3));
        const float cube = x * x2;
        value = fmaf(cube, polynomial, x);
    }
    else
    {
        float polynomial = fmaf(from_bits(0x37ccf5ce), x2, from_bits(0xbab6061a));
        polynomial = fmaf(polynomial, x2, from_bits(0x3d2aaaa5));
        polynomial = fmaf(polynomial, x2, from_bits(0xbf000000));
        value = fmaf(polynomial, x2, 1.0f);
    }
    return value * value;
}

/* snake_dac_into (src/scalar/dsp.cpp:86-111): x + sin^2(a x) / (a + eps) per
 * channel, frames [count / channels][channels]. */
int orc_snake(const float* x, size_t count, size_t channels, const float* alpha, float* out)
{
    const float epsilon = from_bits(0x3089705f);
    for (size_t c = 0; c < channels; ++c)
    {
        if (!isfinite(alpha[c] + epsilon) || alpha[c] + epsilon == 0.0f)
        {
            return orc_fail("invalid Snake denominator");
        }
    }
    for (size_t i = 0; i < count; ++i)
    {
        const float a = alpha[i % channels];
        const float phase = a * x[i];
        if (!isfinite(phase))
        {
            return orc_fail("nonfinite Snake phase");
        }
        const float squared = orc_dac_sine_squared(phase);
        volatile float denominator = a + epsilon;
        volatile float quotient = squared / denominator;
        out[i] = x[i] + quotient;
        if (!isfinite(out[i]))
        {
            return orc_fail("nonfinite DSP value");
        }
    }
    return 0;
}

/* ---- weight preparation ------------------------------------------------------ */

/* fold_dac_weight_norm_into (src/weights/normalization.cpp:47-95): per column
 * of fan_in values, squares reduced by a balanced adjacent-pair tree (odd tail
 * carried), RMS normalise, times 1/sqrt(fan_in), times the column's gain. */
int orc_fold_dac_weight_norm(const float* v, const float* g, size_t fan_in, size_t columns, float* out)
{
    if (!fan_in || !columns)
    {
        return orc_fail("empty weight normalization shape");
    }
    volatile float width_f = (float)fan_in;
    const float inverse_width = 1.0f / sqrtf(width_f);
    const float reciprocal_width = 1.0f / width_f;
    float* squares = orc_alloc(fan_in * sizeof(float));
    for (size_t c = 0; c < columns; ++c)
    {
        const float* column = v + c * fan_in;
        for (size_t i = 0; i < fan_in; ++i)
        {
            if (!isfinite(column[i]))
            {
                free(squares);
                return orc_fail("nonfinite weight normalization value");
            }
            squares[i] = column[i] * column[i];
        }
        for (size_t width = fan_in; width > 1; width = (width + 1) / 2)
        {
            for (size_t i = 0; i < width / 2; ++i)
            {
                squares[i] = squares[2 * i] + squares[2 * i + 1];
            }
            if (width % 2)
            {
                squares[width / 2] = squares[width - 1];
            }
        }
        const float mean = squares[0] * reciprocal_width;
        if (!(mean > 0) || !isfinite(mean))
        {
            free(squares);
            return orc_fail("invalid weight normalization norm");
        }
        const float inverse_rms = 1.0f / sqrtf(mean);
        for (size_t i = 0; i < fan_in; ++i)
        {
            const float normalized = column[i] * inverse_rms;
            const float unit = normalized * inverse_width;
            out[c * fan_in + i] = unit * g[c];
            if (!isfinite(out[c * fan_in + i]))
            {
                free(squares);
                return orc_fail("nonfinite weight normalization value");
            }
        }
    }
    free(squares);
    return 0;
}

/* weights::expand_into for BF8 (src/weights/preparation.cpp:31-56): axes
 * [rows, cols, outer] (rows fastest), int8 data plane in element order, one
 * BF16 scale per 32 rows of each column at scales[(outer*(rows/32) + b)*align8(cols) + col]. */
int orc_expand_bf8(const int8_t* data, const uint16_t* scales, size_t rows, size_t cols, size_t outer, float* out)
{
    if (!rows || !cols || rows % 32)
    {
        return orc_fail("invalid quantized source shape");
    }
    const size_t padded = (cols + 7) / 8 * 8;
    for (size_t column = 0; column < cols * outer; ++column)
    {
        for (size_t b = 0; b < rows / 32; ++b)
        {
            const uint16_t bits = scales[(column / cols * (rows / 32) + b) * padded + column % cols];
            const float scale = orc_float(bits);
            for (size_t i = 0; i < 32; ++i)
            {
                const size_t k = column * rows + b * 32 + i;
                out[k] = (float)data[k] * scale;
                if (!isfinite(out[k]))
                {
                    return orc_fail("nonfinite source weights");
                }
            }
        }
    }
    return 0;
}

/* ---- convolution (src/common/dsp.tpp:175-210, src/scalar/dsp.cpp:9-45) -------- */

size_t orc_conv_output_frames(const orc_conv* c, size_t frames)
{
    const size_t span = (c->kernel - 1) * c->dilation + 1;
    if (!c->transposed)
    {
        const size_t padded = frames + 2 * c->padding;
        return padded < span ? 0 : (padded - span) / c->stride + 1;
    }
    const size_t full = (frames - 1) * c->stride + span;
    return full > 2 * c->padding ? full - 2 * c->padding : 0;
}

/* Convolution::source_frame: the input frame tap `tap` of output `frame` reads,
 * or -1 when it falls in the padding or between strided samples. */
static long long source_frame(const orc_conv* c, size_t frame, size_t tap)
{
    if (!c->transposed)
    {
        const size_t position = frame * c->stride + tap * c->dilation;
        return position < c->padding ? -1 : (long long)(position - c->padding);
    }
    const size_t position = frame + c->padding, offset = tap * c->dilation;
    if (position < offset || (position - offset) % c->stride)
    {
        return -1;
    }
    return (long long)((position - offset) / c->stride);
}

typedef struct
{
    const orc_conv* c;
    const float *w, *bias, *x;
    size_t frames, out_frames, groups;
    float* y;
    size_t first, last; /* output channels */
} conv_job;

/* Conv1d::sample: one serial sum per output, taps ascending, input channels
 * ascending within a tap, each term a product then an addition (no FMA);
 * out-of-range taps are skipped; the bias is added last. */
static void* conv_worker(void* argument)
{
    const conv_job* j = argument;
    const orc_conv* c = j->c;
    const size_t stored = c->transposed ? c->out : c->in;
    const size_t column = stored * c->kernel;
    for (size_t g = 0; g < j->groups; ++g)
    {
        for (size_t f = 0; f < j->out_frames; ++f)
        {
            for (size_t o = j->first; o < j->last; ++o)
            {
                float sum = 0.0f;
                for (size_t tap = 0; tap < c->kernel; ++tap)
                {
                    const long long s = source_frame(c, f, tap);
                    if (s < 0 || (size_t)s >= j->frames)
                    {
                        continue;
                    }
                    const float* row = j->x + (g * j->frames + (size_t)s) * c->in;
                    for (size_t i = 0; i < c->in; ++i)
                    {
                        const size_t index = c->transposed ? o + tap * stored + i * column : i + tap * stored + o * column;
                        const float product = row[i] * j->w[index];
                        sum = sum + product;
                    }
                }
                j->y[(g * j->out_frames + f) * c->out + o] = sum + j->bias[o];
            }
        }
    }
    return NULL;
}

int orc_conv1d(const orc_conv* c, const float* w, const float* bias, const float* x, size_t frames, size_t groups,
               float* y, unsigned threads)
{
    const size_t out_frames = orc_conv_output_frames(c, frames);
    if (!out_frames)
    {
        return orc_fail("convolution has no output frames");
    }
    for (size_t i = 0; i < frames * groups * c->in; ++i)
    {
        if (!isfinite(x[i]))
        {
            return orc_fail("nonfinite DSP value");
        }
    }
    if (threads < 1)
    {
        threads = 1;
    }
    if (threads > c->out)
    {
        threads = (unsigned)c->out;
    }
    pthread_t* handles = orc_alloc(threads * sizeof(pthread_t));
    conv_job* jobs = orc_alloc(threads * sizeof(conv_job));
    for (unsigned t = 0; t < threads; ++t)
    {
        jobs[t] = (conv_job){c, w, bias, x, frames, out_frames, groups, y, c->out * t / threads, c->out * (t + 1) / threads};
        if (t + 1 < threads)
        {
            pthread_create(&handles[t], NULL, conv_worker, &jobs[t]);
        }
    }
    conv_worker(&jobs[threads - 1]);
    for (unsigned t = 0; t + 1 < threads; ++t)
    {
        pthread_join(handles[t], NULL);
    }
    free(handles);
    free(jobs);
    for (size_t i = 0; i < out_frames * groups * c->out; ++i)
    {
        if (!isfinite(y[i]))
        {
            return orc_fail("nonfinite DSP value");
        }
    }
    return 0;
}

/* ---- the DAC graphs (src/common/analysis.tpp:150-230, synthesis.tpp:140-220) ---- */

/* Convolution i's geometry (src/models/contract.cpp:55-84 shapes;
 * src/common/{analysis,synthesis}.tpp strides, dilations, transposition;
 * padding of src/common/dsp.tpp:105-113). */
int orc_dac_conv_config(int synthesis, unsigned channels, unsigned index, orc_conv* c)
{
    static const unsigned analysis_stride[4] = {2, 4, 8, 8}, synthesis_stride[4] = {8, 8, 4, 2};
    static const unsigned dilation[3] = {1, 3, 9};
    size_t first, kernel, last, stride = 1, dil = 1;
    int transposed = 0;
    if (index >= 30 || (channels != 1 && channels != 2))
    {
        return orc_fail("invalid DAC convolution");
    }
    if (index == 0)
    {
        first = synthesis ? 1024 : channels, kernel = 7, last = synthesis ? 1536 : 64;
    }
    else if (index == 29)
    {
        first = synthesis ? 96 : 1024, kernel = synthesis ? 7 : 3, last = synthesis ? channels : 1024;
    }
    else
    {
        const unsigned stage = (index - 1) / 7, within = (index - 1) % 7;
        const size_t width = synthesis ? (1536u >> stage) : (64u << stage);
        const unsigned s = synthesis ? synthesis_stride[stage] : analysis_stride[stage];
        if (synthesis && within == 0)
        {
            first = width / 2, kernel = 2 * s, last = width, stride = s, transposed = 1;
        }
        else if (!synthesis && within == 6)
        {
            first = width, kernel = 2 * s, last = width * 2, stride = s;
        }
        else
        {
            const unsigned residual = synthesis ? within - 1 : within;
            const size_t w = synthesis ? width / 2 : width;
            first = w, last = w, kernel = residual % 2 == 0 ? 7 : 1;
            dil = residual % 2 == 0 ? dilation[residual / 2] : 1;
        }
    }
    c->in = transposed ? last : first;
    c->out = transposed ? first : last;
    c->kernel = kernel;
    c->stride = stride;
    c->dilation = dil;
    c->padding = stride == 1 ? (kernel - 1) * dil / 2 : (stride + 1) / 2;
    c->transposed = transposed;
    return 0;
}

size_t orc_dac_activation_width(int synthesis, unsigned index)
{
    if (index == 28)
    {
        return synthesis ? 96 : 1024;
    }
    return synthesis ? (1536u >> (index / 7)) / (index % 7 == 0 ? 1u : 2u) : (64u << (index / 7));
}

typedef struct
{
    const orc_dac* m;
    unsigned threads;
    float *x, *scratch, *temporary; /* capacity each: largest signal */
    size_t frames, channels;         /* current x shape (one group) */
} graph;

static int conv_step(graph* s, unsigned index, float** from, float** to)
{
    orc_conv c;
    if (orc_dac_conv_config(s->m->synthesis, s->m->channels, index, &c))
    {
        return 1;
    }
    if (c.in != s->channels)
    {
        return orc_fail("convolution input channel mismatch");
    }
    const size_t out = orc_conv_output_frames(&c, s->frames);
    if (orc_conv1d(&c, s->m->weights[index], s->m->bias[index], *from, s->frames, 1, *to, s->threads))
    {
        return 1;
    }
    s->frames = out;
    s->channels = c.out;
    return 0;
}

static int snake_step(graph* s, unsigned activation, const float* from, float* to)
{
    return orc_snake(from, s->frames * s->channels, s->channels, s->m->alpha[activation], to);
}

/* ResidualUnit::apply_into: snake, dilated conv, snake, pointwise conv, then
 * the input added back (input + result). x holds the input; on return x holds
 * the output (buffers are swapped). */
static int residual_unit(graph* s, unsigned activation, unsigned convolution)
{
    float* input = s->x;
    const size_t frames = s->frames, channels = s->channels;
    if (snake_step(s, activation, input, s->scratch) || conv_step(s, convolution, &s->scratch, &s->temporary) ||
        snake_step(s, activation + 1, s->temporary, s->scratch) ||
        conv_step(s, convolution + 1, &s->scratch, &s->temporary))
    {
        return 1;
    }
    if (s->frames != frames || s->channels != channels)
    {
        return orc_fail("residual shape mismatch");
    }
    for (size_t i = 0; i < frames * channels; ++i)
    {
        s->temporary[i] = input[i] + s->temporary[i];
        if (!isfinite(s->temporary[i]))
        {
            return orc_fail("nonfinite residual");
        }
    }
    float* t = s->x;
    s->x = s->temporary;
    s->temporary = t;
    return 0;
}

static size_t graph_capacity(const orc_dac* m, size_t frames)
{
    /* the widest signal of either graph, per input frame (synthesis: latent frames) */
    return m->synthesis ? (frames * 8 * 768 > frames * 1536 ? frames * 8 * 768 : frames * 1536) + frames * 512 * 96
                        : frames * 64 + 64 * 7;
}

/* DacAnalysis::apply / DacSynthesis::apply on one group: in [frames][in
 * channels] -> out [out frames][out channels]. */
int orc_dac_apply(const orc_dac* m, const float* in, size_t frames, float* out, size_t* out_frames, unsigned threads)
{
    const size_t capacity = graph_capacity(m, frames) + 4096;
    graph s = {m, threads, orc_alloc(capacity * 4), orc_alloc(capacity * 4), orc_alloc(capacity * 4), frames,
               m->synthesis ? 1024 : m->channels};
    float* entry_input = (float*)in;
    int status = conv_step(&s, 0, &entry_input, &s.x);
    for (unsigned stage = 0; !status && stage < 4; ++stage)
    {
        if (m->synthesis)
        {
            /* snake, upsample, three residual units */
            status = snake_step(&s, stage * 7, s.x, s.scratch) || conv_step(&s, 1 + stage * 7, &s.scratch, &s.x);
            for (unsigned unit = 0; !status && unit < 3; ++unit)
            {
                status = residual_unit(&s, stage * 7 + 1 + unit * 2, 1 + stage * 7 + 1 + unit * 2);
            }
        }
        else
        {
            /* three residual units, snake, downsample */
            for (unsigned unit = 0; !status && unit < 3; ++unit)
            {
                status = residual_unit(&s, stage * 7 + unit * 2, 1 + stage * 7 + unit * 2);
            }
            status = status || snake_step(&s, stage * 7 + 6, s.x, s.scratch) ||
                     conv_step(&s, 1 + stage * 7 + 6, &s.scratch, &s.x);
        }
    }
    status = status || snake_step(&s, 28, s.x, s.scratch) || conv_step(&s, 29, &s.scratch, &s.x);
    if (!status)
    {
        memcpy(out, s.x, s.frames * s.channels * 4);
        *out_frames = s.frames;
    }
    free(s.x);
    free(s.scratch);
    free(s.temporary);
    return status;
}

/* ---- residual vector quantizer (src/common/rvq.{cpp,tpp}, src/weights/preparation.cpp) -- */

/* normalize_search (src/weights/preparation.cpp:62-84). */
void orc_normalize_search(const float* input, float* output)
{
    const float epsilon = from_bits(0x2b8cbccc);
    float squares[8];
    for (int i = 0; i < 8; ++i)
    {
        squares[i] = input[i] * input[i];
    }
    for (int width = 8; width > 1; width /= 2)
    {
        for (int i = 0; i < width / 2; ++i)
        {
            squares[i] = squares[2 * i] + squares[2 * i + 1];
        }
    }
    const float mean = squares[0] * (1.0f / 8.0f);
    volatile float shifted = mean + epsilon;
    const float inverse_rms = 1.0f / sqrtf(shifted);
    const float inverse_width = 1.0f / sqrtf(8.0f);
    for (int i = 0; i < 8; ++i)
    {
        const float normalized = input[i] * inverse_rms;
        output[i] = normalized * inverse_width;
    }
}

/* nearest_rvq_index (src/common/rvq.cpp:131-151): cosine search over the
 * normalised vectors with eight ordered FMAs, strict > (lowest index wins ties). */
uint16_t orc_nearest_rvq(const float* input, const float* vectors)
{
    float query[8];
    orc_normalize_search(input, query);
    float best = -INFINITY;
    uint16_t selected = 0;
    for (size_t index = 0; index < 1024; ++index)
    {
        float similarity = 0.0f;
        for (int i = 0; i < 8; ++i)
        {
            similarity = fmaf(vectors[index * 8 + i], query[i], similarity);
        }
        if (similarity > best)
        {
            best = similarity;
            selected = (uint16_t)index;
        }
    }
    return selected;
}

/* project_codebook, fused (src/weights/preparation.cpp:86-104). */
void orc_project_codebook(uint16_t index, const float* codebook, const float* weights, const float* bias, float* out)
{
    for (size_t j = 0; j < 1024; ++j)
    {
        float sum = 0.0f;
        for (int i = 0; i < 8; ++i)
        {
            sum = fmaf(weights[j * 8 + i], codebook[index * 8 + i], sum);
        }
        out[j] = sum + bias[j];
    }
}

/* RvqEncoder::encode for one group's latent [frames][1024] (src/common/rvq.tpp:40-97):
 * per codebook in order, the input projection (an ordinary 1024 -> 8 pointwise
 * convolution), the search, and the chosen vector's projection subtracted from
 * the residual. tokens [frames][books]. */
int orc_rvq_encode(const orc_rvq* q, const float* latent, size_t frames, uint16_t* tokens)
{
    float* residual = orc_alloc(frames * 1024 * 4);
    float* projected = orc_alloc(frames * 8 * 4);
    float contribution[1024];
    memcpy(residual, latent, frames * 1024 * 4);
    const orc_conv input = {1024, 8, 1, 1, 0, 1, 0};
    int status = 0;
    for (unsigned book = 0; !status && book < q->books; ++book)
    {
        status = orc_conv1d(&input, q->input_weights[book], q->input_bias[book], residual, frames, 1, projected, 1);
        for (size_t f = 0; !status && f < frames; ++f)
        {
            const uint16_t token = orc_nearest_rvq(projected + f * 8, q->search[book]);
            tokens[f * q->books + book] = token;
            orc_project_codebook(token, q->codebook[book], q->output_weights[book], q->output_bias[book], contribution);
            for (size_t i = 0; i < 1024; ++i)
            {
                residual[f * 1024 + i] -= contribution[i];
            }
        }
        for (size_t i = 0; !status && i < frames * 1024; ++i)
        {
            if (!isfinite(residual[i]))
            {
                status = orc_fail("nonfinite RVQ residual");
            }
        }
    }
    free(residual);
    free(projected);
    return status;
}

/* RvqDecoder::decode for one group (src/common/rvq.cpp:84-127): the books'
 * projections added to zero in book order. */
int orc_rvq_decode(const orc_rvq* q, const uint16_t* tokens, size_t frames, float* latent)
{
    float contribution[1024];
    memset(latent, 0, frames * 1024 * 4);
    for (size_t f = 0; f < frames; ++f)
    {
        for (unsigned book = 0; book < q->books; ++book)
        {
            const uint16_t token = tokens[f * q->books + book];
            if (token >= 1024)
            {
                return orc_fail("index outside 10-bit alphabet");
            }
            orc_project_codebook(token, q->codebook[book], q->output_weights[book], q->output_bias[book], contribution);
            for (size_t i = 0; i < 1024; ++i)
            {
                latent[f * 1024 + i] += contribution[i];
            }
        }
    }
    for (size_t i = 0; i < frames * 1024; ++i)
    {
        if (!isfinite(latent[i]))
        {
            return orc_fail("nonfinite RVQ value");
        }
    }
    return 0;
}

/* ---- the audio pipeline (src/common/audio_pipeline.hpp, audio_analyzer.cpp) ---- */

/* audio_chunk (src/common/audio_analyzer.cpp:172-181). */
static void audio_chunk(size_t begin, size_t frames, size_t size, size_t left_context, size_t right_context,
                        size_t* count, size_t* left, size_t* right)
{
    *count = size < frames - begin ? size : frames - begin;
    const size_t end = begin + *count;
    *left = begin > left_context ? begin - left_context : 0;
    *right = end + (right_context < frames - end ? right_context : frames - end);
}

/* analyze_audio (src/common/audio_pipeline.hpp:37-58): padded PCM [groups][frames*512][channels]
 * -> tokens [frame][group][book], chunks of `chunk` latent frames with 8 left and
 * 9 right context frames. */
int orc_analyze_audio(const orc_dac* analysis, const orc_rvq* q, const float* pcm, size_t frames, size_t groups,
                      size_t chunk, unsigned threads, uint16_t* tokens)
{
    const size_t channels = analysis->channels;
    int status = 0;
    for (size_t g = 0; !status && g < groups; ++g)
    {
        for (size_t begin = 0; !status && begin < frames;)
        {
            size_t count, left, right;
            audio_chunk(begin, frames, chunk, 8, 9, &count, &left, &right);
            const float* window = pcm + (g * frames * 512 + left * 512) * channels;
            float* latent = orc_alloc((right - left) * 1024 * 4);
            uint16_t* selected = orc_alloc(count * q->books * 2);
            size_t produced = 0;
            status = orc_dac_apply(analysis, window, (right - left) * 512, latent, &produced, threads);
            if (!status && produced != right - left)
            {
                status = orc_fail("analysis output length mismatch");
            }
            status = status || orc_rvq_encode(q, latent + (begin - left) * 1024, count, selected);
            for (size_t f = 0; !status && f < count; ++f)
            {
                memcpy(tokens + ((begin + f) * groups + g) * q->books, selected + f * q->books, q->books * 2);
            }
            free(latent);
            free(selected);
            begin += count;
        }
    }
    return status;
}

/* synthesize_audio (src/common/audio_pipeline.hpp:60-79): tokens -> PCM
 * [frames*512][groups*channels] interleaved, chunks with 11 context frames on
 * each side. */
int orc_synthesize_audio(const orc_dac* synthesis, const orc_rvq* q, const uint16_t* tokens, size_t frames,
                         size_t groups, size_t chunk, unsigned threads, float* pcm)
{
    const size_t channels = synthesis->channels;
    int status = 0;
    for (size_t g = 0; !status && g < groups; ++g)
    {
        for (size_t begin = 0; !status && begin < frames;)
        {
            size_t count, left, right;
            audio_chunk(begin, frames, chunk, 11, 11, &count, &left, &right);
            const size_t n = right - left;
            uint16_t* selected = orc_alloc(n * q->books * 2);
            float* latent = orc_alloc(n * 1024 * 4);
            float* evaluated = orc_alloc(n * 512 * channels * 4);
            for (size_t f = left; f < right; ++f)
            {
                memcpy(selected + (f - left) * q->books, tokens + (f * groups + g) * q->books, q->books * 2);
            }
            size_t produced = 0;
            status = orc_rvq_decode(q, selected, n, latent) ||
                     orc_dac_apply(synthesis, latent, n, evaluated, &produced, threads);
            if (!status && produced != n * 512)
            {
                status = orc_fail("synthesis output length mismatch");
            }
            for (size_t s = 0; !status && s < count * 512; ++s)
            {
                for (size_t c = 0; c < channels; ++c)
                {
                    pcm[(begin * 512 + s) * groups * channels + g * channels + c] =
                        evaluated[((begin - left) * 512 + s) * channels + c];
                }
            }
            free(selected);
            free(latent);
            free(evaluated);
            begin += count;
        }
    }
    return status;
}

/* pcm16_wave's sample conversion (src/audio.cpp:229-241): clamp(x * 32768) to
 * [-32768, 32767] in double, round half to even. */
int16_t orc_pcm16(float x)
{
    double scaled = (double)x * 32768.0;
    scaled = scaled < -32768.0 ? -32768.0 : (scaled > 32767.0 ? 32767.0 : scaled);
    const double lower = floor(scaled);
    const int32_t integer = (int32_t)lower;
    const double fraction = scaled - lower;
    return (int16_t)(integer + (fraction > 0.5 || (fraction == 0.5 && integer % 2 != 0)));
}
