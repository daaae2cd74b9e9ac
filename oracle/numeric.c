/*
 * TEST INFRASTRUCTURE ONLY: CPU oracle, numerics and kernels. Built with
 * -ffp-contract=off so every float operation below is one IEEE binary32
 * operation with round-to-nearest-even, as in the reference (CMakeLists.txt:123).
 */
#include "oracle_internal.h"

#include <math.h>
#include <stdio.h>
#include <string.h>

static _Thread_local char last_error[256];

const char* orc_last_error(void)
{
    return last_error;
}

int orc_fail(const char* message)
{
    snprintf(last_error, sizeof last_error, "%s", message);
    return 1;
}

static uint32_t bits_of(float x)
{
    uint32_t b;
    memcpy(&b, &x, 4);
    return b;
}

static float float_of(uint32_t b)
{
    float x;
    memcpy(&x, &b, 4);
    return x;
}

/* src/common/numeric/bf16.hpp:9-13: raw integer ties-to-even, no NaN canonicalisation. */
uint16_t orc_bf16(float value)
{
    const uint32_t b = bits_of(value);
    return (uint16_t)((b + 0x7fffu + ((b >> 16) & 1u)) >> 16);
}

/* src/common/numeric/bf16.hpp:15-18 */
float orc_float(uint16_t value)
{
    return float_of((uint32_t)value << 16);
}

/* src/common/numeric/float_math.hpp:33-37: zero exponent -> signed zero. */
float orc_flush(float x)
{
    const uint32_t b = bits_of(x);
    return (b & 0x7f800000u) == 0 ? float_of(b & 0x80000000u) : x;
}

/* src/common/numeric/float_math.hpp:39-61 */
float orc_add(float x, float y)
{
    return orc_flush(orc_flush(x) + orc_flush(y));
}

float orc_subtract(float x, float y)
{
    return orc_flush(orc_flush(x) - orc_flush(y));
}

float orc_multiply(float x, float y)
{
    return orc_flush(orc_flush(x) * orc_flush(y));
}

float orc_divide(float x, float y)
{
    return orc_flush(orc_flush(x) / orc_flush(y));
}

/* src/common/numeric/probability.hpp:14-33 */
float orc_exp(float z)
{
    z = 87.0f < z ? 87.0f : z;
    z = -88.0f > z ? -88.0f : z;
    const float exponent = z * 0x1.715476p+0f;
    const int32_t n = isfinite(exponent) ? (int32_t)nearbyintf(exponent) : INT32_MIN;
    z = fmaf((float)n, -0x1.630000p-1f, z);
    z = fmaf((float)n, 0x1.bd0106p-13f, z);
    float p = fmaf(0x1.a01a02p-13f, z, 0x1.6c16c2p-10f);
    p = fmaf(p, z, 0x1.111112p-7f);
    p = fmaf(p, z, 0x1.555556p-5f);
    p = fmaf(p, z, 0x1.555556p-3f);
    const float square = z * z;
    p = fmaf(p, z, 0.5f);
    z = fmaf(p, square, z);
    const float plus_one = z + 1.0f;
    return float_of(bits_of(plus_one) + ((uint32_t)n << 23));
}

/* src/format/categorical.cpp:17-30: zero-padded adjacent-pair tree of `width`. */
static float pair_sum(const float* input, size_t count, size_t width)
{
    float values[64];
    memset(values, 0, sizeof values);
    memcpy(values, input, count * sizeof(float));
    while (width > 1)
    {
        width /= 2;
        for (size_t i = 0; i < width; ++i)
        {
            values[i] = orc_add(values[2 * i], values[2 * i + 1]);
        }
    }
    return values[0];
}

static unsigned count_trailing_zeros(size_t x)
{
    unsigned n = 0;
    while (!(x & 1))
    {
        x >>= 1;
        ++n;
    }
    return n;
}

static unsigned bit_width(size_t x)
{
    unsigned n = 0;
    while (x)
    {
        x >>= 1;
        ++n;
    }
    return n;
}

/* src/format/categorical.cpp:44-74: 64-value blocks merged by binary carry. */
float orc_probability_sum(const float* values, size_t count)
{
    if (count <= 8)
    {
        return pair_sum(values, count, 8);
    }
    float partial[64];
    memset(partial, 0, sizeof partial);
    size_t blocks = 0;
    for (size_t offset = 0; offset < count;)
    {
        const size_t n = count - offset < 64 ? count - offset : 64;
        float value = pair_sum(values + offset, n, 64);
        ++blocks;
        const unsigned level = count_trailing_zeros(blocks);
        for (unsigned i = 0; i < level; ++i)
        {
            value = orc_add(value, partial[i]);
            partial[i] = 0;
        }
        partial[level] = value;
        offset += n;
    }
    float value = partial[0];
    for (unsigned i = 1; i < bit_width(blocks); ++i)
    {
        value = orc_add(value, partial[i]);
    }
    return value;
}

/* src/format/categorical.cpp:76-89 */
uint16_t orc_conditional_q15(float left_mass, float mass)
{
    const float value = orc_divide(orc_multiply(left_mass, 32768.0f), mass);
    if (!isfinite(value) || value >= 0x1p63f || value < -0x1p63f)
    {
        return 1;
    }
    const int64_t integer = (int64_t)nearbyintf(value);
    const int32_t low = (int32_t)(uint32_t)integer;
    return (uint16_t)(low < 1 ? 1 : low > 32767 ? 32767 : low);
}

/* src/common/numeric.hpp:11-23 */
static int all_finite(const float* values, size_t count)
{
    uint32_t maximum = 0;
    for (size_t i = 0; i < count; ++i)
    {
        const uint32_t b = bits_of(values[i]) & 0x7fffffffu;
        maximum = b > maximum ? b : maximum;
    }
    return maximum < 0x7f800000u;
}

/* src/scalar/probability.cpp:16-40 */
int orc_bf8l(const float* values, size_t count, int8_t* quantized, uint16_t* scales)
{
    if (count % 256)
    {
        return orc_fail("BF8L activations require 256-value blocks");
    }
    if (!all_finite(values, count))
    {
        return orc_fail("BF8L activations must be finite");
    }
    for (size_t offset = 0; offset < count; offset += 256)
    {
        float maximum = 0;
        for (size_t i = 0; i < 256; ++i)
        {
            const float a = fabsf(orc_flush(values[offset + i]));
            maximum = maximum < a ? a : maximum;
        }
        float s = orc_divide(maximum, 127.0f);
        s = s < 1e-35f ? 1e-35f : s;
        const uint16_t scale = orc_bf16(s);
        scales[offset / 256] = scale;
        const float reciprocal = orc_divide(1.0f, orc_float(scale));
        for (size_t i = 0; i < 256; ++i)
        {
            float r = nearbyintf(orc_multiply(values[offset + i], reciprocal));
            r = r < -128.0f ? -128.0f : (127.0f < r ? 127.0f : r);
            quantized[offset + i] = (int8_t)r;
        }
    }
    return 0;
}

/* src/common/packed_linear.tpp:85-123 with src/scalar/packed_linear.cpp:8-30,
 * restated for the canonical [N][K] weight layout (the R4 interleave is a pure
 * byte permutation of the same weights). */
int orc_qlinear(const int8_t* weights, const float* weight_scales, const float* bias, size_t K,
                size_t N, const uint16_t* x, size_t M, uint16_t* y)
{
    if (!K || K % 256)
    {
        return orc_fail("packed linear input shape mismatch");
    }
    const size_t blocks = K / 256;
    float* expanded = orc_alloc(K * sizeof(float));
    int8_t* q = orc_alloc(K);
    uint16_t* s = orc_alloc(blocks * sizeof(uint16_t));
    float* as = orc_alloc(blocks * sizeof(float));
    int status = 0;
    for (size_t m = 0; m < M && !status; ++m)
    {
        for (size_t k = 0; k < K; ++k)
        {
            expanded[k] = orc_float(x[m * K + k]);
        }
        status = orc_bf8l(expanded, K, q, s);
        if (status)
        {
            break;
        }
        for (size_t b = 0; b < blocks; ++b)
        {
            as[b] = orc_float(s[b]);
        }
        for (size_t n = 0; n < N; ++n)
        {
            const int8_t* w = weights + n * K;
            float sum = 0;
            for (size_t b = 0; b < blocks; ++b)
            {
                int32_t dot = 0;
                for (size_t i = 0; i < 256; ++i)
                {
                    dot += (int32_t)w[b * 256 + i] * (int32_t)q[b * 256 + i];
                }
                const float scale = weight_scales[b * N + n] * as[b];
                sum = fmaf((float)dot, scale, sum);
            }
            y[m * N + n] = orc_bf16(sum + bias[n]);
        }
    }
    orc_free(expanded);
    orc_free(q);
    orc_free(s);
    orc_free(as);
    return status;
}

/* src/common/probability.cpp:138-169 */
int orc_layer_norm(const uint16_t* x, const uint16_t* gain, const uint16_t* bias, size_t n,
                   uint16_t* out)
{
    if (!n)
    {
        return orc_fail("layer normalization shape mismatch");
    }
    float* values = orc_alloc(n * sizeof(float));
    float* squares = orc_alloc(n * sizeof(float));
    for (size_t i = 0; i < n; ++i)
    {
        values[i] = orc_float(x[i]);
        squares[i] = values[i] * values[i];
    }
    const float reciprocal = 1.0f / (float)n;
    const float mean = orc_probability_sum(values, n) * reciprocal;
    float variance = fmaf(orc_probability_sum(squares, n), reciprocal, 0.0f);
    variance = fmaf(mean, -mean, variance);
    variance += 1e-5f;
    const float inverse = 1.0f / sqrtf(variance);
    const float offset = -mean * inverse;
    for (size_t i = 0; i < n; ++i)
    {
        const float normalized = fmaf(values[i], inverse, offset);
        out[i] = orc_bf16(fmaf(normalized, orc_float(gain[i]), orc_float(bias[i])));
    }
    orc_free(values);
    orc_free(squares);
    return 0;
}

/* src/common/probability.cpp:45-63 (the 65,536-entry table of :65-85 holds
 * exactly these values). */
uint16_t orc_gelu(uint16_t value)
{
    const float x = orc_float(value);
    const float cubic = 0x1.2444f2p-5f * x;
    float z = fmaf(cubic, x, 0x1.988454p-1f);
    z = z * x;
    const float half = x * 0.5f;
    z = z * -2.0f;
    const float exponential = orc_exp(z);
    const float denominator = exponential + 1.0f;
    const float sigmoid = 2.0f / denominator;
    const float tanh_value = sigmoid - 1.0f;
    const float plus = tanh_value + 1.0f;
    return orc_bf16(half * plus);
}

/* src/common/probability.cpp:7-12 */
uint16_t orc_add_bf16(uint16_t left, uint16_t right)
{
    return orc_bf16(orc_float(left) + orc_float(right));
}

/* src/common/probability.cpp:24-43: interleaved (real, imaginary) pairs. */
int orc_rotary(const uint16_t* values, const uint16_t* coefficients, size_t n, uint16_t* out)
{
    if (n % 2)
    {
        return orc_fail("rotary pair shape mismatch");
    }
    for (size_t i = 0; i < n; i += 2)
    {
        const float re = orc_float(values[i]), im = orc_float(values[i + 1]);
        const float c = orc_float(coefficients[i]), s = orc_float(coefficients[i + 1]);
        const float im_s = im * s;
        const float re_s = re * s;
        out[i] = orc_bf16(fmaf(re, c, -im_s));
        out[i + 1] = orc_bf16(fmaf(im, c, re_s));
    }
    return 0;
}

/* src/common/probability.cpp:96-122 */
int orc_softmax(const uint16_t* x, size_t n, uint16_t* out)
{
    if (!n)
    {
        return orc_fail("softmax shape mismatch");
    }
    float maximum = -INFINITY;
    for (size_t i = 0; i < n; ++i)
    {
        const float v = orc_float(x[i]);
        if (!isfinite(v))
        {
            return orc_fail("softmax input must be finite");
        }
        maximum = maximum < v ? v : maximum;
    }
    float* e = orc_alloc(n * sizeof(float));
    for (size_t i = 0; i < n; ++i)
    {
        const float shifted = orc_float(x[i]) - maximum;
        e[i] = orc_exp(shifted);
    }
    const float total = orc_probability_sum(e, n);
    const float reciprocal = 1.0f / total;
    for (size_t i = 0; i < n; ++i)
    {
        out[i] = orc_bf16(e[i] * reciprocal);
    }
    orc_free(e);
    return 0;
}

/* src/scalar/attention.cpp:12-131 for row-major keys (tests/attention.cpp:71-79
 * shows the reference's tiled-key layout yields the same bits). */
int orc_attention(const uint16_t* query, const uint16_t* keys, const uint16_t* values,
                  size_t time, size_t heads, size_t head_width, float scale, int prefill,
                  uint16_t* out)
{
    const size_t width = heads * head_width;
    if (!width || !time)
    {
        return orc_fail("attention shape mismatch");
    }
    const int round_values = time > 64 || prefill;
    float* numerator = orc_alloc(head_width * sizeof(float));
    float scores[64];
    for (size_t head = 0; head < heads; ++head)
    {
        float running_maximum = -INFINITY, total = 0;
        memset(numerator, 0, head_width * sizeof(float));
        for (size_t start = 0; start < time; start += 64)
        {
            const size_t count = time - start < 64 ? time - start : 64;
            float maximum = -INFINITY;
            for (size_t t = 0; t < count; ++t)
            {
                const uint16_t* k = keys + (start + t) * width + head * head_width;
                const uint16_t* q = query + head * head_width;
                float dot = 0;
                for (size_t j = 0; j < head_width; ++j)
                {
                    dot = fmaf(orc_float(q[j]), orc_float(k[j]), dot);
                }
                scores[t] = dot * scale;
                maximum = maximum < scores[t] ? scores[t] : maximum;
            }
            for (size_t t = 0; t < count; ++t)
            {
                const float shifted = scores[t] - maximum;
                scores[t] = orc_exp(shifted);
            }
            const float difference = maximum - running_maximum;
            const float factor = orc_exp(-fabsf(difference));
            const float old_scale = running_maximum > maximum ? 1.0f : factor;
            const float new_scale = running_maximum > maximum ? factor : 1.0f;
            const float old_total = total * old_scale;
            total = fmaf(orc_probability_sum(scores, count), new_scale, old_total);
            for (size_t j = 0; j < head_width; ++j)
            {
                float sum = 0;
                for (size_t t = 0; t < count; ++t)
                {
                    sum = fmaf(orc_float(values[(start + t) * width + head * head_width + j]),
                               scores[t], sum);
                }
                if (round_values)
                {
                    sum = orc_float(orc_bf16(sum));
                }
                const float old = numerator[j] * old_scale;
                numerator[j] = fmaf(sum, new_scale, old);
            }
            running_maximum = running_maximum < maximum ? maximum : running_maximum;
        }
        const float reciprocal = 1.0f / total;
        for (size_t j = 0; j < head_width; ++j)
        {
            out[head * head_width + j] = orc_bf16(numerator[j] * reciprocal);
        }
    }
    orc_free(numerator);
    return 0;
}

/* Batch helpers so tests can sweep large input sets through one call. */
void orc_exp_batch(const float* z, size_t count, float* out)
{
    for (size_t i = 0; i < count; ++i)
    {
        out[i] = orc_exp(z[i]);
    }
}

void orc_gelu_batch(const uint16_t* x, size_t count, uint16_t* out)
{
    for (size_t i = 0; i < count; ++i)
    {
        out[i] = orc_gelu(x[i]);
    }
}

void orc_bf16_batch(const float* x, size_t count, uint16_t* out)
{
    for (size_t i = 0; i < count; ++i)
    {
        out[i] = orc_bf16(x[i]);
    }
}
