/*
 * TEST INFRASTRUCTURE ONLY: CPU oracle for the range coder, the categorical
 * bisection and the FBAZ container (src/format/).
 */
#include "oracle_internal.h"
#include "oracle_format.h"

#include <math.h>
#include <string.h>

void orc_free(void* pointer)
{
    free(pointer);
}

/* src/format/range.cpp:17-24 */
enum
{
    minimum_range = 0xff01
};

static int split(uint32_t range, uint16_t p0, uint32_t* out)
{
    if (!(p0 > 0 && p0 < 32768))
    {
        return orc_fail("Q15 probability must be in [1,32767]");
    }
    if (range < minimum_range)
    {
        return orc_fail("unnormalized range state");
    }
    *out = (uint32_t)(((uint64_t)range * p0) >> 15);
    return 0;
}

void orc_encoder_init(orc_encoder* e, size_t max_bytes)
{
    memset(e, 0, sizeof *e);
    e->range = 0xff0000;
    e->low = 0;
    e->pending_byte = 0xff;
    e->max_bytes = max_bytes;
}

static int emit(orc_encoder* e, uint32_t value)
{
    if (e->size >= e->max_bytes)
    {
        return orc_fail("range output exceeds limit");
    }
    if (e->size == e->capacity)
    {
        e->capacity = e->capacity ? e->capacity * 2 : 4096;
        uint8_t* grown = realloc(e->bytes, e->capacity);
        if (!grown)
        {
            abort();
        }
        e->bytes = grown;
    }
    e->bytes[e->size++] = (uint8_t)value;
    return 0;
}

/* src/format/range.cpp:25-39 */
static int flush_pending(orc_encoder* e, uint32_t value)
{
    const uint32_t carry = (value >> 8) & 255;
    if (e->pending_count)
    {
        if (emit(e, (uint32_t)e->pending_byte + carry))
        {
            return 1;
        }
        while (e->pending_count > 1)
        {
            if (emit(e, carry - 1))
            {
                return 1;
            }
            --e->pending_count;
        }
    }
    e->pending_byte = (uint8_t)value;
    e->pending_count = 1;
    return 0;
}

/* src/format/range.cpp:41-54 */
static int shift(orc_encoder* e)
{
    if ((e->low >> 16) == 0xff)
    {
        ++e->pending_count;
        if (e->pending_count > e->max_bytes)
        {
            return orc_fail("pending range output exceeds limit");
        }
    }
    else if (flush_pending(e, e->low >> 16))
    {
        return 1;
    }
    e->low = (e->low & 0xffff) << 8;
    e->range <<= 8;
    return 0;
}

/* src/format/range.cpp:56-73 */
int orc_encoder_put(orc_encoder* e, uint16_t probability_zero, int bit)
{
    if (e->finished)
    {
        return orc_fail("range encoder already finished");
    }
    uint32_t range0 = 0;
    if (split(e->range, probability_zero, &range0))
    {
        return 1;
    }
    if (bit)
    {
        e->low += range0;
        e->range -= range0;
    }
    else
    {
        e->range = range0;
    }
    while (e->range < minimum_range)
    {
        if (shift(e))
        {
            return 1;
        }
    }
    return 0;
}

/* src/format/range.cpp:81-87: whole bytes (emitted and pending) times 8 plus the
 * bits the range has consumed below 24. */
size_t orc_encoder_bit_position(const orc_encoder* e)
{
    unsigned width = 0;
    for (uint32_t r = e->range; r; r >>= 1)
    {
        ++width;
    }
    return (e->pending_count + e->size) * 8 + (size_t)(24 - width);
}

/* src/format/range.cpp:83-110 */
int orc_encoder_finish(orc_encoder* e)
{
    if (e->finished)
    {
        return orc_fail("range encoder already finished");
    }
    if (e->range < 0x10000 && shift(e))
    {
        return 1;
    }
    unsigned n = 0;
    for (uint32_t r = e->range; r > 1; r >>= 1)
    {
        ++n;
    }
    if (n < 16 || n > 23)
    {
        return orc_fail("invalid final range");
    }
    const uint32_t unit = 1u << n;
    const uint32_t val = (e->low & (unit - 1)) == 0 ? e->low : (e->low + unit) & (0u - unit);
    if (!(val >= e->low && val < e->low + e->range))
    {
        return orc_fail("invalid range termination");
    }
    if ((val >> 16) == 0xff)
    {
        ++e->pending_count;
        if (e->pending_count > e->max_bytes)
        {
            return orc_fail("pending range output exceeds limit");
        }
    }
    else if (flush_pending(e, val >> 16))
    {
        return 1;
    }
    if (e->pending_count && flush_pending(e, 0))
    {
        return 1;
    }
    e->finished = 1;
    return 0;
}

/* src/format/range.cpp:112-130 */
static uint32_t read_byte(orc_decoder* d)
{
    if (d->offset < d->length)
    {
        return d->bytes[d->offset++];
    }
    ++d->zero_bytes;
    return 0;
}

int orc_decoder_init(orc_decoder* d, const uint8_t* bytes, size_t length)
{
    memset(d, 0, sizeof *d);
    d->bytes = bytes;
    d->length = length;
    d->range = 0xff0000;
    d->code = read_byte(d) << 16;
    d->code |= read_byte(d) << 8;
    d->code |= read_byte(d);
    if (!(d->code < d->range))
    {
        return orc_fail("range code outside initial interval");
    }
    return 0;
}

/* src/format/range.cpp:131-151 */
int orc_decoder_get(orc_decoder* d, uint16_t probability_zero, int* bit)
{
    uint32_t range0 = 0;
    if (split(d->range, probability_zero, &range0))
    {
        return 1;
    }
    *bit = d->code >= range0;
    if (*bit)
    {
        d->code -= range0;
        d->range -= range0;
    }
    else
    {
        d->range = range0;
    }
    while (d->range < minimum_range)
    {
        d->range <<= 8;
        d->code = (d->code << 8) + read_byte(d);
    }
    if (!(d->code < d->range))
    {
        return orc_fail("range code outside interval");
    }
    return 0;
}

/* src/format/categorical.cpp:32-41 */
static int validate_probabilities(const float* p, size_t n)
{
    if (!n)
    {
        return orc_fail("empty categorical alphabet");
    }
    for (size_t i = 0; i < n; ++i)
    {
        if (!(isfinite(p[i]) && p[i] >= 0))
        {
            return orc_fail("categorical probabilities must be finite and nonnegative");
        }
    }
    return 0;
}

/* src/format/categorical.cpp:91-117 */
int orc_encode_categorical(orc_encoder* e, const float* p, size_t n, size_t symbol)
{
    if (validate_probabilities(p, n))
    {
        return 1;
    }
    if (symbol >= n)
    {
        return orc_fail("categorical symbol outside alphabet");
    }
    size_t base = 0, count = n;
    float mass = 1;
    while (count > 1)
    {
        const size_t half = count / 2;
        const float left = orc_probability_sum(p + base, half);
        const int bit = symbol >= base + half;
        if (orc_encoder_put(e, orc_conditional_q15(left, mass), bit))
        {
            return 1;
        }
        if (bit)
        {
            base += half;
            count -= half;
            mass = orc_subtract(mass, left);
        }
        else
        {
            count = half;
            mass = left;
        }
    }
    return 0;
}

/* src/format/categorical.cpp:119-142 */
int orc_decode_categorical(orc_decoder* d, const float* p, size_t n, size_t* symbol)
{
    if (validate_probabilities(p, n))
    {
        return 1;
    }
    size_t base = 0, count = n;
    float mass = 1;
    while (count > 1)
    {
        const size_t half = count / 2;
        const float left = orc_probability_sum(p + base, half);
        int bit;
        if (orc_decoder_get(d, orc_conditional_q15(left, mass), &bit))
        {
            return 1;
        }
        if (bit)
        {
            base += half;
            count -= half;
            mass = orc_subtract(mass, left);
        }
        else
        {
            count = half;
            mass = left;
        }
    }
    *symbol = base;
    return 0;
}

/* src/format/container.cpp:137-153: CRC-32/MPEG-2 over little-endian uint32 tokens. */
uint32_t orc_token_crc32(const uint16_t* tokens, size_t count)
{
    uint32_t crc = 0xffffffff;
    for (size_t i = 0; i < count; ++i)
    {
        for (unsigned shift_bits = 0; shift_bits < 32; shift_bits += 8)
        {
            crc ^= (((uint32_t)tokens[i] >> shift_bits) & 255) << 24;
            for (unsigned bit = 0; bit < 8; ++bit)
            {
                crc = (crc << 1) ^ ((crc & 0x80000000u) ? 0x04c11db7u : 0);
            }
        }
    }
    return crc;
}

/* src/format/container.cpp:9-21 (default Limits of include/tsac/types.hpp:21-31) */
int orc_validate_header(const orc_header* h)
{
    if (h->method > 1)
    {
        return orc_fail("unsupported method");
    }
    if (!(h->groups > 0 && h->groups <= 127))
    {
        return orc_fail("invalid channel groups");
    }
    if (!(h->model_channels == 1 || h->model_channels == 2))
    {
        return orc_fail("invalid model channels");
    }
    if (!(h->codebooks > 0 && h->codebooks <= (h->model_channels == 1 ? 9 : 12)))
    {
        return orc_fail("invalid codebook count");
    }
    if (!(h->method == 0 || h->batch > 0))
    {
        return orc_fail("zero entropy batch size");
    }
    const uint64_t symbols = h->frames * h->groups * h->codebooks;
    if (symbols > (uint64_t)64 * 1024 * 1024)
    {
        return orc_fail("symbol count exceeds limit");
    }
    if (h->frames * 512 * h->groups * h->model_channels * 2 > (uint64_t)1024 * 1024 * 1024)
    {
        return orc_fail("decoded PCM size exceeds limit");
    }
    return 0;
}

/* src/format/container.cpp:43-80 */
int orc_parse_header(const uint8_t* bytes, size_t length, orc_header* h, size_t* payload_offset,
                     size_t* payload_bytes, uint32_t* crc)
{
    if (length > (size_t)512 * 1024 * 1024)
    {
        return orc_fail("input exceeds file size limit");
    }
    if (length < 4)
    {
        return orc_fail("truncated input");
    }
    if (!(bytes[0] == 'F' && bytes[1] == 'B' && bytes[2] == 'A' && bytes[3] == 'Z'))
    {
        return orc_fail("invalid FBAZ magic");
    }
    if (length < 8)
    {
        return orc_fail("truncated input");
    }
    if (bytes[4] != 0)
    {
        return orc_fail("unsupported TSAC version");
    }
    memset(h, 0, sizeof *h);
    h->method = bytes[5];
    h->groups = bytes[6] & 127;
    h->model_channels = 1 + (bytes[6] >> 7);
    h->codebooks = bytes[7];
    h->batch = 1;
    if (h->method > 1)
    {
        return orc_fail("unsupported TSAC method");
    }
    if (!h->groups || !h->codebooks)
    {
        return orc_fail("zero groups or codebooks");
    }
    *crc = 0;
    if (h->method == 0)
    {
        *payload_offset = 8;
        *payload_bytes = length - 8;
        const uint64_t bits_per_frame = (uint64_t)h->groups * h->codebooks * 10;
        const uint64_t bits = (uint64_t)*payload_bytes * 8;
        h->frames = bits / bits_per_frame;
        const uint64_t padding = bits % bits_per_frame;
        if (padding >= 8)
        {
            return orc_fail("incomplete fast frame or excess padding");
        }
        if (padding && (bytes[length - 1] & ((1u << padding) - 1)))
        {
            return orc_fail("nonzero fast padding");
        }
    }
    else
    {
        if (length < 19)
        {
            return orc_fail("truncated normal stream");
        }
        h->frames = ((uint32_t)bytes[8] << 24) | ((uint32_t)bytes[9] << 16) |
                    ((uint32_t)bytes[10] << 8) | bytes[11];
        h->batch = (uint16_t)(((uint16_t)bytes[12] << 8) | bytes[13]);
        *payload_offset = 14;
        *payload_bytes = length - 18;
        *crc = ((uint32_t)bytes[length - 4] << 24) | ((uint32_t)bytes[length - 3] << 16) |
               ((uint32_t)bytes[length - 2] << 8) | bytes[length - 1];
    }
    return orc_validate_header(h);
}

int orc_range_roundtrip_encode(const float* probabilities, const uint16_t* symbols, size_t count,
                               size_t alphabet, uint8_t* out, size_t capacity, size_t* written)
{
    orc_encoder e;
    orc_encoder_init(&e, (size_t)64 * 1024 * 1024);
    int status = 0;
    for (size_t i = 0; i < count && !status; ++i)
    {
        status = orc_encode_categorical(&e, probabilities + i * alphabet, alphabet, symbols[i]);
    }
    if (!status)
    {
        status = orc_encoder_finish(&e);
    }
    if (!status)
    {
        if (e.size > capacity)
        {
            status = orc_fail("output capacity too small");
        }
        else
        {
            memcpy(out, e.bytes, e.size);
            *written = e.size;
        }
    }
    free(e.bytes);
    return status;
}

int orc_range_roundtrip_decode(const float* probabilities, size_t count, size_t alphabet,
                               const uint8_t* bytes, size_t length, uint16_t* symbols)
{
    orc_decoder d;
    if (orc_decoder_init(&d, bytes, length))
    {
        return 1;
    }
    for (size_t i = 0; i < count; ++i)
    {
        size_t s;
        if (orc_decode_categorical(&d, probabilities + i * alphabet, alphabet, &s))
        {
            return 1;
        }
        symbols[i] = (uint16_t)s;
    }
    return 0;
}
