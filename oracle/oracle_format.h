/* TEST INFRASTRUCTURE ONLY: range coder state of the CPU oracle (src/format/range.hpp). */
#ifndef TSAC_ORACLE_FORMAT_H
#define TSAC_ORACLE_FORMAT_H

#include "tsac_oracle.h"

typedef struct orc_encoder
{
    uint32_t range, low;
    uint8_t pending_byte;
    size_t pending_count, max_bytes;
    int finished;
    uint8_t* bytes;
    size_t size, capacity;
} orc_encoder;

typedef struct orc_decoder
{
    const uint8_t* bytes;
    size_t length, offset, zero_bytes;
    uint32_t range, code;
} orc_decoder;

void orc_encoder_init(orc_encoder* e, size_t max_bytes);
int orc_encoder_put(orc_encoder* e, uint16_t probability_zero, int bit);
int orc_encoder_finish(orc_encoder* e);
size_t orc_encoder_bit_position(const orc_encoder* e);
int orc_decoder_init(orc_decoder* d, const uint8_t* bytes, size_t length);
int orc_decoder_get(orc_decoder* d, uint16_t probability_zero, int* bit);
int orc_encode_categorical(orc_encoder* e, const float* p, size_t n, size_t symbol);
int orc_decode_categorical(orc_decoder* d, const float* p, size_t n, size_t* symbol);
int orc_validate_header(const orc_header* h);

#endif
