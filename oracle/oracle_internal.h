/* TEST INFRASTRUCTURE ONLY: private helpers of the CPU oracle. */
#ifndef TSAC_ORACLE_INTERNAL_H
#define TSAC_ORACLE_INTERNAL_H

#include "tsac_oracle.h"

#include <stdlib.h>

int orc_fail(const char* message);

static inline void* orc_alloc(size_t bytes)
{
    void* p = calloc(1, bytes ? bytes : 1);
    if (!p)
    {
        abort();
    }
    return p;
}

#endif
