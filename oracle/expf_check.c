/* SPDX-License-Identifier: Apache-2.0 */
/* expf_check — the oracle's expf against the host libm's on every one of the
 * 2^32 float bit patterns.  Test infrastructure (tests/test_oracle.py, opt-in).
 * On glibc 2.35 (x86-64, FMA ifunc) it prints "mismatches 0". */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>
#include "oracle.h"

int main(void)
{
    uint64_t bad = 0;
    for (uint64_t u = 0; u < (1ULL << 32); u++) {
        const uint32_t b = (uint32_t)u;
        float x, a, c;
        memcpy(&x, &b, 4);
        a = expf(x);
        c = orc_expf(x);
        uint32_t ua, uc;
        memcpy(&ua, &a, 4);
        memcpy(&uc, &c, 4);
        if (ua != uc && !(isnan(a) && isnan(c))) bad++;
    }
    printf("expf: %llu inputs, mismatches %llu\n", 1ULL << 32, (unsigned long long)bad);
    return bad != 0;
}
