/* Test tool: the device's log1pf (warp_amd/csrc/hip/log1pf.h, compiled for
 * the host) against the host libm's over every non-NaN float.  Prints the
 * count of inputs whose results differ in any bit; exit 1 if any.
 *   make -C oracle log1pf_check && oracle/log1pf_check [stride] */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include "../warp_amd/csrc/hip/log1pf.h"

int main(int argc, char **argv)
{
    const uint64_t stride = argc > 1 ? strtoull(argv[1], NULL, 10) : 1;
    uint64_t n = 0, bad = 0;
    for (uint64_t i = 0; i < (1ull << 32); i += stride ? stride : 1) {
        float x;
        const uint32_t b = (uint32_t)i;
        memcpy(&x, &b, 4);
        if (isnan(x)) continue;
        const float a = log1pf(x), d = wh_log1pf(x);
        uint32_t ua, ud;
        memcpy(&ua, &a, 4);
        memcpy(&ud, &d, 4);
        n++;
        if (ua != ud && !(isnan(a) && isnan(d))) {
            if (bad < 8) printf("x = %a: libm %a, device %a\n", x, a, d);
            bad++;
        }
    }
    printf("log1pf: %llu inputs, %llu differ\n", (unsigned long long)n, (unsigned long long)bad);
    return bad != 0;
}
