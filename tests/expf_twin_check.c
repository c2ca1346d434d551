/* Exhaustive check that r9vx_expf (the GPU/host twin used by the router
 * kernel) equals the host libm expf bit for bit over [lo, hi]. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include "r9vx_expf.h"

int main(int argc, char **argv) {
    int all = argc > 1 && strcmp(argv[1], "all") == 0;
    int64_t b0, b1;
    if (all) {
        b0 = 0;
        b1 = 0xffffffffll;
    } else {
        float lo = -104.0f;
        uint32_t ulo;
        memcpy(&ulo, &lo, 4);
        b0 = 0x80000000ll; /* -0.0 */
        b1 = ulo;          /* negative floats grow in bits as they fall */
    }
    unsigned long long bad = 0, n = 0;
#pragma omp parallel for reduction(+ : bad, n) schedule(static)
    for (int64_t b = b0; b <= b1; ++b) {
        uint32_t u = (uint32_t)b, ua, uc;
        float x, a, c;
        memcpy(&x, &u, 4);
        a = expf(x);
        c = r9vx_expf(x);
        memcpy(&ua, &a, 4);
        memcpy(&uc, &c, 4);
        n++;
        if (ua != uc && !(isnan(a) && isnan(c))) bad++;
    }
    printf("%llu %llu\n", n, bad);
    return bad != 0;
}
