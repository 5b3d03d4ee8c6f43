// Compares fm_expf_ref (the device routing's expf, compiled here for the
// host from the same header) with the libm expf that the oracle and the
// compiled reference link, over every non-NaN float (or every stride-th one).
// Usage: expf_check [stride]  -> prints "checked N mismatches M"
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "../../flash-moe_amd/csrc/fm_expf.h"

static float as_float(unsigned u) { float f; memcpy(&f, &u, 4); return f; }
static unsigned as_bits(float f) { unsigned u; memcpy(&u, &f, 4); return u; }

int main(int argc, char **argv) {
    const long long stride = argc > 1 ? atoll(argv[1]) : 1;
    long long n = 0, bad = 0;
    // both signs: bit patterns 0 .. 0x7f800000 (+0 .. +inf) and the same with the sign bit
#pragma omp parallel for reduction(+ : n, bad) schedule(static, 1 << 16)
    for (long long u = 0; u <= 0x7f800000LL; u += stride) {
        for (unsigned sgn = 0; sgn < 2; sgn++) {
            const float x = as_float((unsigned)u | (sgn << 31));
            volatile float ref = expf(x);
            const float mine = fm_expf_ref(x);
            n++;
            if (as_bits(mine) != as_bits(ref)) {
                if (bad < 4) fprintf(stderr, "x=%a libm=%a mine=%a\n", x, (float)ref, mine);
                bad++;
            }
        }
    }
    printf("checked %lld mismatches %lld\n", n, bad);
    return bad != 0;
}
