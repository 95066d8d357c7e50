/* Checks the division-free form of peak / 127 used by the device quantiser
 * (int8_scale_from_peak in rustyneedle_amd/csrc/rn_device.hpp) against the
 * correctly rounded float division of ops.rs:103-110, over every positive
 * finite float whose bit pattern is a multiple of `stride` (argv[1]; 1 checks
 * all 2^31 - 2^23 - 1 of them). Prints the number of mismatches. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static float from_bits(uint32_t b) {
    float f;
    memcpy(&f, &b, sizeof f);
    return f;
}

int main(int argc, char** argv) {
    const long stride = argc > 1 ? atol(argv[1]) : 1;
    const float inv127 = 1.0f / 127.0f;
    long bad = 0, checked = 0;
#pragma omp parallel for reduction(+ : bad, checked) schedule(static)
    for (long i = stride; i <= 0x7f7fffffL; i += stride) {
        const float a = from_bits((uint32_t)i);
        const float q0 = a * inv127;
        const float q = fmaf(fmaf(-q0, 127.0f, a), inv127, q0);
        bad += q != a / 127.0f;
        checked += 1;
    }
    printf("%ld %ld\n", bad, checked);
    return 0;
}
