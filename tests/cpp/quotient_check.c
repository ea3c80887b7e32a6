/* quotient_check.c - exhaustive check of the int8 quantizer's quotient (q8_code in sc_kernels.hip).
 *
 * The kernel forms x / sf from y = RN(1/sf), computed once per group, as q0 = RN(x * y), then
 * q = RN(q0 + RN_exact(x - q0 * sf) * y) with both steps fused multiply-adds.  This program checks, for every binary32
 * significand a in [1, 2) (2^23 values) against every binary16 significand b in [1, 2) (2^10 values; a subnormal
 * binary16 scale normalises to one of them), that q equals the IEEE quotient a / b bit for bit.  The operations scale
 * exactly with the operands' exponents as long as nothing leaves the normal range, so equality here is equality for
 * the quantizer's operands.  Built with -ffp-contract=off and -mfma: `*` and `/` round once each, fmaf is the
 * hardware fused operation.  Prints the count of mismatches and exits non-zero on any.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

int main(void) {
    unsigned long long bad = 0, checked = 0;
#pragma omp parallel for reduction(+ : bad, checked) schedule(dynamic, 8)
    for (int M = 0; M < 1024; ++M) {
        const float b = 1.0f + (float) M / 1024.0f;
        const float y = 1.0f / b;
        for (uint32_t m = 0; m < (1u << 23); ++m) {
            const uint32_t bits = 0x3F800000u | m;
            float a;
            memcpy(&a, &bits, 4);
            const float q0 = a * y;
            const float q = fmaf(fmaf(-q0, b, a), y, q0);
            bad += q != a / b;
        }
        checked += 1u << 23;
    }
    printf("quotient_check: %llu pairs, %llu mismatches\n", checked, bad);
    return bad != 0;
}
