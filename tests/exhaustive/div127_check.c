/* Exhaustive check of the device quantizer's division-free scale (qmh_div127 in
 * quillm_amd/csrc/qmh_device.h): q1 = fma(fma(-q0, 127, m), r, q0) with q0 = m*r, r = fl(1/127),
 * against the IEEE quotient m/127 (reference src/quant.c:47) for every non-negative float m.
 * +inf is excluded: the device selects it explicitly. Prints the mismatch count; exit 0 iff none. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

int main(void) {
    const float r = 1.0f / 127.0f;
    uint64_t bad = 0, checked = 0;
    for (uint64_t u = 0; u <= 0x7fffffffu; u++) {
        const uint32_t b = (uint32_t)u;
        float m;
        memcpy(&m, &b, 4);
        if (isinf(m)) continue;
        const float want = m / 127.0f;
        const float q0 = m * r;
        const float q1 = fmaf(fmaf(-q0, 127.0f, m), r, q0);
        checked++;
        if (isnan(want) ? !isnan(q1) : memcmp(&want, &q1, 4) != 0) {
            if (bad < 5) printf("m=%a want %a got %a\n", m, want, q1);
            bad++;
        }
    }
    printf("checked %llu, mismatches %llu\n", (unsigned long long)checked, (unsigned long long)bad);
    return bad != 0;
}
