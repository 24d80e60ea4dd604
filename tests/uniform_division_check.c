/* The quotient tc::div_uniform (tensorcrate_amd/csrc/device.hpp) forms for a
 * divisor shared by a group of elements, checked against the f32 division
 * on the CPU: RN32(RN64(x * RN64(1 / d))), taken where it is a normal
 * float, must be the bits of x / d.  Every x of a stride through all 2^32
 * bit patterns for divisors near the ends of the binades, subnormal and
 * extreme ones, then random pairs.  Prints the counts; exits 1 on the first
 * mismatch.  Built and run by tests/test_uniform_division.py. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

static float from_bits(uint32_t u) {
    float f;
    memcpy(&f, &u, 4);
    return f;
}

static uint32_t to_bits(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}

static long fast, slow;

static int check(float x, float d) {
    const double r = 1.0 / (double)d;
    const float q = (float)((double)x * r);
    if (!isnormal(q)) {
        slow++;
        return 0;
    }
    fast++;
    const float want = x / d;
    if (to_bits(q) != to_bits(want)) {
        printf("mismatch: x %a d %a quotient %a division %a\n", x, d, q, want);
        return 1;
    }
    return 0;
}

int main(void) {
    static const uint32_t divisors[] = {
        0x40400000u, 0x40e00000u, 0x3dcccccdu, 0x3fd9999au, 0x3f800001u, 0x3fffffffu, 0x3f7fffffu,
        0x00000001u, 0x00000003u, 0x007fffffu, 0x00800000u, 0x00800001u, 0x7f7fffffu, 0x7f000001u,
        0x4b7fffffu, 0x42c80000u, 0x3a83126fu, 0xc0400000u, 0xbf800001u, 0x3eaaaaabu};
    for (unsigned k = 0; k < sizeof divisors / sizeof divisors[0]; k++) {
        const float d = from_bits(divisors[k]);
        for (uint64_t u = k; u < (1ull << 32); u += 4099) {
            if (check(from_bits((uint32_t)u), d)) return 1;
        }
    }
    uint64_t state = 0x9e3779b97f4a7c15ull;
    for (long i = 0; i < 20000000; i++) {
        state ^= state << 13, state ^= state >> 7, state ^= state << 17;
        if (check(from_bits((uint32_t)state), from_bits((uint32_t)(state >> 32)))) return 1;
    }
    printf("normal quotients %ld, others (left to the division) %ld, mismatches 0\n", fast, slow);
    return 0;
}
