// pcg32 of tinygs/include/tinygs/random/pcg32.hpp:35-125, for host and device.
#pragma once

#include <stdint.h>

#include "detmath.h"

namespace tgs {

// PCG-XSH-RR 64/32 (M. E. O'Neill, "PCG: A family of simple fast
// space-efficient statistically good algorithms for random number
// generation", 2014) with the multiplier, seeding and float conversion of
// pcg32.hpp:35-125.
constexpr uint64_t kPcgMult = 0x5851f42d4c957f2dull;

TGS_HD uint32_t pcg_next(uint64_t& state, uint64_t inc) {
    const uint64_t old = state;
    state = old * kPcgMult + inc;
    const uint32_t xs = (uint32_t)(((old >> 18u) ^ old) >> 27u);
    const uint32_t rot = (uint32_t)(old >> 59u);
    return (xs >> rot) | (xs << ((~rot + 1u) & 31u));
}

// state after `delta` steps (Brown, "Random number generation with arbitrary
// strides", 1994: the affine map x -> a x + c composed by squaring)
TGS_HD uint64_t pcg_advance(uint64_t state, uint64_t inc, uint64_t delta) {
    uint64_t cur_mult = kPcgMult, cur_plus = inc, acc_mult = 1u, acc_plus = 0u;
    while (delta > 0) {
        if (delta & 1u) {
            acc_mult *= cur_mult;
            acc_plus = acc_plus * cur_mult + cur_plus;
        }
        cur_plus = (cur_mult + 1u) * cur_plus;
        cur_mult *= cur_mult;
        delta >>= 1u;
    }
    return acc_mult * state + acc_plus;
}

// [0, 1): 23 random mantissa bits under exponent 0, minus 1
TGS_HD float pcg_float(uint64_t& state, uint64_t inc) {
    return u2f((pcg_next(state, inc) >> 9) | 0x3f800000u) - 1.0f;
}

// pcg32::next_uint(bound) (pcg32.hpp:68-94): rejection of the low
// (2^32 - bound) % bound outputs keeps the result unbiased
inline uint32_t pcg_next_bounded(uint64_t& state, uint64_t inc, uint32_t bound) {
    const uint32_t threshold = (~bound + 1u) % bound;
    for (;;) {
        const uint32_t r = pcg_next(state, inc);
        if (r >= threshold) return r % bound;
    }
}

// pcg32::seed(initstate, initseq) (pcg32.hpp:45-53)
inline void pcg_seed(uint64_t& state, uint64_t& inc, uint64_t initstate, uint64_t initseq) {
    state = 0u;
    inc = (initseq << 1u) | 1u;
    (void)pcg_next(state, inc);
    state += initstate;
    (void)pcg_next(state, inc);
}

}  // namespace tgs
