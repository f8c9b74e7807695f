// Host build of the HIP library's E4M3 encoder (lcml::e4m3_encode) for the
// exhaustive CPU comparison with the oracle (tests/test_oracle_codec.py).
#include <stdint.h>
#include "lcml_device.hpp"

extern "C" void enc_range(uint32_t first, uint64_t count, uint8_t *out) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < (int64_t)count; ++i)
        out[i] = (uint8_t)lcml::e4m3_encode(lcml::bits_f32(first + (uint32_t)i));
}

// Host build of lcml::div448_corrected: the number of fp32 patterns in
// [first, last) where it differs from the IEEE quotient a / 448.
extern "C" uint64_t div448_mismatches(uint32_t first, uint32_t last) {
    uint64_t bad = 0;
#pragma omp parallel for schedule(static) reduction(+ : bad)
    for (int64_t i = first; i < (int64_t)last; ++i) {
        const float a = lcml::bits_f32((uint32_t)i);
        const float q = lcml::div448_corrected(a), e = a / 448.0f;
        bad += lcml::f32_bits(q) != lcml::f32_bits(e);
    }
    return bad;
}
