// Host build of the HIP library's E4M3 encoder (lcml::e4m3_encode) for the
// exhaustive CPU comparison with the oracle (tests/test_oracle_codec.py).
#include <stdint.h>
#include "lcml_device.hpp"

extern "C" void enc_range(uint32_t first, uint64_t count, uint8_t *out) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < (int64_t)count; ++i)
        out[i] = (uint8_t)lcml::e4m3_encode(lcml::bits_f32(first + (uint32_t)i));
}
