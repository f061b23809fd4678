// Host build of the product's R64 sub-block decode (sx8-quantization_amd/csrc/
// sx8_device.h), so CPU tests can compare the exact device function with the oracle.
// Built host-only by tests/test_device_decode_cpu.py; never loaded on the GPU path.
#include "sx8_device.h"

extern "C" void sx8e_dequant_split(int64_t n_blocks, int64_t n_cb, const uint16_t* dmin,
                                   const uint16_t* dmax, const uint8_t* config,
                                   const uint8_t* coeff, const uint8_t* hi, const uint8_t* lo,
                                   const float* basis, const float* scales, int32_t pca,
                                   uint16_t* out) {
    for (int64_t bid = 0; bid < n_blocks; ++bid) {
        const int64_t kb = bid % n_cb;
        for (int sb = 0; sb < 4; ++sb) {
            double b0[8], b1[8];
            for (int i = 0; i < 8; ++i) {
                b0[i] = basis[kb * 64 + 8 * sb + i];
                b1[i] = basis[kb * 64 + 32 + 8 * sb + i];
            }
            const uint32_t H = (uint32_t)hi[bid * 16 + 4 * sb] | ((uint32_t)hi[bid * 16 + 4 * sb + 1] << 8) |
                               ((uint32_t)hi[bid * 16 + 4 * sb + 2] << 16) |
                               ((uint32_t)hi[bid * 16 + 4 * sb + 3] << 24);
            const uint32_t P16 = (uint32_t)lo[bid * 8 + 2 * sb] | ((uint32_t)lo[bid * 8 + 2 * sb + 1] << 8);
            uint32_t w[4];
            if (pca)
                sx8_r64_subblock<true>(sx8_h2f(dmin[bid]), sx8_h2f(dmax[bid]), config[bid], coeff[bid],
                                       sb, H, P16, b0, b1, scales[kb * 2], scales[kb * 2 + 1], w);
            else
                sx8_r64_subblock<false>(sx8_h2f(dmin[bid]), sx8_h2f(dmax[bid]), config[bid], coeff[bid],
                                        sb, H, P16, b0, b1, 0.0, 0.0, w);
            for (int j = 0; j < 4; ++j) {
                out[bid * 32 + 8 * sb + 2 * j] = (uint16_t)(w[j] & 0xFFFFu);
                out[bid * 32 + 8 * sb + 2 * j + 1] = (uint16_t)(w[j] >> 16);
            }
        }
    }
}
