/* C restatement of the block-FP8 dequantisation of inference/ops.py:30-43.
 *
 * TEST INFRASTRUCTURE ONLY: loaded by tests/ (ctypes) as the bit-exact checker
 * of the GPU dequant; never linked into the product library.
 *
 * e4m3fn (OCP 8-bit float, "fn" = finite, no infinities): 1 sign bit, 4 exponent
 * bits with bias 7, 3 mantissa bits.  exponent 0 encodes subnormals m * 2^-9;
 * S.1111.111 is NaN; everything else is (1 + m/8) * 2^(e-7); max 448.
 * Dequant is one IEEE binary32 multiply f32(w) * scale_inv[i/128][j/128] rounded
 * to nearest even; this file is compiled with -ffp-contract=off so no multiply
 * is fused with anything.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

float oracle_e4m3_to_f32(uint8_t code) {
    int sign = code >> 7;
    int e = (code >> 3) & 0xF;
    int m = code & 0x7;
    float v;
    if (e == 0xF && m == 0x7) {
        uint32_t nan_bits = sign ? 0xFFC00000u : 0x7FC00000u;
        memcpy(&v, &nan_bits, 4);
        return v;
    }
    if (e == 0)
        v = ldexpf((float)m, -9);              /* subnormal: m/8 * 2^(1-7) */
    else
        v = ldexpf(1.0f + (float)m / 8.0f, e - 7);
    return sign ? -v : v;
}

/* out[i*K + j] = e4m3(w[i*K + j]) * scale[(i/block) * kb + j/block] */
void oracle_fp8_block_dequant(const uint8_t *w, const float *scale, int64_t N, int64_t K,
                              int64_t block, float *out) {
    int64_t kb = (K + block - 1) / block;
    float table[256];
    for (int c = 0; c < 256; ++c) table[c] = oracle_e4m3_to_f32((uint8_t)c);
    for (int64_t i = 0; i < N; ++i) {
        const float *srow = scale + (i / block) * kb;
        for (int64_t j = 0; j < K; ++j) {
            volatile float prod = table[w[i * K + j]] * srow[j / block];
            out[i * K + j] = prod;
        }
    }
}
