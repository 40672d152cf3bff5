/*
 * CPU oracle for the .nrm container's checksum and InferCtx::new's rope table
 * -- TEST INFRASTRUCTURE ONLY. Only tests/ and bench.py's cpu_baseline leg use
 * this file, as the checker; libnrq never links it.
 *
 * CRC-32 here is IEEE 802.3 (reflected polynomial 0xEDB88320, register preset
 * to all ones, result inverted), the checksum of crates/nr-model/src/crc32.rs.
 * Both entry points follow zlib's convention for a running value:
 * crc(crc(0, a), b) == crc(0, a || b), which is Crc32::new / update / finish
 * (crc32.rs:38-68) with the inversion moved to the call boundary.
 */
#include <math.h>
#include <string.h>

#include "nrq_oracle.h"

#define NRO_CRC_POLY 0xEDB88320u

/* crc32.rs:6-33: table 0 holds the register after one byte (eight reflected
 * shift/xor rounds); table s is table s-1 advanced by one more zero byte, so
 * table s maps a byte that is followed by s further bytes. */
static uint32_t crc_tab_[8][256];
static int crc_tab_ready_;

static void crc_tables_(void) {
    if (crc_tab_ready_) return;
    for (uint32_t i = 0; i < 256; i++) {
        uint32_t c = i;
        for (int k = 0; k < 8; k++) c = (c & 1u) ? (c >> 1) ^ NRO_CRC_POLY : c >> 1;
        crc_tab_[0][i] = c;
    }
    for (int s = 1; s < 8; s++)
        for (int i = 0; i < 256; i++) {
            uint32_t p = crc_tab_[s - 1][i];
            crc_tab_[s][i] = crc_tab_[0][p & 0xffu] ^ (p >> 8);
        }
    crc_tab_ready_ = 1;
}

/* crc32.rs:45-68, Crc32::update: eight bytes per step (the register is xored
 * into the first four, each byte then looked up in the table for its distance
 * to the end of the step), the remainder a byte at a time. */
uint32_t nro_crc32(uint32_t crc, const void *data, size_t n) {
    crc_tables_();
    const uint8_t *p = (const uint8_t *)data;
    uint32_t c = ~crc;
    for (; n >= 8; n -= 8, p += 8) {
        uint32_t lo = ((uint32_t)p[0] | (uint32_t)p[1] << 8 | (uint32_t)p[2] << 16 | (uint32_t)p[3] << 24) ^ c;
        c = crc_tab_[7][lo & 0xffu] ^ crc_tab_[6][(lo >> 8) & 0xffu] ^ crc_tab_[5][(lo >> 16) & 0xffu] ^
            crc_tab_[4][lo >> 24] ^ crc_tab_[3][p[4]] ^ crc_tab_[2][p[5]] ^ crc_tab_[1][p[6]] ^ crc_tab_[0][p[7]];
    }
    for (; n; n--, p++) c = crc_tab_[0][(c ^ *p) & 0xffu] ^ (c >> 8);
    return ~c;
}

/* The classic one-bit-at-a-time CRC (crates/nr-model/tests/verify.rs:16-30),
 * independent of every table: the pin for nro_crc32. */
uint32_t nro_crc32_bitwise(uint32_t crc, const void *data, size_t n) {
    const uint8_t *p = (const uint8_t *)data;
    uint32_t c = ~crc;
    for (size_t i = 0; i < n; i++) {
        c ^= p[i];
        for (int k = 0; k < 8; k++) c = (c & 1u) ? NRO_CRC_POLY ^ (c >> 1) : c >> 1;
    }
    return ~c;
}

/* InferCtx::new's rope table (infer.rs:433-447) over rope::rope_freqs
 * (rope.rs:14-34). With `factors` (a RopeFreqs tensor, head_dim/2 divisors)
 * the base spectrum theta^(-2i/head_dim) is divided by them and the header's
 * scaling is ignored; otherwise factor > 0 applies Llama-3 wavelength scaling:
 * wavelengths past original_ctx/low are divided by factor, those between
 * original_ctx/high and original_ctx/low are blended linearly. */
void nro_infer_freqs(float *out, size_t head_dim, float theta, float factor, float low, float high, float orig_ctx,
                     const float *factors) {
    const float pi = 3.14159265358979323846f; /* core::f32::consts::PI */
    for (size_t i = 0; i < head_dim / 2; i++) {
        float exponent = -2.0f * (float)i / (float)head_dim;
        float freq = powf(theta, exponent);
        if (!factors && factor > 0.0f) {
            float wavelen = 2.0f * pi / freq;
            float low_wavelen = orig_ctx / low;
            float high_wavelen = orig_ctx / high;
            if (wavelen > low_wavelen) {
                freq /= factor;
            } else if (wavelen > high_wavelen) {
                float smooth = (orig_ctx / wavelen - low) / (high - low);
                freq = (1.0f - smooth) * freq / factor + smooth * freq;
            }
        }
        if (factors) freq /= factors[i];
        out[i] = freq;
    }
}
