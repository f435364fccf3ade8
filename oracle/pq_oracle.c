/*
 * C restatement of the PolarQuant-KV encoder's bit-exact part.
 *
 * TEST INFRASTRUCTURE ONLY: linked by tests/ (through ctypes) as a second,
 * independent restatement of oracle.quantize_rotated, and timed as a CPU
 * baseline. The product library never links it.
 *
 * Reference: csrc/flash_turboquant.cu:141-173 and
 * integration/polarquant-kv.patch:226-268 (same code in the ggml copy):
 *   buf[t] = rot[t] * rot[t]   (t < D; 0 for D <= t < slots)
 *   for (s = slots/2; s > 0; s >>= 1) buf[t] += buf[t + s]   (t < s)
 *   r = sqrtf(buf[0])
 *   dir[t] = r > 1e-30f ? rot[t] / r : 0
 *   idx = first i minimising fabsf(dir - cb[i])  (strict '<' scan)
 * slots = max(128, next power of two >= D) (patch:455-457).
 *
 * Built with -ffp-contract=off so that rot*rot and the tree adds round
 * separately, as they do in the reference (the square is stored to shared
 * memory before the adds).
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

static int tree_slots(int d) {
    int s = 1;
    while (s < d) s <<= 1;
    return s < 128 ? 128 : s;
}

/* x_rot: [n, d] fp32 rotated vectors; out radius f32 [n], idx u8 [n, d]. */
int pq_oracle_quantize_rotated(const float *x_rot, const float *cb, int n_levels,
                               float *radius, uint8_t *idx, long n, int d) {
    if (d <= 0 || d > 4096 || n_levels < 2 || n_levels > 16) return -1;
    int slots = tree_slots(d);
    float buf[4096];
    for (long v = 0; v < n; ++v) {
        const float *x = x_rot + v * (long)d;
        for (int t = 0; t < slots; ++t) buf[t] = t < d ? x[t] * x[t] : 0.0f;
        for (int s = slots / 2; s > 0; s >>= 1)
            for (int t = 0; t < s; ++t) buf[t] = buf[t] + buf[t + s];
        float r = sqrtf(buf[0]);
        radius[v] = r;
        for (int t = 0; t < d; ++t) {
            float dir = r > 1e-30f ? x[t] / r : 0.0f;
            int best = 0;
            float bd = 1e30f;
            for (int i = 0; i < n_levels; ++i) {
                float dist = fabsf(dir - cb[i]);
                if (dist < bd) { bd = dist; best = i; }
            }
            idx[v * (long)d + t] = (uint8_t)best;
        }
    }
    return 0;
}

/* y[j] = fp32 FMA chain over k ascending of x[k] * R[j][k] (inverse = 0) or
 * x[k] * R[k][j] (inverse = 1): the arithmetic of the reference's rotation
 * loops (flash_turboquant.cu:132-137, patch:217-223,405-411,430-435), where
 * `sum += a * b` is contracted to one fused multiply-add. fmaf rounds once. */
int pq_oracle_rotate_fma(const float *x, const float *R, float *y, long n, int d, int inverse) {
    if (d <= 0) return -1;
    for (long v = 0; v < n; ++v)
        for (int j = 0; j < d; ++j) {
            float acc = 0.0f;
            for (int k = 0; k < d; ++k)
                acc = fmaf(x[v * d + k], inverse ? R[k * d + j] : R[j * d + k], acc);
            y[v * d + j] = acc;
        }
    return 0;
}

/* fp32 -> fp16 bits, round to nearest even (IEEE 754 binary16). */
static uint16_t f32_to_f16_rne(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t exp = (x >> 23) & 0xFFu;
    uint32_t man = x & 0x7FFFFFu;
    if (exp == 0xFFu) return (uint16_t)(sign | 0x7C00u | (man ? 0x200u : 0));
    int e = (int)exp - 127 + 15;
    if (e >= 31) return (uint16_t)(sign | 0x7C00u);
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        man |= 0x800000u;
        int shift = 14 - e;
        uint32_t half = man >> shift;
        uint32_t rem = man & ((1u << shift) - 1u);
        uint32_t mid = 1u << (shift - 1);
        if (rem > mid || (rem == mid && (half & 1u))) half++;
        return (uint16_t)(sign | half);
    }
    uint32_t h = ((uint32_t)e << 10) | (man >> 13);
    uint32_t rem = man & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
    return (uint16_t)(sign | h);
}

/* Serialise to block_pq4 (n_bits 4, 18 B / 32 coords) or block_pq2
 * (n_bits 2, 10 B / 32 coords): {fp16 radius; packed codes}. The radius is
 * saturated to 65504 before the fp16 rounding, as the reference's fp16
 * radius store does (src/polarquant_kv_cuda/compress_kernel.py:178,
 * clamp(-65504, 65504).half()); NaN stays NaN. */
int pq_oracle_pack_blocks(const float *radius, const uint8_t *idx, int n_bits,
                          uint8_t *out, long n, int d) {
    if (d % 32 || (n_bits != 4 && n_bits != 2)) return -1;
    int bb = n_bits == 4 ? 18 : 10;
    int nb = d / 32;
    for (long v = 0; v < n; ++v) {
        uint16_t r16 = f32_to_f16_rne(radius[v] > 65504.0f ? 65504.0f : radius[v]);
        for (int b = 0; b < nb; ++b) {
            uint8_t *blk = out + (v * nb + b) * (long)bb;
            const uint8_t *c = idx + v * (long)d + b * 32;
            blk[0] = (uint8_t)(r16 & 0xFF);
            blk[1] = (uint8_t)(r16 >> 8);
            if (n_bits == 4)
                for (int i = 0; i < 16; ++i) blk[2 + i] = (uint8_t)(c[2 * i] | (c[2 * i + 1] << 4));
            else
                for (int i = 0; i < 8; ++i)
                    blk[2 + i] = (uint8_t)(c[4 * i] | (c[4 * i + 1] << 2) | (c[4 * i + 2] << 4) |
                                           (c[4 * i + 3] << 6));
        }
    }
    return 0;
}
