/*
 * CPU oracle, C restatement of the INT4-G32 byte/integer work (TEST INFRASTRUCTURE ONLY).
 *
 * Written as plain scalar loops, independently of the numpy restatement in
 * oracle/w4g32.py, so the two pin each other bit for bit.  Nothing here is linked into
 * or called by the product library.
 *
 * Reference anchors:
 *   dequant  w = bf16(float(q - z) * float(s))      src/moss_tts/_runtime/calibrated_quant.py:41-42
 *   signed nibble export / unpack                   src/moss_tts/calibration.py:190-191,
 *                                                   src/moss_tts/_runtime/calibrated_backend.py:8-13
 *   dequant-then-matmul                             src/moss_tts/calibration.py:185-188
 */
#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <string.h>

static uint16_t bf16_rne(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) /* NaN */
        return (uint16_t)(((u >> 16) & 0x8000u) | 0x7fc0u);
    uint32_t lsb = (u >> 16) & 1u;
    return (uint16_t)((u + 0x7fffu + lsb) >> 16);
}

static float bf16_to_f32(uint16_t b) {
    uint32_t u = (uint32_t)b << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

void oracle_bf16_rne(const float *in, uint16_t *out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = bf16_rne(in[i]);
}

/* qweight int32 [K/8, N]: nibble j of word (i, n) is the code of k = 8i + j. */
void oracle_unpack_gptq(const uint32_t *qweight, int K, int N, uint8_t *q /* [N, K] */) {
    for (int n = 0; n < N; ++n)
        for (int k = 0; k < K; ++k) {
            uint32_t word = qweight[(size_t)(k / 8) * N + n];
            q[(size_t)n * K + k] = (uint8_t)((word >> (4 * (k % 8))) & 15u);
        }
}

/* qzeros int32 [G, N/8]: nibble j of word (g, c) is the zero of column 8c + j. */
void oracle_unpack_gptq_zeros(const uint32_t *qzeros, int G, int N, uint8_t *z /* [N, G] */) {
    for (int n = 0; n < N; ++n)
        for (int g = 0; g < G; ++g) {
            uint32_t word = qzeros[(size_t)g * (N / 8) + n / 8];
            z[(size_t)n * G + g] = (uint8_t)((word >> (4 * (n % 8))) & 15u);
        }
}

void oracle_dequant(const uint8_t *q, const uint8_t *z, const uint16_t *s, int N, int K,
                    uint16_t *w /* bf16 bits [N, K] */) {
    int G = K / 32;
    for (int n = 0; n < N; ++n)
        for (int k = 0; k < K; ++k) {
            int g = k / 32;
            float d = (float)((int)q[(size_t)n * K + k] - (int)z[(size_t)n * G + g]);
            float p = d * bf16_to_f32(s[(size_t)n * G + g]);
            w[(size_t)n * K + k] = bf16_rne(p);
        }
}

/* The reference's signed export: byte j of row n holds codes 2j (low) and 2j+1 (high). */
void oracle_unpack_signed(const uint8_t *packed, int N, int K, int8_t *codes /* [N, K] */) {
    for (int n = 0; n < N; ++n)
        for (int j = 0; j < K / 2; ++j) {
            uint8_t b = packed[(size_t)n * (K / 2) + j];
            int lo = b & 15, hi = b >> 4;
            codes[(size_t)n * K + 2 * j] = (int8_t)(lo >= 8 ? lo - 16 : lo);
            codes[(size_t)n * K + 2 * j + 1] = (int8_t)(hi >= 8 ? hi - 16 : hi);
        }
}

/* Kernel row-packed layout (see oracle/w4g32.py: rowpack). */
void oracle_rowpack(const uint8_t *q, const uint8_t *z, int N, int K, uint32_t *qw /* [N, K/8] */,
                    uint8_t *zp /* [N, G/2] */) {
    int G = K / 32;
    for (int n = 0; n < N; ++n) {
        for (int w = 0; w < K / 8; ++w) {
            uint32_t word = 0;
            for (int t = 0; t < 8; ++t) {
                uint32_t code = q[(size_t)n * K + 8 * w + t] & 15u;
                int shift = (t % 2 == 0) ? 4 * (t / 2) : 16 + 4 * (t / 2);
                word |= code << shift;
            }
            qw[(size_t)n * (K / 8) + w] = word;
        }
        /* zero points in blocks of 128 groups: byte 64c + b = z[128c + b] | z[128c + r/2 + b] << 4 */
        for (int c0 = 0; c0 < G; c0 += 128) {
            int r = G - c0 < 128 ? G - c0 : 128;
            for (int b = 0; b < r / 2; ++b)
                zp[(size_t)n * (G / 2) + c0 / 2 + b] = (uint8_t)((z[(size_t)n * G + c0 + b] & 15u) |
                                                                ((z[(size_t)n * G + c0 + r / 2 + b] & 15u) << 4));
        }
    }
}

/* y[m, n] = sum_k x[m, k] * w[n, k], fp64 accumulation of exact bf16 x bf16 products. */
void oracle_linear_f64(const uint16_t *x, const uint16_t *w, int M, int N, int K, double *y) {
    for (int m = 0; m < M; ++m)
        for (int n = 0; n < N; ++n) {
            double acc = 0.0;
            for (int k = 0; k < K; ++k)
                acc += (double)bf16_to_f32(x[(size_t)m * K + k]) * (double)bf16_to_f32(w[(size_t)n * K + k]);
            y[(size_t)m * N + n] = acc;
        }
}
