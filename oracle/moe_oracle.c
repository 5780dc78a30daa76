/*
 * moe_oracle.c — fp64 brute-force restatement of the MXFP4 dequant-matvec
 * and of the synthetic-block generator.
 *
 * TEST INFRASTRUCTURE ONLY: loaded by tests/ (ctypes) as a checker; the
 * product path never links it.
 *
 *  oracle_dequant_matvec_f64: y[r] = sum_c e2m1(nib) * 2^(s[r,c/32]-127) * x[c],
 *    accumulated in double, plus absacc[r] = sum |w*x| — the term-relative
 *    denominator of the reference's unit test (src/test_glm_mxfp4.cu:46-67,
 *    95-105). Low nibble = even column; 0xFF scale -> NaN
 *    (src/test_glm_mxfp4.cu:31-34).
 *  oracle_bf16_matvec_f64: the same for a bf16 [N,K] matrix.
 *  oracle_synth_region: the counter-based generator of
 *    windlass_amd/csrc/synth.hip, restated independently of oracle/synth.py.
 */
#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <string.h>

static const float kE2M1[16] = {0.0f,  0.5f,  1.0f,  1.5f,  2.0f,  3.0f,  4.0f,  6.0f,
                                -0.0f, -0.5f, -1.0f, -1.5f, -2.0f, -3.0f, -4.0f, -6.0f};

static float e8m0(uint8_t b) {
    if (b == 0xFF) return nanf("");
    return ldexpf(1.0f, (int)b - 127);
}

void oracle_dequant_matvec_f64(const uint8_t* W, const uint8_t* S, const float* x, double* y,
                               double* absacc, uint32_t N, uint32_t K) {
    const uint32_t nb = K / 2, ns = K / 32;
    for (uint32_t r = 0; r < N; r++) {
        const uint8_t* wr = W + (size_t)r * nb;
        const uint8_t* sr = S + (size_t)r * ns;
        double acc = 0.0, aacc = 0.0;
        for (uint32_t b = 0; b < nb; b++) {
            const float sc = e8m0(sr[b / 16]);
            const double t0 = (double)(kE2M1[wr[b] & 0xF] * sc) * (double)x[2 * b];
            const double t1 = (double)(kE2M1[wr[b] >> 4] * sc) * (double)x[2 * b + 1];
            acc += t0 + t1;
            aacc += fabs(t0) + fabs(t1);
        }
        y[r] = acc;
        absacc[r] = aacc;
    }
}

static float bf16f(uint16_t b) {
    uint32_t u = (uint32_t)b << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

void oracle_bf16_matvec_f64(const uint16_t* W, const float* x, double* y, double* absacc, uint32_t N,
                            uint32_t K) {
    for (uint32_t r = 0; r < N; r++) {
        double acc = 0.0, aacc = 0.0;
        for (uint32_t c = 0; c < K; c++) {
            const double t = (double)bf16f(W[(size_t)r * K + c]) * (double)x[c];
            acc += t;
            aacc += fabs(t);
        }
        y[r] = acc;
        absacc[r] = aacc;
    }
}

static uint32_t mix32(uint32_t x) {
    x ^= x >> 16;
    x *= 0x7FEB352Du;
    x ^= x >> 15;
    x *= 0x846CA68Bu;
    x ^= x >> 16;
    return x;
}

uint32_t oracle_synth_key(uint32_t seed, uint32_t layer, uint32_t expert) {
    return mix32(mix32(seed ^ 0x9E3779B9u) ^ (layer * 0x85EBCA6Bu + expert * 0xC2B2AE35u + 0x27D4EB2Fu));
}

/* Region r (0..5) of an expert block: weight regions (even r) hold the bytes of
 * word(r, j/4); scale regions (odd r) hold 118 + word(r, j) % 9. */
void oracle_synth_region(uint32_t key, uint32_t r, uint8_t* out, size_t nbytes) {
    const uint32_t salt = mix32(0x632BE5ABu * (r + 1));
    for (size_t j = 0; j < nbytes; j++) {
        if ((r & 1u) == 0) {
            const uint32_t w = mix32(mix32((uint32_t)(j >> 2) ^ salt) ^ key);
            out[j] = (uint8_t)(w >> (8 * (j & 3)));
        } else {
            out[j] = (uint8_t)(118u + mix32(mix32((uint32_t)j ^ salt) ^ key) % 9u);
        }
    }
}
