/*
 * ffn_ref.c -- oracle, TEST INFRASTRUCTURE ONLY (never linked into the product).
 *
 * Independent plain-C restatement of the reference golden FFN
 * (validation/reference.py:16-23) used to pin the torch restatement in
 * oracle/reference.py: both matmuls accumulate in double, the exact GELU uses
 * libm's erf, the rational GELU follows validation/reference.py:5-13 in FP32
 * operation by operation, and the FP32 -> FP16/BF16 casts are written out
 * (round to nearest even, overflow to infinity, NaN kept NaN).
 */
#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <string.h>

static uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* FP32 -> BF16 bits, round to nearest even */
uint16_t ffn_ref_to_bf16(float f) {
    uint32_t u = f2u(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u); /* quiet NaN */
    uint32_t lsb = (u >> 16) & 1u;
    u += 0x7fffu + lsb;
    return (uint16_t)(u >> 16);
}

float ffn_ref_from_bf16(uint16_t h) { return u2f((uint32_t)h << 16); }

/* FP32 -> FP16 bits, round to nearest even, overflow -> inf */
uint16_t ffn_ref_to_fp16(float f) {
    uint32_t u = f2u(f);
    uint32_t sign = (u >> 16) & 0x8000u;
    uint32_t a = u & 0x7fffffffu;
    if (a > 0x7f800000u) return (uint16_t)(sign | 0x7e00u);          /* NaN */
    if (a >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);         /* >= 65520: inf */
    if (a < 0x38800000u) {                                           /* subnormal or zero */
        /* value * 2^24 rounded to nearest even integer = subnormal mantissa */
        float v = u2f(a) * 16777216.0f;                              /* exact scaling */
        float r = nearbyintf(v);                                     /* default mode: RNE */
        return (uint16_t)(sign | (uint32_t)r);
    }
    uint32_t exp = (a >> 23) - 127 + 15;
    uint32_t mant = a & 0x7fffffu;
    uint32_t h = (exp << 10) | (mant >> 13);
    uint32_t rest = mant & 0x1fffu;
    if (rest > 0x1000u || (rest == 0x1000u && (h & 1u))) h += 1;     /* may carry into exp */
    return (uint16_t)(sign | h);
}

float ffn_ref_from_fp16(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu, mant = h & 0x3ffu;
    if (exp == 0) return (sign ? -1.0f : 1.0f) * (float)mant * 5.9604644775390625e-8f; /* 2^-24 */
    if (exp == 31) return u2f(sign | 0x7f800000u | (mant << 13));
    return u2f(sign | ((exp - 15 + 127) << 23) | (mant << 13));
}

/* round each value through the storage type: dtype 0 fp16, 1 bf16 */
void ffn_ref_round(const float* in, float* out, size_t n, int dtype) {
    for (size_t i = 0; i < n; ++i)
        out[i] = dtype ? ffn_ref_from_bf16(ffn_ref_to_bf16(in[i])) : ffn_ref_from_fp16(ffn_ref_to_fp16(in[i]));
}

float ffn_ref_gelu_rational(float z) {
    float t = z * 0.70710678118654752f;
    if (t < -3.92f) t = -3.92f;
    if (t > 3.92f) t = 3.92f;
    float t2 = t * t;
    float p = t2 * 0.053443748819f;
    p = p + 7.5517016694f;
    p = p * t2; p = p + 101.62808918f;
    p = p * t2; p = p + 1393.8061484f;
    p = p * t2; p = p + 5063.7915060f;
    p = p * t2; p = p + 29639.384698f;
    p = p * t;
    float q = t2 + 31.212858877f;
    q = q * t2; q = q + 398.56963806f;
    q = q * t2; q = q + 3023.1248150f;
    q = q * t2; q = q + 13243.365831f;
    q = q * t2; q = q + 26267.224157f;
    float r = p / q;
    float y = 0.5f * z;
    return y * (1.0f + r);
}

double ffn_ref_gelu_erf(double z) { return 0.5 * z * (1.0 + erf(z * 0.70710678118654752440)); }

/*
 * x [m,k], w1 [h,k], w2 [n,h] (already-rounded input values as float) -> out [m,n] (float,
 * before the final cast).  gelu: 0 erf, 1 rational.  stage: -1 keep FP32 hidden, 0/1 round
 * hidden through fp16/bf16.  hidden (optional, [m,h]) receives the activation.
 */
void ffn_ref_run(const float* x, const float* w1, const float* w2, float* hidden, float* out,
                 int m, int k, int h, int n, int gelu, int stage) {
    for (int i = 0; i < m; ++i) {
        for (int j = 0; j < h; ++j) {
            double z = 0.0;
            for (int l = 0; l < k; ++l) z += (double)x[(size_t)i * k + l] * (double)w1[(size_t)j * k + l];
            float a = gelu ? ffn_ref_gelu_rational((float)z) : (float)ffn_ref_gelu_erf((double)(float)z);
            if (stage >= 0) ffn_ref_round(&a, &a, 1, stage);
            if (hidden) hidden[(size_t)i * h + j] = a;
        }
    }
    for (int i = 0; i < m; ++i)
        for (int c = 0; c < n; ++c) {
            double acc = 0.0;
            for (int j = 0; j < h; ++j) {
                double a;
                if (hidden) {
                    a = hidden[(size_t)i * h + j];
                } else {
                    double z = 0.0;
                    for (int l = 0; l < k; ++l) z += (double)x[(size_t)i * k + l] * (double)w1[(size_t)j * k + l];
                    float g = gelu ? ffn_ref_gelu_rational((float)z) : (float)ffn_ref_gelu_erf((double)(float)z);
                    if (stage >= 0) ffn_ref_round(&g, &g, 1, stage);
                    a = g;
                }
                acc += a * (double)w2[(size_t)c * h + j];
            }
            out[(size_t)i * n + c] = (float)acc;
        }
}
