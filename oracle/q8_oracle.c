/*
 * q8_oracle.c -- CPU restatement of the reference's INT8 group-quantized,
 * weight-only (W8A32) linear-layer path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker: it may be built and
 * called by tests/, by __graft_entry__.smoke() and by bench.py's cpu_baseline
 * leg, and by nothing else.  The product path (libq8hip.so) never links,
 * loads or calls it.
 *
 * Every function cites the reference file:line it restates.  Reference
 * citations are relative to the plutonium-guy/lama32_mojo source tree.
 *
 * Packed row layout (qwen3_mojo/scripts/quantize.py:4-12, src/llama_q8.mojo:3-9):
 *     [ (m/G) scales | m int8 codes ]
 * stored as little-endian u16 elements.  The reference layout is G=64 with
 * f16 scales (rowstride m/64 + m/2 u16, src/llama_q8.mojo:26-28).  The same
 * code also covers G=32 with f32 scales (each f32 scale occupies two u16),
 * where the scale is kept in f32 instead of being rounded to f16.
 *
 * Pinning (what checks this file): tests/test_oracle.py compares it against
 * golden vectors written by the reference's own pack_q8, against an
 * independent numpy restatement, against numpy's float16 conversion on every
 * rounding boundary, and against closed forms (one-hot inputs, zero inputs,
 * float64 dequantised matmul, linearity).
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#define Q8O_SCALE_F16 1
#define Q8O_SCALE_F32 2

/* ----------------------------------------------------------------------- */
/* Scalar format conversions                                                */
/* ----------------------------------------------------------------------- */

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* f32 -> IEEE binary16, round to nearest even, subnormals kept, overflow to
 * inf.  This is numpy's astype(np.float16) (quantize.py:37). */
uint16_t q8o_f32_to_f16(float f)
{
    uint32_t x = f2u(f);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    uint32_t ax = x & 0x7fffffffu;
    if (ax > 0x7f800000u)                      /* NaN: keep it quiet */
        return (uint16_t)(sign | 0x7e00u | ((ax >> 13) & 0x3ffu));
    if (ax >= 0x477ff000u)                     /* >= 65520 rounds to inf */
        return (uint16_t)(sign | 0x7c00u);
    if (ax >= 0x38800000u) {                   /* normal f16 range, >= 2^-14 */
        uint32_t mant = ax & 0x7fffffu;
        uint32_t e = (ax >> 23) - 127u + 15u;
        uint32_t h = (e << 10) | (mant >> 13);
        uint32_t rem = mant & 0x1fffu;
        if (rem > 0x1000u || (rem == 0x1000u && (h & 1u)))
            h++;                               /* carry may bump the exponent */
        return (uint16_t)(sign | h);
    }
    if (ax <= 0x33000000u)                     /* <= 2^-25: ties-to-even gives 0 */
        return sign;
    /* f16 subnormal: value / 2^-24 rounded to an integer */
    int32_t E = (int32_t)(ax >> 23) - 127;     /* -25 .. -15 */
    uint32_t m24 = (ax & 0x7fffffu) | 0x800000u;
    int shift = -E - 1;                        /* 14 .. 24 */
    uint32_t h = m24 >> shift;
    uint32_t rem = m24 & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (h & 1u)))
        h++;
    return (uint16_t)(sign | h);
}

/* binary16 -> f32, exact (src/llama_q8.mojo:31-35). */
float q8o_f16_to_f32(uint16_t h)
{
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t e = ((uint32_t)h >> 10) & 0x1fu;
    uint32_t m = (uint32_t)h & 0x3ffu;
    if (e == 0) {
        float v = (float)m * 5.9604644775390625e-08f;   /* m * 2^-24, exact */
        return u2f(f2u(v) | sign);
    }
    if (e == 31)
        return u2f(sign | 0x7f800000u | (m << 13));
    return u2f(sign | ((e - 15u + 127u) << 23) | (m << 13));
}

/* bf16 bits -> f32, exact (torch Tensor.float() at quantize.py:34). */
float q8o_bf16_to_f32(uint16_t b) { return u2f((uint32_t)b << 16); }

/* f32 -> bf16, round to nearest even (torch's to(bfloat16)); used to build
 * bf16 synthetic weights and activations the same way on every side. */
uint16_t q8o_f32_to_bf16(float f)
{
    uint32_t x = f2u(f);
    if ((x & 0x7fffffffu) > 0x7f800000u)
        return (uint16_t)((x >> 16) | 0x40u);
    uint32_t lsb = (x >> 16) & 1u;
    x += 0x7fffu + lsb;
    return (uint16_t)(x >> 16);
}

/* ----------------------------------------------------------------------- */
/* Layout helpers                                                           */
/* ----------------------------------------------------------------------- */

static inline int scale_u16(int kind) { return kind == Q8O_SCALE_F32 ? 2 : 1; }

/* Packed row length in u16 elements (src/llama_q8.mojo:26-28 for G=64/f16). */
int64_t q8o_rowstride_u16(int64_t m, int G, int kind)
{
    return (m / G) * scale_u16(kind) + m / 2;
}

/* Scale of group g of a packed row, as f32. */
static inline float row_scale(const uint16_t *row, int64_t g, int kind)
{
    if (kind == Q8O_SCALE_F32) {
        uint32_t u = (uint32_t)row[2 * g] | ((uint32_t)row[2 * g + 1] << 16);
        return u2f(u);
    }
    return q8o_f16_to_f32(row[g]);
}

static inline const int8_t *row_codes(const uint16_t *row, int64_t m, int G, int kind)
{
    return (const int8_t *)(row + (m / G) * scale_u16(kind));
}

/* ----------------------------------------------------------------------- */
/* pack_q8 (qwen3_mojo/scripts/quantize.py:31-43)                           */
/* ----------------------------------------------------------------------- */

/* Quantize one group of G f32 weights.  Steps follow quantize.py:36-39:
 *   scale = max|w| / 127            (f32 division, :36)
 *   scale = max(scale, f32(1e-8))   (f32, :37) then RNE to f16 (:37)
 *   q     = rint(w / f32(scale16))  (f32 division, half-to-even, :38)
 *   q     = clip(q, -127, 127) -> int8 (:39); NaN (0/0 when scale16 == 0)
 *           converts to 0, which is what numpy's float->int8 cast gives.
 * With kind == Q8O_SCALE_F32 the scale stays f32 (no f16 rounding). */
static void pack_group(const float *w, int G, int kind, uint16_t *scale_out,
                       int8_t *q_out)
{
    float amax = 0.0f;
    for (int k = 0; k < G; ++k) {
        float a = fabsf(w[k]);
        if (a > amax || isnan(a))         /* np.max propagates NaN */
            amax = isnan(amax) ? amax : a;
    }
    float sc = amax / 127.0f;
    const float floor_ = 1e-8f;
    if (!(sc >= floor_))              /* np.maximum: NaN stays NaN */
        sc = isnan(sc) ? sc : floor_;
    float sf;
    if (kind == Q8O_SCALE_F32) {
        sf = sc;
        uint32_t u = f2u(sf);
        scale_out[0] = (uint16_t)(u & 0xffffu);
        scale_out[1] = (uint16_t)(u >> 16);
    } else {
        uint16_t s16 = q8o_f32_to_f16(sc);
        scale_out[0] = s16;
        sf = q8o_f16_to_f32(s16);
    }
    for (int k = 0; k < G; ++k) {
        float r = w[k] / sf;
        float qr = nearbyintf(r);          /* current mode = nearest-even */
        int8_t c;
        if (isnan(qr))
            c = 0;
        else if (qr > 127.0f)
            c = 127;
        else if (qr < -127.0f)
            c = -127;
        else
            c = (int8_t)qr;
        q_out[k] = c;
    }
}

/* Pack an f32 weight matrix [n, m] into rows of q8o_rowstride_u16(m) u16.
 * Returns 0, or -1 for an unsupported shape (quantize.py:33 asserts
 * m % GROUP == 0 and m even). */
int q8o_pack_f32(const float *w, int64_t n, int64_t m, int G, int kind,
                 uint16_t *out)
{
    if (n < 0 || m <= 0 || G <= 0 || m % G != 0 || m % 2 != 0)
        return -1;
    if (kind != Q8O_SCALE_F16 && kind != Q8O_SCALE_F32)
        return -1;
    int64_t rs = q8o_rowstride_u16(m, G, kind);
    int64_t ng = m / G;
    int su = scale_u16(kind);
    for (int64_t j = 0; j < n; ++j) {
        uint16_t *row = out + j * rs;
        int8_t *codes = (int8_t *)(row + ng * su);
        for (int64_t g = 0; g < ng; ++g)
            pack_group(w + j * m + g * G, G, kind, row + g * su, codes + g * G);
    }
    return 0;
}

/* Same, for bf16 weights (the reference's input dtype; w.float() is exact). */
int q8o_pack_bf16(const uint16_t *w, int64_t n, int64_t m, int G, int kind,
                  uint16_t *out)
{
    if (n < 0 || m <= 0 || G <= 0 || m % G != 0 || m % 2 != 0 || G > 4096)
        return -1;
    if (kind != Q8O_SCALE_F16 && kind != Q8O_SCALE_F32)
        return -1;
    int64_t rs = q8o_rowstride_u16(m, G, kind);
    int64_t ng = m / G;
    int su = scale_u16(kind);
    float buf[4096];
    for (int64_t j = 0; j < n; ++j) {
        uint16_t *row = out + j * rs;
        int8_t *codes = (int8_t *)(row + ng * su);
        for (int64_t g = 0; g < ng; ++g) {
            for (int k = 0; k < G; ++k)
                buf[k] = q8o_bf16_to_f32(w[j * m + g * G + k]);
            pack_group(buf, G, kind, row + g * su, codes + g * G);
        }
    }
    return 0;
}

/* ----------------------------------------------------------------------- */
/* Linear y[s,n] = x[s,m] . deq(W[n,m])^T  (src/llama_q8.mojo:54-93)         */
/* ----------------------------------------------------------------------- */

/* float64 closed form: y[i,j] = sum_g s[j,g] * sum_{k in g} x[i,k] * q[j,k].
 * Every product is exact in float64; this is the parity reference.  Each
 * output is summed on its own in a fixed order, so the OpenMP split over
 * outputs does not change any result. */
void q8o_linear_f64(const uint16_t *wpk, const float *x, int64_t s, int64_t m,
                    int64_t n, int G, int kind, double *y)
{
    int64_t rs = q8o_rowstride_u16(m, G, kind);
    int64_t ng = m / G;
#pragma omp parallel for schedule(static)
    for (int64_t t = 0; t < s * n; ++t) {
        const int64_t i = t / n, j = t % n;
        const float *xi = x + i * m;
        const uint16_t *row = wpk + j * rs;
        const int8_t *q = row_codes(row, m, G, kind);
        double acc = 0.0;
        for (int64_t g = 0; g < ng; ++g) {
            double part = 0.0;
            for (int k = 0; k < G; ++k)
                part += (double)xi[g * G + k] * (double)q[g * G + k];
            acc += (double)row_scale(row, g, kind) * part;
        }
        y[t] = acc;
    }
}

/* The same float64 closed form for float64 inputs (the model oracle's
 * activations are float64 between its layers): y[i,j] = sum_g s[j,g] *
 * sum_{k in g} x[i,k] * q[j,k], every product and sum in float64. */
void q8o_linear_f64x(const uint16_t *wpk, const double *x, int64_t s, int64_t m,
                     int64_t n, int G, int kind, double *y)
{
    int64_t rs = q8o_rowstride_u16(m, G, kind);
    int64_t ng = m / G;
#pragma omp parallel for schedule(static)
    for (int64_t t = 0; t < s * n; ++t) {
        const int64_t i = t / n, j = t % n;
        const double *xi = x + i * m;
        const uint16_t *row = wpk + j * rs;
        const int8_t *q = row_codes(row, m, G, kind);
        double acc = 0.0;
        for (int64_t g = 0; g < ng; ++g) {
            double part = 0.0;
            for (int k = 0; k < G; ++k)
                part += xi[g * G + k] * (double)q[g * G + k];
            acc += (double)row_scale(row, g, kind) * part;
        }
        y[t] = acc;
    }
}

/* Group-major fp32 restatement of k_mm_q8's arithmetic (src/llama_q8.mojo:73-93):
 * 32 lanes (TG_MM) stride over groups; per group a 16-wide fp32 fma chain
 * over 16-element chunks gives the unscaled dot, reduced and scaled once
 * (:76-84); the 32 lane partials are then summed in 4-wide steps (:85-93).
 * Used as the timed CPU baseline; OpenMP over output rows when enabled. */
void q8o_linear_f32(const uint16_t *wpk, const float *x, int64_t s, int64_t m,
                    int64_t n, int G, int kind, float *y)
{
    int64_t rs = q8o_rowstride_u16(m, G, kind);
    int64_t ng = m / G;
    int chunks = G / 16;
    for (int64_t i = 0; i < s; ++i) {
        const float *xi = x + i * m;
#pragma omp parallel for schedule(static)
        for (int64_t j = 0; j < n; ++j) {
            const uint16_t *row = wpk + j * rs;
            const int8_t *q = row_codes(row, m, G, kind);
            float lane[32];
            for (int t = 0; t < 32; ++t) {
                float acc = 0.0f;
                for (int64_t g = t; g < ng; g += 32) {
                    int64_t k = g * G;
                    float gacc[16];
                    for (int l = 0; l < 16; ++l)
                        gacc[l] = 0.0f;
                    for (int c = 0; c < chunks; ++c)
                        for (int l = 0; l < 16; ++l)
                            gacc[l] = fmaf(xi[k + 16 * c + l],
                                           (float)q[k + 16 * c + l], gacc[l]);
                    float r = 0.0f;
                    for (int l = 0; l < 16; ++l)
                        r += gacc[l];
                    acc += row_scale(row, g, kind) * r;
                }
                lane[t] = acc;
            }
            float tot[4] = {0.0f, 0.0f, 0.0f, 0.0f};
            for (int qd = 0; qd < 32; qd += 4)
                for (int l = 0; l < 4; ++l)
                    tot[l] += lane[qd + l];
            y[i * n + j] = (tot[0] + tot[1]) + (tot[2] + tot[3]);
        }
    }
}

/* OpenMP threads for the parallel loops above (the CPU baseline runs the
 * fp32 restatement on all host cores and on one). */
#ifdef _OPENMP
#include <omp.h>
void q8o_set_threads(int n) { omp_set_num_threads(n > 0 ? n : 1); }
int q8o_get_threads(void) { return omp_get_max_threads(); }
#else
void q8o_set_threads(int n) { (void)n; }
int q8o_get_threads(void) { return 1; }
#endif

/* ----------------------------------------------------------------------- */
/* Embedding gather (src/llama_q8.mojo:96-109)                              */
/* ----------------------------------------------------------------------- */

/* y[i,c] = f32(int8 q[id_i, c]) * f32(scale[id_i, c/G]); one f32 rounding. */
void q8o_embed_gather(const uint16_t *wpk, const int32_t *ids, int64_t s,
                      int64_t d, int G, int kind, float *y)
{
    int64_t rs = q8o_rowstride_u16(d, G, kind);
    for (int64_t i = 0; i < s; ++i) {
        const uint16_t *row = wpk + (int64_t)ids[i] * rs;
        const int8_t *q = row_codes(row, d, G, kind);
        for (int64_t c = 0; c < d; ++c)
            y[i * d + c] = (float)q[c] * row_scale(row, c / G, kind);
    }
}

/* Array forms of the format conversions, for exhaustive checks. */
void q8o_f32_to_f16_array(const float *x, int64_t n, uint16_t *out)
{
    for (int64_t i = 0; i < n; ++i)
        out[i] = q8o_f32_to_f16(x[i]);
}

void q8o_f16_to_f32_array(const uint16_t *h, int64_t n, float *out)
{
    for (int64_t i = 0; i < n; ++i)
        out[i] = q8o_f16_to_f32(h[i]);
}
