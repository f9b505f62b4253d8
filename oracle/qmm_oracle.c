/*
 * qmm_oracle.c -- CPU restatement of DFlashKit's small-M affine-quantised matmul.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product path may link, load or call
 * this file: it is the reference result that tests/, __graft_entry__.smoke() and
 * the cpu_baseline leg of bench.py compare the HIP kernels against.
 *
 * What it restates (paths relative to the reference repository root):
 *
 *   Sources/DFlashKit/SmallMQuantizedMatmul.swift:56-61   4-bit unpack: code t of word p
 *                                                         is (p >> 4t) & 15, row base
 *                                                         n*(K/8), little-endian in the word
 *   Sources/DFlashKit/SmallMQuantizedMatmul.swift:64-69   8-bit unpack: (p >> 8t) & 255,
 *                                                         row base n*(K/4)
 *   Sources/DFlashKit/SmallMQuantizedMatmul.swift:127-129 group g = k / group_size, scale and
 *                                                         bias at [n*(K/gs) + g], widened to fp32
 *   Sources/DFlashKit/SmallMQuantizedMatmul.swift:59,69   dequant w = (float)code * s + b
 *   Sources/DFlashKit/SmallMQuantizedMatmul.swift:209     y[M,N] = x[M,K] . dequant(W)[N,K]^T
 *   Sources/DFlashKit/SmallMQuantizedMatmul.swift:288-290 optional linear bias added to y
 *   Sources/DFlashKit/SmallMQuantizedMatmul.swift:95-163  the reference kernel's own
 *                                                         accumulation order (orc_qmm_ref_kernel)
 *
 * The MLX affine format itself belongs to mlx-swift 0.31.6 (Package.resolved:14-21), which
 * is not vendored; the unpack / dequant closed forms above are what the reference source
 * fixes, and the tests pin each function here against hand-derived known answers, brute
 * force round trips, closed-form special cases and a library fp64 matmul.
 *
 * Dequant exactness: with bf16/fp16 scales (8 / 11 significant bits) and codes < 256
 * (8 bits), s*q carries at most 19 significant bits, so it is exact in fp32 and the only
 * rounding in s*q + b is the final add -- the result is the same with or without FMA
 * contraction.  orc_dequant is therefore bit-exact and reproducible.
 *
 * dtype codes: 0 = bf16, 1 = fp16, 2 = fp32 (the same values as dfq_dtype).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define ORC_BF16 0
#define ORC_F16 1
#define ORC_F32 2

/* ------------------------------------------------------------------ */
/* 16-bit float conversions (round to nearest even)                    */
/* ------------------------------------------------------------------ */

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

float orc_bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

uint16_t orc_f32_to_bf16(float f) {
    uint32_t u = f2u(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x0040u); /* quiet NaN */
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu;
    uint32_t man = h & 0x3ffu;
    if (exp == 0) {
        /* zero or subnormal: man * 2^-24, exact in fp32 */
        float v = (float)man * 5.9604644775390625e-08f;
        return sign ? -v : v;
    }
    if (exp == 31) return u2f(sign | 0x7f800000u | (man << 13));
    return u2f(sign | ((exp + 112u) << 23) | (man << 13));
}

uint16_t orc_f32_to_f16(float f) {
    uint32_t u = f2u(f);
    uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    uint32_t a = u & 0x7fffffffu;
    if (a > 0x7f800000u) return (uint16_t)(sign | 0x7e00u);          /* NaN */
    if (a >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);         /* >= 65520 rounds to inf */
    if (a < 0x38800000u) {                                           /* below 2^-14: subnormal */
        /* value / 2^-24 rounded to nearest even integer */
        float v = u2f(a) * 16777216.0f;                              /* exact (power of 2) */
        float r = nearbyintf(v);                                     /* default mode: RNE */
        return (uint16_t)(sign | (uint16_t)r);
    }
    uint32_t exp = (a >> 23) - 112u;
    uint32_t man = a & 0x7fffffu;
    uint32_t h = (exp << 10) | (man >> 13);
    uint32_t rem = man & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1u;     /* carries into exp ok */
    return (uint16_t)(sign | h);
}

float orc_load(const void* p, int dt, int64_t i) {
    if (dt == ORC_BF16) return orc_bf16_to_f32(((const uint16_t*)p)[i]);
    if (dt == ORC_F16) return orc_f16_to_f32(((const uint16_t*)p)[i]);
    return ((const float*)p)[i];
}

static int valid_bits(int bits) { return bits == 2 || bits == 4 || bits == 8; }

/* ------------------------------------------------------------------ */
/* Packing (SmallMQuantizedMatmul.swift:56-61, 64-69)                  */
/* ------------------------------------------------------------------ */

/* codes[N][K] (one code per byte) from w[N][K*bits/32]; element t of word p is
 * (p >> bits*t) & (2^bits-1), i.e. element 0 in the low bits. */
int orc_unpack(int bits, const uint32_t* w, int64_t N, int64_t K, uint8_t* codes) {
    if (!valid_bits(bits) || (K * bits) % 32) return -1;
    const int per = 32 / bits;
    const uint32_t mask = (1u << bits) - 1u;
    const int64_t wpr = K / per;
    for (int64_t n = 0; n < N; ++n)
        for (int64_t k = 0; k < K; ++k) {
            uint32_t p = w[n * wpr + k / per];
            codes[n * K + k] = (uint8_t)((p >> (bits * (int)(k % per))) & mask);
        }
    return 0;
}

int orc_pack(int bits, const uint8_t* codes, int64_t N, int64_t K, uint32_t* w) {
    if (!valid_bits(bits) || (K * bits) % 32) return -1;
    const int per = 32 / bits;
    const uint32_t mask = (1u << bits) - 1u;
    const int64_t wpr = K / per;
    for (int64_t n = 0; n < N; ++n)
        for (int64_t j = 0; j < wpr; ++j) {
            uint32_t p = 0;
            for (int t = 0; t < per; ++t)
                p |= ((uint32_t)codes[n * K + j * per + t] & mask) << (bits * t);
            w[n * wpr + j] = p;
        }
    return 0;
}

/* ------------------------------------------------------------------ */
/* Dequant (SmallMQuantizedMatmul.swift:59, 69, 127-129)               */
/* ------------------------------------------------------------------ */

int orc_dequant(int bits, int gs, const uint32_t* w, const void* scales, const void* biases,
                int sdt, int64_t N, int64_t K, float* out) {
    if (!valid_bits(bits) || gs <= 0 || K % gs || (K * bits) % 32) return -1;
    const int per = 32 / bits;
    const uint32_t mask = (1u << bits) - 1u;
    const int64_t wpr = K / per, gpr = K / gs;
    for (int64_t n = 0; n < N; ++n)
        for (int64_t k = 0; k < K; ++k) {
            uint32_t p = w[n * wpr + k / per];
            float q = (float)((p >> (bits * (int)(k % per))) & mask);
            float s = orc_load(scales, sdt, n * gpr + k / gs);
            float b = orc_load(biases, sdt, n * gpr + k / gs);
            volatile float sq = q * s; /* exact; volatile keeps the add un-contracted */
            out[n * K + k] = sq + b;
        }
    return 0;
}

/* ------------------------------------------------------------------ */
/* fp64 reference matmul (SmallMQuantizedMatmul.swift:209, 288-290)    */
/* ------------------------------------------------------------------ */

/* y[m][n] = sum_k x[m][k] * (s[n][k/gs]*q[n][k] + b[n][k/gs])  (+ lbias[n]), all in fp64. */
int orc_qmm_f64(int64_t M, int64_t N, int64_t K, int bits, int gs, const void* x, int xdt,
                const uint32_t* w, const void* scales, const void* biases, int sdt,
                const void* lbias, int lbdt, double* y) {
    if (!valid_bits(bits) || gs <= 0 || K % gs || (K * bits) % 32 || M < 0 || N < 0) return -1;
    const int per = 32 / bits;
    const uint32_t mask = (1u << bits) - 1u;
    const int64_t wpr = K / per, gpr = K / gs;
    double* xd = (double*)malloc(sizeof(double) * (size_t)(M * K > 0 ? M * K : 1));
    if (!xd) return -2;
    for (int64_t i = 0; i < M * K; ++i) xd[i] = (double)orc_load(x, xdt, i);
#pragma omp parallel for schedule(static)
    for (int64_t n = 0; n < N; ++n) {
        double* acc = (double*)calloc((size_t)(M > 0 ? M : 1), sizeof(double));
        double* wrow = (double*)malloc(sizeof(double) * (size_t)K);
        for (int64_t k = 0; k < K; ++k) {
            uint32_t p = w[n * wpr + k / per];
            double q = (double)((p >> (bits * (int)(k % per))) & mask);
            double s = (double)orc_load(scales, sdt, n * gpr + k / gs);
            double b = (double)orc_load(biases, sdt, n * gpr + k / gs);
            wrow[k] = s * q + b;
        }
        for (int64_t m = 0; m < M; ++m) {
            double a = 0.0;
            const double* xr = xd + m * K;
            for (int64_t k = 0; k < K; ++k) a += xr[k] * wrow[k];
            acc[m] = a;
        }
        double lb = lbias ? (double)orc_load(lbias, lbdt, n) : 0.0;
        for (int64_t m = 0; m < M; ++m) y[m * N + n] = acc[m] + lb;
        free(acc);
        free(wrow);
    }
    free(xd);
    return 0;
}

/* ------------------------------------------------------------------ */
/* fp32 restatement with MLX's semantics: dequantise a group, then     */
/* multiply-accumulate in fp32 (the CPU baseline algorithm).           */
/* ------------------------------------------------------------------ */

int orc_qmm_f32(int64_t M, int64_t N, int64_t K, int bits, int gs, const void* x, int xdt,
                const uint32_t* w, const void* scales, const void* biases, int sdt,
                int nthreads, float* y) {
    if (!valid_bits(bits) || gs <= 0 || gs > 256 || K % gs || (K * bits) % 32 || M < 0 ||
        M > 64)
        return -1;
    const int per = 32 / bits;
    const uint32_t mask = (1u << bits) - 1u;
    const int64_t wpr = K / per, gpr = K / gs;
    float* xf = (float*)malloc(sizeof(float) * (size_t)(M * K > 0 ? M * K : 1));
    if (!xf) return -2;
    for (int64_t i = 0; i < M * K; ++i) xf[i] = orc_load(x, xdt, i);
#ifdef _OPENMP
    if (nthreads > 0) omp_set_num_threads(nthreads);
#else
    (void)nthreads;
#endif
#pragma omp parallel for schedule(static)
    for (int64_t n = 0; n < N; ++n) {
        float acc[64];
        float wg[256];
        for (int64_t m = 0; m < M; ++m) acc[m] = 0.0f;
        for (int64_t g = 0; g < gpr; ++g) {
            const float s = orc_load(scales, sdt, n * gpr + g);
            const float b = orc_load(biases, sdt, n * gpr + g);
            for (int j = 0; j < gs; ++j) {
                int64_t k = g * gs + j;
                uint32_t p = w[n * wpr + k / per];
                wg[j] = (float)((p >> (bits * (int)(k % per))) & mask) * s + b;
            }
            for (int64_t m = 0; m < M; ++m) {
                const float* xr = xf + m * K + g * gs;
                float a = acc[m];
                for (int j = 0; j < gs; ++j) a += xr[j] * wg[j];
                acc[m] = a;
            }
        }
        for (int64_t m = 0; m < M; ++m) y[m * N + n] = acc[m];
    }
    free(xf);
    return 0;
}

/* ------------------------------------------------------------------ */
/* The reference kernel's arithmetic (SmallMQuantizedMatmul.swift:95-163) */
/* ------------------------------------------------------------------ */

/* Restates the Metal kernel's accumulation structure for M <= 16, group 64, bits 4/8,
 * K % 512 == 0: the dequantised weight is rounded to bf16 before the MMA (:59, :69); K is
 * split into 8 slices of K/8 (:96, :118); each slice accumulates 64-k steps of eight 8-k
 * MMA sub-steps into an fp32 tile (:119-143); the 8 slice partials are summed in order
 * q = 0..7 (:160) and rounded to bf16 (:161).  The order of the 8 products inside one
 * simdgroup MMA is not specified by Metal; they are summed here in k order, so this
 * function pins the structure, not the last bit, of the Apple kernel. */
int orc_qmm_ref_kernel(int64_t M, int64_t N, int64_t K, int bits, const void* x, int xdt,
                       const uint32_t* w, const void* scales, const void* biases, int sdt,
                       uint16_t* y_bf16) {
    const int gs = 64;
    if ((bits != 4 && bits != 8) || K % 512 || M < 1 || M > 16) return -1;
    const int per = 32 / bits;
    const uint32_t mask = (1u << bits) - 1u;
    const int64_t wpr = K / per, gpr = K / gs, kps = K / 8;
#pragma omp parallel for schedule(static)
    for (int64_t n = 0; n < N; ++n) {
        float part[8][16];
        for (int q = 0; q < 8; ++q) {
            for (int m = 0; m < 16; ++m) part[q][m] = 0.0f;
            for (int64_t kk = 0; kk < kps; kk += 64) {
                int64_t ka = q * kps + kk;
                const float s = orc_load(scales, sdt, n * gpr + (ka >> 6));
                const float b = orc_load(biases, sdt, n * gpr + (ka >> 6));
                for (int kt = 0; kt < 8; ++kt)
                    for (int m = 0; m < M; ++m) {
                        float sub = 0.0f;
                        for (int e = 0; e < 8; ++e) {
                            int64_t k = ka + kt * 8 + e;
                            uint32_t p = w[n * wpr + k / per];
                            float q8 = (float)((p >> (bits * (int)(k % per))) & mask);
                            float wb = orc_bf16_to_f32(orc_f32_to_bf16(q8 * s + b));
                            float xv = orc_bf16_to_f32(orc_f32_to_bf16(orc_load(x, xdt, m * K + k)));
                            sub += xv * wb;
                        }
                        part[q][m] += sub;
                    }
            }
        }
        for (int m = 0; m < M; ++m) {
            float v = 0.0f;
            for (int q = 0; q < 8; ++q) v += part[q][m];
            y_bf16[m * N + n] = orc_f32_to_bf16(v);
        }
    }
    return 0;
}

/* Round an fp64 result to the output dtype. */
int orc_round_output(const double* y, int64_t count, int ydt, void* out) {
    for (int64_t i = 0; i < count; ++i) {
        float f = (float)y[i];
        if (ydt == ORC_BF16) ((uint16_t*)out)[i] = orc_f32_to_bf16(f);
        else if (ydt == ORC_F16) ((uint16_t*)out)[i] = orc_f32_to_f16(f);
        else ((float*)out)[i] = f;
    }
    return 0;
}

int orc_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
