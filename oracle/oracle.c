/*
 * CPU oracle (test infrastructure only) -- see oracle.h for the contract and
 * the reference citations.  Built with -ffp-contract=off so every fp32
 * expression rounds exactly as written.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif
#include <time.h>

/* ------------------------------------------------------------------------- */
/* fp16 conversion                                                            */
/* ------------------------------------------------------------------------- */

uint16_t or_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u) {                       /* inf / nan */
        if (ax == 0x7F800000u) return (uint16_t)(sign | 0x7C00u);
        return (uint16_t)(sign | 0x7E00u | ((ax >> 13) & 0x3FFu));
    }
    if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u);   /* >= 65520 -> inf */
    if (ax >= 0x38800000u) {                       /* normal half: |f| >= 2^-14 */
        uint32_t r = ax - 0x38000000u;             /* rebias 127 -> 15 */
        uint32_t h = r >> 13, rem = r & 0x1FFFu;
        if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
        return (uint16_t)(sign | h);
    }
    if (ax < 0x33000000u) return (uint16_t)sign;   /* |f| <= 2^-25 -> 0 (tie to even) */
    uint32_t e = ax >> 23;                         /* 102 .. 112 */
    uint32_t m = (ax & 0x7FFFFFu) | 0x800000u;
    uint32_t shift = 126u - e;                     /* units of 2^-24 */
    uint32_t h = m >> shift, rem = m & ((1u << shift) - 1u), hw = 1u << (shift - 1u);
    if (rem > hw || (rem == hw && (h & 1u))) h++;
    return (uint16_t)(sign | h);
}

float or_f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t e = ((uint32_t)h >> 10) & 0x1Fu, m = (uint32_t)h & 0x3FFu, x;
    float f;
    if (e == 0) {
        f = (float)m * 5.9604644775390625e-8f;     /* m * 2^-24, exact */
        memcpy(&x, &f, 4);
        x |= sign;
    } else if (e == 31) {
        x = sign | 0x7F800000u | (m << 13);
    } else {
        x = sign | ((e + 112u) << 23) | (m << 13);
    }
    memcpy(&f, &x, 4);
    return f;
}

void or_f32_to_f16_array(const float* in, uint16_t* out, size_t n) {
    for (size_t i = 0; i < n; i++) out[i] = or_f32_to_f16(in[i]);
}
void or_f16_to_f32_array(const uint16_t* in, float* out, size_t n) {
    for (size_t i = 0; i < n; i++) out[i] = or_f16_to_f32(in[i]);
}

/* ------------------------------------------------------------------------- */
/* generator                                                                  */
/* ------------------------------------------------------------------------- */

static uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

uint64_t or_rand(uint64_t seed, uint64_t stream, uint64_t index) {
    uint64_t s = mix64(seed + 0x9E3779B97F4A7C15ull * (stream + 1));
    return mix64(s + 0x9E3779B97F4A7C15ull * (index + 1));
}

uint16_t or_unif_f16(uint64_t draw, float lo, float hi) {
    double u = (double)(draw >> 40) * (1.0 / 16777216.0);   /* [0,1), 24 bits */
    double v = (double)lo + ((double)hi - (double)lo) * u;
    return or_f32_to_f16((float)v);
}

static inline uint8_t q4_0_code(uint64_t seed, int64_t b, int e) {
    uint64_t w = or_rand(seed, 2, (uint64_t)(2 * b + e / 16));
    return (uint8_t)((w >> (4 * (e % 16))) & 0xF);
}

void or_gen_q4_0_planes(uint64_t seed, int N, int K, float dlo, float dhi,
                        uint8_t* Wq, uint16_t* Ws) {
    int nb = K / 32;
#pragma omp parallel for schedule(static)
    for (int n = 0; n < N; n++) {
        for (int j = 0; j < nb; j++) {
            int64_t b = (int64_t)n * nb + j;
            Ws[b] = or_unif_f16(or_rand(seed, 1, (uint64_t)b), dlo, dhi);
            for (int i = 0; i < 16; i++) {              /* byte i: elems 2i (lo), 2i+1 (hi) */
                uint8_t lo = q4_0_code(seed, b, 2 * i), hi = q4_0_code(seed, b, 2 * i + 1);
                Wq[(size_t)n * (K / 2) + (size_t)j * 16 + i] = (uint8_t)(lo | (hi << 4));
            }
        }
    }
}

void or_gen_q4_0_blocks(uint64_t seed, int N, int K, float dlo, float dhi, uint8_t* blocks) {
    int nb = K / 32;
#pragma omp parallel for schedule(static)
    for (int n = 0; n < N; n++) {
        for (int j = 0; j < nb; j++) {
            int64_t b = (int64_t)n * nb + j;
            uint8_t* blk = blocks + (size_t)b * 18;
            uint16_t d = or_unif_f16(or_rand(seed, 1, (uint64_t)b), dlo, dhi);
            blk[0] = (uint8_t)(d & 0xFF);
            blk[1] = (uint8_t)(d >> 8);
            for (int i = 0; i < 16; i++) {              /* qs[i]: elems i (lo), i+16 (hi) */
                uint8_t lo = q4_0_code(seed, b, i), hi = q4_0_code(seed, b, i + 16);
                blk[2 + i] = (uint8_t)(lo | (hi << 4));
            }
        }
    }
}

void or_gen_q4_k(uint64_t seed, int N, int K, float lo, float hi, uint8_t* blocks) {
    int64_t nblk = (int64_t)N * (K / 256);
#pragma omp parallel for schedule(static)
    for (int64_t b = 0; b < nblk; b++) {
        uint8_t* blk = blocks + (size_t)b * 144;
        uint16_t d = or_unif_f16(or_rand(seed, 1, (uint64_t)b), lo, hi);
        uint16_t dm = or_unif_f16(or_rand(seed, 3, (uint64_t)b), lo, hi);
        blk[0] = (uint8_t)(d & 0xFF);  blk[1] = (uint8_t)(d >> 8);
        blk[2] = (uint8_t)(dm & 0xFF); blk[3] = (uint8_t)(dm >> 8);
        uint64_t s0 = or_rand(seed, 4, (uint64_t)(2 * b)), s1 = or_rand(seed, 4, (uint64_t)(2 * b + 1));
        for (int i = 0; i < 8; i++) blk[4 + i] = (uint8_t)(s0 >> (8 * i));
        for (int i = 0; i < 4; i++) blk[12 + i] = (uint8_t)(s1 >> (8 * i));
        for (int w = 0; w < 16; w++) {
            uint64_t q = or_rand(seed, 2, (uint64_t)(16 * b + w));
            for (int i = 0; i < 8; i++) blk[16 + 8 * w + i] = (uint8_t)(q >> (8 * i));
        }
    }
}

void or_gen_act(uint64_t seed, int M, int K, uint16_t* A) {
    int64_t total = (int64_t)M * K;
    int64_t npairs = (total + 1) / 2;
#pragma omp parallel for schedule(static)
    for (int64_t p = 0; p < npairs; p++) {
        uint64_t a = or_rand(seed, 5, (uint64_t)(2 * p)), b = or_rand(seed, 5, (uint64_t)(2 * p + 1));
        double u1 = ((double)(a >> 11) + 1.0) * (1.0 / 9007199254740992.0);   /* (0,1] */
        double u2 = (double)(b >> 11) * (1.0 / 9007199254740992.0);           /* [0,1) */
        double r = sqrt(-2.0 * log(u1)), t = 6.283185307179586 * u2;
        A[2 * p] = or_f32_to_f16((float)(r * cos(t)));
        if (2 * p + 1 < total) A[2 * p + 1] = or_f32_to_f16((float)(r * sin(t)));
    }
}

/* ------------------------------------------------------------------------- */
/* format helpers                                                             */
/* ------------------------------------------------------------------------- */

/* ggml get_scale_min_k4: 8 six-bit (scale, min) pairs in 12 bytes. */
void or_q4k_get_scale_min(int j, const uint8_t* q, uint8_t* sc, uint8_t* m) {
    if (j < 4) {
        *sc = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *sc = (uint8_t)((q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4));
        *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

/* Writes the 12 bytes from the low-to-high bit allocation of the format:
 *   bytes 0-3 : sc[0..3] in bits 0-5, bits 4-5 of sc[4..7] in bits 6-7
 *   bytes 4-7 : m[0..3]  in bits 0-5, bits 4-5 of m[4..7]  in bits 6-7
 *   bytes 8-11: bits 0-3 of sc[4..7] low nibble, bits 0-3 of m[4..7] high nibble */
void or_q4k_pack_scales(const uint8_t* sc, const uint8_t* m, uint8_t* s) {
    for (int i = 0; i < 4; i++) {
        s[i] = (uint8_t)((sc[i] & 63) | (((sc[i + 4] >> 4) & 3) << 6));
        s[i + 4] = (uint8_t)((m[i] & 63) | (((m[i + 4] >> 4) & 3) << 6));
        s[i + 8] = (uint8_t)((sc[i + 4] & 0xF) | ((m[i + 4] & 0xF) << 4));
    }
}

void or_q4_0_planes_to_blocks(const uint8_t* Wq, const uint16_t* Ws, int N, int K, uint8_t* blocks) {
    int nb = K / 32;
    for (int64_t b = 0; b < (int64_t)N * nb; b++) {
        int64_t n = b / nb, j = b % nb;
        const uint8_t* src = Wq + (size_t)n * (K / 2) + (size_t)j * 16;
        uint8_t* blk = blocks + (size_t)b * 18;
        blk[0] = (uint8_t)(Ws[b] & 0xFF);
        blk[1] = (uint8_t)(Ws[b] >> 8);
        uint8_t q[32];
        for (int i = 0; i < 16; i++) { q[2 * i] = src[i] & 0xF; q[2 * i + 1] = src[i] >> 4; }
        for (int i = 0; i < 16; i++) blk[2 + i] = (uint8_t)(q[i] | (q[i + 16] << 4));
    }
}

void or_q4_0_blocks_to_planes(const uint8_t* blocks, int N, int K, uint8_t* Wq, uint16_t* Ws) {
    int nb = K / 32;
    for (int64_t b = 0; b < (int64_t)N * nb; b++) {
        int64_t n = b / nb, j = b % nb;
        const uint8_t* blk = blocks + (size_t)b * 18;
        uint8_t* dst = Wq + (size_t)n * (K / 2) + (size_t)j * 16;
        Ws[b] = (uint16_t)(blk[0] | (blk[1] << 8));
        uint8_t q[32];
        for (int i = 0; i < 16; i++) { q[i] = blk[2 + i] & 0xF; q[i + 16] = blk[2 + i] >> 4; }
        for (int i = 0; i < 16; i++) dst[i] = (uint8_t)(q[2 * i] | (q[2 * i + 1] << 4));
    }
}

/* ------------------------------------------------------------------------- */
/* dequant                                                                    */
/* ------------------------------------------------------------------------- */

static inline uint16_t rd16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* one row of N, fp32 values exactly as the reference builds refW */
static void dequant_row_f32(int qtype, const void* W, const void* W_aux, int K, int64_t n, float* y) {
    if (qtype == OR_Q4_0_PLANES) {
        /* kernels/busfill_v0.cu:119-125: byte j of block = elems 2j (lo), 2j+1 (hi) */
        const uint8_t* q = (const uint8_t*)W + (size_t)n * (K / 2);
        const uint16_t* s = (const uint16_t*)W_aux + (size_t)n * (K / 32);
        for (int j = 0; j < K / 32; j++) {
            float d = or_f16_to_f32(s[j]);
            for (int i = 0; i < 16; i++) {
                uint8_t b = q[j * 16 + i];
                y[j * 32 + 2 * i] = (float)((int)(b & 0xF) - 8) * d;
                y[j * 32 + 2 * i + 1] = (float)((int)(b >> 4) - 8) * d;
            }
        }
    } else if (qtype == OR_Q4_0) {
        /* ggml dequantize_row_q4_0: elem j = qs[j]&0xF, elem j+16 = qs[j]>>4 */
        const uint8_t* blk = (const uint8_t*)W + (size_t)n * (K / 32) * 18;
        for (int j = 0; j < K / 32; j++, blk += 18) {
            float d = or_f16_to_f32(rd16(blk));
            for (int i = 0; i < 16; i++) {
                uint8_t b = blk[2 + i];
                y[j * 32 + i] = (float)((int)(b & 0xF) - 8) * d;
                y[j * 32 + i + 16] = (float)((int)(b >> 4) - 8) * d;
            }
        }
    } else {
        /* ggml dequantize_row_q4_K: chunk c of 32 qs bytes -> sub-blocks 2c (lo), 2c+1 (hi);
         * y = (d*sc)*q - dmin*m in fp32.  d*sc and (d*sc)*q are exact products. */
        const uint8_t* blk = (const uint8_t*)W + (size_t)n * (K / 256) * 144;
        for (int s = 0; s < K / 256; s++, blk += 144) {
            float d = or_f16_to_f32(rd16(blk)), dmin = or_f16_to_f32(rd16(blk + 2));
            const uint8_t* q = blk + 16;
            for (int c = 0; c < 4; c++) {
                uint8_t sc0, m0, sc1, m1;
                or_q4k_get_scale_min(2 * c, blk + 4, &sc0, &m0);
                or_q4k_get_scale_min(2 * c + 1, blk + 4, &sc1, &m1);
                float d1 = d * (float)sc0, mm1 = dmin * (float)m0;
                float d2 = d * (float)sc1, mm2 = dmin * (float)m1;
                float* yy = y + s * 256 + c * 64;
                for (int l = 0; l < 32; l++) {
                    yy[l] = d1 * (float)(q[32 * c + l] & 0xF) - mm1;
                    yy[32 + l] = d2 * (float)(q[32 * c + l] >> 4) - mm2;
                }
            }
        }
    }
}

static int shape_ok(int qtype, int N, int K) {
    if (N <= 0 || K <= 0) return 0;
    if (qtype == OR_Q4_K) return K % 256 == 0;
    if (qtype == OR_Q4_0 || qtype == OR_Q4_0_PLANES) return K % 32 == 0;
    return 0;
}

int or_dequant_f32(int qtype, const void* W, const void* W_aux, int N, int K, float* out) {
    if (!shape_ok(qtype, N, K)) return -1;
#pragma omp parallel for schedule(static)
    for (int n = 0; n < N; n++) dequant_row_f32(qtype, W, W_aux, K, n, out + (size_t)n * K);
    return 0;
}

int or_dequant_f16(int qtype, const void* W, const void* W_aux, int N, int K, uint16_t* out) {
    if (!shape_ok(qtype, N, K)) return -1;
int ok = 1;
#pragma omp parallel
    {
        float* row = (float*)malloc(sizeof(float) * (size_t)K);
        if (!row) {
#pragma omp atomic write
            ok = 0;
        } else {
#pragma omp for schedule(static)
            for (int n = 0; n < N; n++) {
                dequant_row_f32(qtype, W, W_aux, K, n, row);
                for (int k = 0; k < K; k++) out[(size_t)n * K + k] = or_f32_to_f16(row[k]);
            }
            free(row);
        }
    }
    return ok ? 0 : -1;
}

/* ------------------------------------------------------------------------- */
/* GEMM references                                                            */
/* ------------------------------------------------------------------------- */

static void set_threads(int threads) {
#ifdef _OPENMP
    omp_set_num_threads(threads > 0 ? threads : omp_get_num_procs());
#else
    (void)threads;
#endif
}

int or_max_threads(void) {
#ifdef _OPENMP
    return omp_get_num_procs();
#else
    return 1;
#endif
}

static int gemm_f64_impl(int qtype, const void* W, const void* W_aux, const uint16_t* A,
                         int M, int N, int K, double* C, int threads, int round_w) {
    if (!shape_ok(qtype, N, K) || M <= 0) return -1;
    set_threads(threads);
    double* Ad = (double*)malloc(sizeof(double) * (size_t)M * K);
    if (!Ad) return -1;
    for (size_t i = 0; i < (size_t)M * K; i++) Ad[i] = (double)or_f16_to_f32(A[i]);
#pragma omp parallel
    {
        float* row = (float*)malloc(sizeof(float) * (size_t)K);
#pragma omp for schedule(static)
        for (int n = 0; n < N; n++) {
            dequant_row_f32(qtype, W, W_aux, K, n, row);
            if (round_w)
                for (int k = 0; k < K; k++) row[k] = or_f16_to_f32(or_f32_to_f16(row[k]));
            for (int m = 0; m < M; m++) {
                const double* a = Ad + (size_t)m * K;
                double s = 0.0;
                for (int k = 0; k < K; k++) s += a[k] * (double)row[k];
                C[(size_t)m * N + n] = s;
            }
        }
        free(row);
    }
    free(Ad);
    return 0;
}

int or_gemm_f64(int qtype, const void* W, const void* W_aux, const uint16_t* A,
                int M, int N, int K, double* C, int threads) {
    return gemm_f64_impl(qtype, W, W_aux, A, M, N, K, C, threads, 0);
}

int or_gemm_f16w_f64(int qtype, const void* W, const void* W_aux, const uint16_t* A,
                     int M, int N, int K, double* C, int threads) {
    return gemm_f64_impl(qtype, W, W_aux, A, M, N, K, C, threads, 1);
}

/* fp32-accumulated dot with eight independent partial sums, so the loop
 * vectorises without reassociation flags; cloned per ISA level at load time. */
__attribute__((target_clones("avx512f", "avx2", "default")))
static float dot8_f32(const float* a, const float* w, int K) {
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int k = 0; k < K; k += 8)
        for (int u = 0; u < 8; u++) acc[u] += a[k + u] * w[k + u];
    return ((acc[0] + acc[1]) + (acc[2] + acc[3])) + ((acc[4] + acc[5]) + (acc[6] + acc[7]));
}

static double now_s(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (double)ts.tv_sec + 1e-9 * (double)ts.tv_nsec;
}

int or_cpu_dequant_matmul(int qtype, const void* W, const void* W_aux, const uint16_t* A,
                          int M, int N, int K, float* W_f32, float* C, int threads,
                          double* t_dq, double* t_mm) {
    if (!shape_ok(qtype, N, K) || M <= 0 || K % 8 != 0) return -1;
    set_threads(threads);
    float* Af = (float*)malloc(sizeof(float) * (size_t)M * K);
    if (!Af) return -1;
    double t0 = now_s();
    for (size_t i = 0; i < (size_t)M * K; i++) Af[i] = or_f16_to_f32(A[i]);
#pragma omp parallel for schedule(static)
    for (int n = 0; n < N; n++) dequant_row_f32(qtype, W, W_aux, K, n, W_f32 + (size_t)n * K);
    double t1 = now_s();
#pragma omp parallel for schedule(static)
    for (int n = 0; n < N; n++)
        for (int m = 0; m < M; m++)
            C[(size_t)m * N + n] = dot8_f32(Af + (size_t)m * K, W_f32 + (size_t)n * K, K);
    double t2 = now_s();
    free(Af);
    if (t_dq) *t_dq = t1 - t0;
    if (t_mm) *t_mm = t2 - t1;
    return 0;
}
