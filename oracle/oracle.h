/*
 * CPU oracle for the batched int4-block-weight x fp16-activation GEMM.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the checker
 * (or, for the CPU baseline, as the thing timed on the host).  The product path
 * in bus-fill_amd/ never links or calls it.
 *
 * Every function restates the reference's algorithm on the CPU in plain C:
 *   - Q4_0 "planes" (reference kernel layout): kernels/busfill_v0.cu:42-44,118-123
 *     value = RN_fp16((q - 8) * fp32(d))                   kernels/busfill_v0.cu:74,78-81
 *   - Q4_0 llama.cpp 18-byte block (config text, kernels/busfill_v0.cu:18-20):
 *     third-party ggml block_q4_0 (fp16 d, qs[16]; elem j = qs[j] & 0xF,
 *     elem j+16 = qs[j] >> 4; value (q - 8) * d).  Not present in the reference.
 *   - Q4_K 144-byte super-block: third-party ggml block_q4_K / get_scale_min_k4 /
 *     dequantize_row_q4_K, described only in prose (RESULTS.md:84-96).
 *   - dequantize-then-matmul: kernels/busfill_v1a.cu:159-167 (fp64 check over the
 *     unrounded fp32 refW of kernels/busfill_v0.cu:124-125) and the torch gate of
 *     kernels/q4k_batched.py:97-104.
 *
 * All fp16 values travel as uint16_t bit patterns.
 */
#ifndef BUSFILL_ORACLE_H
#define BUSFILL_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* weight formats (same numbering as the product C-ABI) */
enum { OR_Q4_0 = 0,          /* llama.cpp block_q4_0, 18 B per 32 weights          */
       OR_Q4_0_PLANES = 1,   /* reference planes: Wq[N][K/2] u8 + Ws[N][K/32] fp16   */
       OR_Q4_K = 2 };        /* llama.cpp block_q4_K, 144 B per 256 weights          */

/* ---- fp16 <-> fp32, round to nearest even, subnormals kept, NaN quieted ---- */
uint16_t or_f32_to_f16(float f);
float    or_f16_to_f32(uint16_t h);
void     or_f32_to_f16_array(const float* in, uint16_t* out, size_t n);
void     or_f16_to_f32_array(const uint16_t* in, float* out, size_t n);

/* ---- seeded counter-based generator (splitmix64 finalizer) ---- */
uint64_t or_rand(uint64_t seed, uint64_t stream, uint64_t index);
/* fp16 ~ U[lo, hi] from one draw */
uint16_t or_unif_f16(uint64_t draw, float lo, float hi);

/* Q4_0 logical matrix (shared by the planes and the 18-byte-block packers):
 * block b = n*(K/32) + k/32, scale d_b = U[dlo,dhi] from stream 1 index b,
 * code of element e = k%32 is nibble (e%16) of draw (stream 2, index 2b + e/16). */
void or_gen_q4_0_planes(uint64_t seed, int N, int K, float dlo, float dhi,
                        uint8_t* Wq, uint16_t* Ws);
void or_gen_q4_0_blocks(uint64_t seed, int N, int K, float dlo, float dhi,
                        uint8_t* blocks);
/* Q4_K: block b = n*(K/256) + k/256; d from stream 1, dmin from stream 3 (both
 * U[lo,hi]), scales[12] = bytes of draws (stream 4, 2b) and the low 4 bytes of
 * (stream 4, 2b+1), qs[128] = bytes of draws (stream 2, 16b .. 16b+15). */
void or_gen_q4_k(uint64_t seed, int N, int K, float lo, float hi, uint8_t* blocks);
/* activations A[M][K] ~ N(0,1) (Box-Muller over stream 5) rounded to fp16 */
void or_gen_act(uint64_t seed, int M, int K, uint16_t* A);

/* ---- format helpers ---- */
void or_q4k_get_scale_min(int j, const uint8_t* scales, uint8_t* sc, uint8_t* m);
/* inverse of or_q4k_get_scale_min over all 8 sub-blocks (6-bit sc[8], m[8]) */
void or_q4k_pack_scales(const uint8_t* sc, const uint8_t* m, uint8_t* scales);
/* planes <-> 18-byte blocks (same logical matrix, byte count unchanged) */
void or_q4_0_planes_to_blocks(const uint8_t* Wq, const uint16_t* Ws, int N, int K, uint8_t* blocks);
void or_q4_0_blocks_to_planes(const uint8_t* blocks, int N, int K, uint8_t* Wq, uint16_t* Ws);

/* ---- dequant: W -> [N][K]; f16 = the bit-exact contract, f32 = unrounded refW ----
 * W_aux is Ws for OR_Q4_0_PLANES and NULL otherwise.  Returns 0, or -1 on a bad
 * shape or type. */
int or_dequant_f16(int qtype, const void* W, const void* W_aux, int N, int K, uint16_t* out);
int or_dequant_f32(int qtype, const void* W, const void* W_aux, int N, int K, float* out);

/* ---- dequantize-then-matmul references ----
 * C[m][n] = sum_k A[m][k] * refW[n][k] accumulated in fp64 (refW unrounded fp32,
 * as kernels/busfill_v1a.cu:131-132,164).  threads <= 0 means all cores. */
int or_gemm_f64(int qtype, const void* W, const void* W_aux, const uint16_t* A,
                int M, int N, int K, double* C, int threads);
/* same over the fp16-rounded dequant (the GPU dequant contract) */
int or_gemm_f16w_f64(int qtype, const void* W, const void* W_aux, const uint16_t* A,
                     int M, int N, int K, double* C, int threads);

/* CPU baseline: dequantize the whole matrix to fp32 (refW), then an
 * fp32-accumulated matmul, OpenMP over output rows.  W_f32 is caller scratch of
 * N*K floats.  Times (seconds) of the two phases are returned through t_dq/t_mm.
 * threads <= 0 means all cores. */
int or_cpu_dequant_matmul(int qtype, const void* W, const void* W_aux, const uint16_t* A,
                          int M, int N, int K, float* W_f32, float* C, int threads,
                          double* t_dq, double* t_mm);
int or_max_threads(void);

#ifdef __cplusplus
}
#endif
#endif
