// Integer-dot activation path: activations quantized to int8 per 32 values
// (bf_quantize_q8), weights multiplied in as 4-bit codes on integer dots:
// v_mfma_i32_16x16x32_i8 from 3 batch rows (k_gemm_q8m), v_dot4_i32_i8 at 1-2
// (k_gemm_q8), where its lower fixed cost wins.
//
// No counterpart in the reference's kernels (kernels/busfill_v1a.cu:41-104
// multiplies fp16 activations by dequantized fp16 weights); its results credit
// llama.cpp's quantized GEMM, which packs activations as int8 per 32 values and
// spends one integer 4-way dot per four weights (RESULTS.md:72-77, 93-96).
//
// Quantized activations (one device buffer, regions contiguous):
//   q [M][K] int8 | d [M][K/32] fp32 | s [M][K/32] int32
// with d = amax/127 over the 32 values, q = round(x/d) (half away from zero,
// 0 for an all-zero block) and s = sum of the block's q.
//
// Both forms compute, per 32-weight block b, the exact integer
// dot_b = sum code*q (the 4-bit codes as bytes 0..15) and
//   C += d8_b * (scale_b * dot_b - offset_b * s_b)
// in fp32 (Q4_0 and planes: scale = d, offset = 8d; Q4_K: scale = d*sc,
// offset = dmin*m), and sum in a fixed order: results are deterministic.
//
// v_dot4 form: a lane owns one 64-weight unit (two 32-weight blocks; for Q4_K
// the two sub-blocks sharing 32 code bytes) of four weight rows, and reuses
// each batch row's 64 activation bytes over those four rows.  16 lanes (units)
// x 4 row groups = 16 rows per workgroup; the workgroup's waves split the
// row's units.  Lane sums reduce over the 16 unit lanes by butterfly and over
// the waves through LDS.
#include <algorithm>
#include <atomic>

#include "bf_device.h"
#include "bf_formats.h"
#include "bf_launch.h"
#include "bf_lds_plan.h"

namespace bf {

namespace {

constexpr int kQ8Rows = 16;       // weight rows per workgroup
constexpr int kQ8MaxWaves = 8;
constexpr int kQ8MaxM = 16;

__device__ __forceinline__ int dot4(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

constexpr uint32_t kNib = 0x0F0F0F0Fu;

// One unit of one row: wl[i] holds the four codes (bytes 0..15) that multiply
// activation word a[i] (a[0..7] = block a, a[8..15] = block b), masked once per
// unit and reused for every batch row.
struct Q8Row {
    uint32_t wl[16];
    float sa, oa, sb, ob;
    __device__ __forceinline__ void dots(const uint32_t a[16], int& da, int& db) const {
        int x = 0, y = 0;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            x = dot4(wl[i], a[i], x);
            y = dot4(wl[8 + i], a[8 + i], y);
        }
        da = x; db = y;
    }
    // Q4_0 order within one 16-byte block: byte i = weights i (low), i+16 (high)
    __device__ __forceinline__ void set_q40(const uint32_t* cw, uint32_t* out) {
#pragma unroll
        for (int t = 0; t < 4; t++) {
            out[t] = cw[t] & kNib;
            out[4 + t] = (cw[t] >> 4) & kNib;
        }
    }
};

template <int QT>
__device__ __forceinline__ void load_q8row(Q8Row& r, const uint8_t* W, const uint8_t* Waux, int64_t n, int j,
                                           int K);

// Q4_K: 32 code bytes (sub-block a = low nibbles, b = high nibbles) + header
template <>
__device__ __forceinline__ void load_q8row<QT_Q4_K>(Q8Row& r, const uint8_t* W, const uint8_t*, int64_t n, int j,
                                                    int K) {
    const uint8_t* base = W + n * ((int64_t)(K >> 8) * 144) + (int64_t)(j >> 2) * 144;
    const int c = j & 3;
    const u4 h = ld16(base), q0 = ld16(base + 16 + 32 * c), q1 = ld16(base + 32 + 32 * c);
    const uint32_t cw[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
#pragma unroll
    for (int t = 0; t < 8; t++) {
        r.wl[t] = cw[t] & kNib;
        r.wl[8 + t] = (cw[t] >> 4) & kNib;
    }
    const float d = half_bits_to_float(h.x & 0xFFFFu), dmin = half_bits_to_float(h.x >> 16);
    // (scale, min) of sub-blocks 2c and 2c+1 without divergent branches (c
    // differs between lanes): both forms of ggml get_scale_min_k4, then a select
    const uint32_t s0 = h.y, s1 = h.z, s2 = h.w;
    const uint32_t sh = 16u * (uint32_t)(c & 1);
    const uint32_t lo_sc = (s0 >> sh) & 0x3F3Fu, lo_m = (s1 >> sh) & 0x3F3Fu;   // c < 2: bytes 2c, 2c+1
    const uint32_t b2 = (s2 >> sh) & 0xFFFFu;
    const uint32_t hi_sc = (b2 & 0x0F0Fu) | (((s0 >> sh) >> 2) & 0x3030u);       // c >= 2
    const uint32_t hi_m = ((b2 >> 4) & 0x0F0Fu) | (((s1 >> sh) >> 2) & 0x3030u);
    const uint32_t scp = c < 2 ? lo_sc : hi_sc, mp = c < 2 ? lo_m : hi_m;
    r.sa = d * (float)(scp & 0xFFu); r.oa = dmin * (float)(mp & 0xFFu);
    r.sb = d * (float)(scp >> 8); r.ob = dmin * (float)(mp >> 8);
}

// Q4_0: blocks 2j, 2j+1 = 36 bytes, 4-byte aligned: [d0][16 codes][d1][16 codes]
template <>
__device__ __forceinline__ void load_q8row<QT_Q4_0>(Q8Row& r, const uint8_t* W, const uint8_t*, int64_t n, int j,
                                                    int K) {
    const uint8_t* base = W + n * ((int64_t)(K >> 5) * 18) + (int64_t)j * 36;
    const u4 a = ld16_a4(base), b = ld16_a4(base + 16);
    const uint32_t c = *(const uint32_t*)(base + 32);
    const uint32_t w[9] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w, c};
    uint32_t cw[8];
#pragma unroll
    for (int t = 0; t < 4; t++) cw[t] = __builtin_amdgcn_alignbyte(w[t + 1], w[t], 2);   // bytes 2..17
#pragma unroll
    for (int t = 0; t < 4; t++) cw[4 + t] = w[5 + t];                                     // bytes 20..35
    r.set_q40(cw, r.wl);
    r.set_q40(cw + 4, r.wl + 8);
    r.sa = half_bits_to_float(a.x & 0xFFFFu);
    r.sb = half_bits_to_float(b.x >> 16);
    r.oa = 8.f * r.sa; r.ob = 8.f * r.sb;
}

// planes: 32 code bytes, byte i = weights 2i (low) and 2i+1 (high); the
// activation words of each block are regrouped as [even elements | odd elements]
// (see k_gemm_q8), so the low nibbles meet words 0-3 and the high ones 4-7
template <>
__device__ __forceinline__ void load_q8row<QT_PLANES>(Q8Row& r, const uint8_t* W, const uint8_t* Waux, int64_t n,
                                                      int j, int K) {
    const uint8_t* base = W + n * (int64_t)(K >> 1) + (int64_t)j * 32;
    const u4 q0 = ld16(base), q1 = ld16(base + 16);
    const uint32_t cw[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
    r.set_q40(cw, r.wl);
    r.set_q40(cw + 4, r.wl + 8);
    const uint32_t sc = *(const uint32_t*)(Waux + 2 * (n * (int64_t)(K >> 5) + 2 * j));
    r.sa = half_bits_to_float(sc & 0xFFFFu);
    r.sb = half_bits_to_float(sc >> 16);
    r.oa = 8.f * r.sa; r.ob = 8.f * r.sb;
}

}  // namespace

// One thread per 8 activations, four threads per 32-value block.
__global__ __launch_bounds__(256) void k_quantize_q8(const uint16_t* __restrict__ A, int lda,
                                                     int8_t* __restrict__ q, float* __restrict__ d,
                                                     int* __restrict__ s, int M, int K) {
    const int64_t per_row = K >> 3, total = (int64_t)M * per_row;
    const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const bool live = t < total;
    const int64_t tt = live ? t : total - 1;    // total % 4 == 0: a block's four threads are all live or all not
    const int64_t m = tt / per_row;
    const int k = (int)(tt - m * per_row) << 3;
    const h8 v = ld_act(A + m * lda + k);
    float x[8], amax = 0.f;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        x[i] = (float)v[i];
        amax = __builtin_fmaxf(amax, __builtin_fabsf(x[i]));
    }
    amax = __builtin_fmaxf(amax, __shfl_xor(amax, 1, 64));
    amax = __builtin_fmaxf(amax, __shfl_xor(amax, 2, 64));
    const float dd = amax / 127.0f;
    int qi[8], sum = 0;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        qi[i] = amax == 0.f ? 0 : (int)__builtin_roundf(x[i] / dd);
        sum += qi[i];
    }
    sum += __shfl_xor(sum, 1, 64);
    sum += __shfl_xor(sum, 2, 64);
    if (live) {
        uint32_t p0 = 0, p1 = 0;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            p0 |= ((uint32_t)qi[i] & 0xFFu) << (8 * i);
            p1 |= ((uint32_t)qi[4 + i] & 0xFFu) << (8 * i);
        }
        *(uint2*)(q + m * K + k) = make_uint2(p0, p1);
        if ((k & 31) == 0) {
            d[m * (K >> 5) + (k >> 5)] = dd;
            s[m * (K >> 5) + (k >> 5)] = sum;
        }
    }
}

template <int QT, int MB>
__global__ __launch_bounds__(64 * kQ8MaxWaves)
void k_gemm_q8(const uint8_t* __restrict__ W, const uint8_t* __restrict__ Waux, const int8_t* __restrict__ q,
               const float* __restrict__ d8, const int* __restrict__ s8, void* __restrict__ C, int ldc, int out_f16,
               int Mall, int N, int K, int nx, int ny) {
    __shared__ float red[kQ8MaxWaves][kQ8Rows][MB];
    // block b -> (row block x, batch group y): the ny groups of one row block sit
    // 8 blocks apart, i.e. on the same XCD, so its L2 serves the weights' reuse
    const int b = blockIdx.x, per = 8 * ny;
    const int y = (b % per) >> 3, x = (b / per) * 8 + (b & 7);
    if (x >= nx) return;                                       // whole workgroup, before any barrier
    const int m0 = y * MB, M = min(MB, Mall - m0);
    q += (int64_t)m0 * K;
    d8 += (int64_t)m0 * (K >> 5);
    s8 += (int64_t)m0 * (K >> 5);
    C = (uint8_t*)C + (int64_t)m0 * ldc * (out_f16 ? 2 : 4);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nwaves = blockDim.x >> 6;
    const int rg = lane >> 4, u = lane & 15;
    const int nunits = K >> 6, nblk = K >> 5;
    const int64_t row0 = (int64_t)x * kQ8Rows + 4 * rg;

    float acc[4][MB];
#pragma unroll
    for (int r = 0; r < 4; r++)
#pragma unroll
        for (int m = 0; m < MB; m++) acc[r][m] = 0.f;

    for (int j = wave * 16 + u; j < nunits; j += nwaves * 16) {
        Q8Row wu[4];
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int64_t n = row0 + r < N ? row0 + r : (int64_t)N - 1;
            load_q8row<QT>(wu[r], W, Waux, n, j, K);
        }
        // batch row m's 64 activation bytes, scales and sums; row m+1's are in
        // flight while row m computes
        auto fetch = [&](int m, u4* av, float2& dm, int2& sm) {
            const int mm = m < M ? m : M - 1;
            const int8_t* qa = q + (int64_t)mm * K + 64 * j;
            av[0] = *(const u4*)qa;
            av[1] = *(const u4*)(qa + 16);
            av[2] = *(const u4*)(qa + 32);
            av[3] = *(const u4*)(qa + 48);
            dm = *(const float2*)(d8 + (int64_t)mm * nblk + 2 * j);
            sm = *(const int2*)(s8 + (int64_t)mm * nblk + 2 * j);
        };
        u4 nav[4];
        float2 ndm;
        int2 nsm;
        fetch(0, nav, ndm, nsm);
#pragma unroll
        for (int m = 0; m < MB; m++) {
            uint32_t a[16] = {nav[0].x, nav[0].y, nav[0].z, nav[0].w, nav[1].x, nav[1].y, nav[1].z, nav[1].w,
                              nav[2].x, nav[2].y, nav[2].z, nav[2].w, nav[3].x, nav[3].y, nav[3].z, nav[3].w};
            const float2 dm = ndm;
            const int2 sm = nsm;
            if (m + 1 < MB) fetch(m + 1, nav, ndm, nsm);
            if constexpr (QT == QT_PLANES) {
                // per block: words 0-7 natural order -> 4 words of even elements, 4 of odd
                uint32_t e[16];
#pragma unroll
                for (int b = 0; b < 2; b++)
#pragma unroll
                    for (int t = 0; t < 4; t++) {
                        const uint32_t lo = a[8 * b + 2 * t], hi = a[8 * b + 2 * t + 1];
                        e[8 * b + t] = perm_b32(hi, lo, 0x06040200u);
                        e[8 * b + 4 + t] = perm_b32(hi, lo, 0x07050301u);
                    }
#pragma unroll
                for (int i = 0; i < 16; i++) a[i] = e[i];
            }
            const float sfa = (float)sm.x, sfb = (float)sm.y;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                int da, db;
                wu[r].dots(a, da, db);
                const float ta = __builtin_fmaf(wu[r].sa, (float)da, -wu[r].oa * sfa);
                const float tb = __builtin_fmaf(wu[r].sb, (float)db, -wu[r].ob * sfb);
                acc[r][m] = __builtin_fmaf(dm.x, ta, acc[r][m]);
                acc[r][m] = __builtin_fmaf(dm.y, tb, acc[r][m]);
            }
        }
    }

    // butterfly over the 16 unit lanes of each row group, then the waves' sums
    // through LDS in wave order
#pragma unroll
    for (int r = 0; r < 4; r++)
#pragma unroll
        for (int m = 0; m < MB; m++) {
            float v = acc[r][m];
            v += __shfl_xor(v, 1, 64);
            v += __shfl_xor(v, 2, 64);
            v += __shfl_xor(v, 4, 64);
            v += __shfl_xor(v, 8, 64);
            acc[r][m] = v;
        }
    if (u == 0) {
#pragma unroll
        for (int r = 0; r < 4; r++)
#pragma unroll
            for (int m = 0; m < MB; m++) red[wave][4 * rg + r][m] = acc[r][m];
    }
    __syncthreads();
    for (int i = threadIdx.x; i < kQ8Rows * MB; i += blockDim.x) {
        const int rr = i / MB, m = i - rr * MB;
        const int64_t n = (int64_t)x * kQ8Rows + rr;
        float v = 0.f;
        for (int w = 0; w < nwaves; w++) v += red[w][rr][m];
        if (m < M && n < N) {
            if (out_f16) ((_Float16*)C)[(int64_t)m * ldc + n] = (_Float16)v;
            else ((float*)C)[(int64_t)m * ldc + n] = v;
        }
    }
}

// ------------------------------------------------------------ the MFMA form
// v_mfma_i32_16x16x32_i8 takes one 32-weight block of 16 weight rows and 16
// batch rows per instruction, so each block's integer dot stays separate and
// exact (the scales differ per block): P[m][n] = sum_k q[m][k] * code[n][k] in
// int32, then C[m][n] += d8[m] * (scale[n] * P[m][n] - offset[n] * s[m]) in
// fp32, per block in block order (deterministic).  The 4-bit codes enter as
// bytes 0..15 after one mask per four of them, where the fp16 GEMM spends
// about 2.5 VALU instructions per weight on its exact decode.
//
// Lane (r = l % 16, g = l / 16) supplies weight row r's and batch row r's
// eight values of k-group g of the block (the MFMA contracts A's and B's
// lanes of one group over the same eight k), and receives P[4g + i][r].  The
// k order inside a group follows the format's nibble order (natural for the
// llama.cpp blocks, even-then-odd for the planes layout, whose activation
// bytes are regrouped to match).  A workgroup owns 16 weight rows; its waves
// take the super-groups s, s + waves, ... and add their sums through LDS in
// wave order.
typedef int i4v __attribute__((ext_vector_type(4)));
constexpr int kQ8mMaxK = 32768;          // the batch rows' block scales and sums fit in LDS

__device__ __forceinline__ i4v mfma_i8(uint64_t a, uint64_t b) {
    return __builtin_amdgcn_mfma_i32_16x16x32_i8((long)a, (long)b, i4v{0, 0, 0, 0}, 0, 0, 0);
}
__device__ __forceinline__ uint64_t pack2(uint32_t lo, uint32_t hi) { return (uint64_t)lo | ((uint64_t)hi << 32); }

// One lane's raw bytes of super-group sg of weight row n (loaded one
// super-group ahead of use), then its codes and (scale, offset) per block.
template <int QT> struct Q8mRaw;
// Q4_K: the header and the lane's eight code bytes of each 32-byte chunk c
// (sub-blocks 2c: low nibbles, 2c + 1: high nibbles): bytes 32c + 8g .. + 7
template <> struct Q8mRaw<QT_Q4_K> { u4 h; uint2 w[4]; };
// Q4_0 blocks (18 bytes: fp16 d, 16 code bytes; weight j = low nibble of byte
// j, j + 16 = its high nibble), in pairs of 36 bytes at 4-byte alignment
template <> struct Q8mRaw<QT_Q4_0> { u4 a[4], b[4]; uint32_t c[4]; };
// planes: the lane's 4 code bytes 4g .. 4g + 3 of each 16-byte block and the
// row's eight fp16 block scales of the super-group
template <> struct Q8mRaw<QT_PLANES> { uint32_t w[8]; u4 ds; };

__device__ __forceinline__ void q8m_load(Q8mRaw<QT_Q4_K>& R, const uint8_t* W, const uint8_t*, int64_t n, int sg,
                                         int g, int K) {
    const uint8_t* base = W + n * ((int64_t)(K >> 8) * 144) + (int64_t)sg * 144;
    R.h = ld16(base);
#pragma unroll
    for (int c = 0; c < 4; c++) R.w[c] = *(const uint2*)(base + 16 + 32 * c + 8 * g);
}
__device__ __forceinline__ void q8m_load(Q8mRaw<QT_Q4_0>& R, const uint8_t* W, const uint8_t*, int64_t n, int sg,
                                         int g, int K) {
    const uint8_t* base = W + n * ((int64_t)(K >> 5) * 18) + (int64_t)sg * 144;
#pragma unroll
    for (int p = 0; p < 4; p++) {
        R.a[p] = ld16_a4(base + 36 * p);
        R.b[p] = ld16_a4(base + 36 * p + 16);
        R.c[p] = *(const uint32_t*)(base + 36 * p + 32);
    }
}
__device__ __forceinline__ void q8m_load(Q8mRaw<QT_PLANES>& R, const uint8_t* W, const uint8_t* Waux, int64_t n,
                                         int sg, int g, int K) {
    const uint8_t* base = W + n * (int64_t)(K >> 1) + (int64_t)sg * 128 + 4 * g;
#pragma unroll
    for (int b = 0; b < 8; b++) R.w[b] = *(const uint32_t*)(base + 16 * b);
    R.ds = ld16_a4(Waux + 2 * (n * (int64_t)(K >> 5) + 8 * sg));
}

__device__ __forceinline__ void q8m_decode(const Q8mRaw<QT_Q4_K>& R, int g, uint64_t code[8], float scale[8],
                                           float off[8]) {
#pragma unroll
    for (int c = 0; c < 4; c++) {
        code[2 * c] = pack2(R.w[c].x & kNib, R.w[c].y & kNib);
        code[2 * c + 1] = pack2((R.w[c].x >> 4) & kNib, (R.w[c].y >> 4) & kNib);
    }
    const float d = half_bits_to_float(R.h.x & 0xFFFFu), dmin = half_bits_to_float(R.h.x >> 16);
    // ggml get_scale_min_k4 over the 12 scale bytes (header bytes 4..15)
    const uint32_t sw[3] = {R.h.y, R.h.z, R.h.w};
    auto byte = [&](int i) { return (sw[i >> 2] >> (8 * (i & 3))) & 0xFFu; };
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const uint32_t scj = j < 4 ? byte(j) & 63u : (byte(j + 4) & 0xFu) | ((byte(j - 4) >> 6) << 4);
        const uint32_t mj = j < 4 ? byte(j + 4) & 63u : (byte(j + 4) >> 4) | ((byte(j) >> 6) << 4);
        scale[j] = d * (float)scj;
        off[j] = dmin * (float)mj;
    }
}
// Q4_0: group g takes code bytes 8 (g & 1) .. + 7 of a block, nibble g / 2
__device__ __forceinline__ void q8m_decode(const Q8mRaw<QT_Q4_0>& R, int g, uint64_t code[8], float scale[8],
                                           float off[8]) {
#pragma unroll
    for (int p = 0; p < 4; p++) {
        const uint32_t w[9] = {R.a[p].x, R.a[p].y, R.a[p].z, R.a[p].w, R.b[p].x, R.b[p].y, R.b[p].z, R.b[p].w, R.c[p]};
        // block 2p: code bytes 2..17; block 2p + 1: bytes 20..35
        const uint32_t b0[4] = {__builtin_amdgcn_alignbyte(w[1], w[0], 2), __builtin_amdgcn_alignbyte(w[2], w[1], 2),
                                __builtin_amdgcn_alignbyte(w[3], w[2], 2), __builtin_amdgcn_alignbyte(w[4], w[3], 2)};
        const uint32_t b1[4] = {w[5], w[6], w[7], w[8]};
        const bool hi = (g & 1) != 0;
        const uint32_t s0 = (g >> 1) ? 4u : 0u;
        const uint32_t x0 = hi ? b0[2] : b0[0], x1 = hi ? b0[3] : b0[1];
        const uint32_t y0 = hi ? b1[2] : b1[0], y1 = hi ? b1[3] : b1[1];
        code[2 * p] = pack2((x0 >> s0) & kNib, (x1 >> s0) & kNib);
        code[2 * p + 1] = pack2((y0 >> s0) & kNib, (y1 >> s0) & kNib);
        scale[2 * p] = half_bits_to_float(R.a[p].x & 0xFFFFu);
        scale[2 * p + 1] = half_bits_to_float(R.b[p].x >> 16);
        off[2 * p] = 8.f * scale[2 * p];
        off[2 * p + 1] = 8.f * scale[2 * p + 1];
    }
}
// planes: the group's eight weights as [low nibbles | high nibbles] (even,
// then odd k)
__device__ __forceinline__ void q8m_decode(const Q8mRaw<QT_PLANES>& R, int g, uint64_t code[8], float scale[8],
                                           float off[8]) {
    const uint32_t dw[4] = {R.ds.x, R.ds.y, R.ds.z, R.ds.w};
#pragma unroll
    for (int b = 0; b < 8; b++) {
        code[b] = pack2(R.w[b] & kNib, (R.w[b] >> 4) & kNib);
        scale[b] = half_bits_to_float((dw[b >> 1] >> (16 * (b & 1))) & 0xFFFFu);
        off[b] = 8.f * scale[b];
    }
}

// One workgroup per CU: workgroup p owns rows [R p, R p + R) (R = ceil(N / G)),
// covered by T = ceil(R / 16) tiles of 16 rows at offsets min(16 t, R - 16)
// (the last tile overlaps the one before it when 16 does not divide R: its
// shared rows are loaded from L1 again and computed twice, stored once), so
// every CU streams the same share of the weights in one round.  Each wave takes
// every tile for the super-groups s, s + waves, ...: one activation fragment
// feeds T MFMAs.
template <int QT, int T, int NW>
__global__ __launch_bounds__(64 * NW)
void k_gemm_q8m(const uint8_t* __restrict__ W, const uint8_t* __restrict__ Waux, const int8_t* __restrict__ q,
                const float* __restrict__ d8, const int* __restrict__ s8, void* __restrict__ C, int ldc, int out_f16,
                int M, int N, int K, int R) {
    // the batch rows' block scales and sums, [block][batch row] (rows past M
    // repeat row M - 1), staged once per workgroup: a lane then reads its four
    // output rows' values of a block with one 16-byte LDS read each
    extern __shared__ __attribute__((aligned(16))) float q8lds[];
    float* const red = q8lds;                                             // [wave][tile][16][17]
    f4* const dsl = (f4*)(q8lds + NW * T * 16 * 17);                      // [block][4 quads of rows]: d8
    f4* const ssl = dsl + (K >> 5) * 4;                                   // same: fp32 sums
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nwaves = blockDim.x >> 6;
    const int r = lane & 15, g = lane >> 4;
    const int64_t base = (int64_t)blockIdx.x * R;
    int64_t n[T];                                                         // this lane's weight row per tile
#pragma unroll
    for (int t = 0; t < T; t++) n[t] = min(base + min(16 * t, R - 16) + r, (int64_t)N - 1);   // clamped: dropped
    const int ma = min(r, M - 1);                                         // this lane's activation row
    const int nsg = K >> 8, nblk = K >> 5;
    for (int x = threadIdx.x; x < nblk * 16; x += blockDim.x) {
        const int b = x >> 4, m = min(x & 15, M - 1);
        ((float*)dsl)[x] = d8[(int64_t)m * nblk + b];
        ((float*)ssl)[x] = (float)s8[(int64_t)m * nblk + b];
    }
    __syncthreads();
    f4 acc[T];
#pragma unroll
    for (int t = 0; t < T; t++) acc[t] = f4{0.f, 0.f, 0.f, 0.f};
    const int8_t* qrow = q + (int64_t)ma * K + 8 * g;
    for (int sg = wave; sg < nsg; sg += nwaves) {
        Q8mRaw<QT> raw[T];
#pragma unroll
        for (int t = 0; t < T; t++) q8m_load(raw[t], W, Waux, n[t], sg, g, K);
        uint2 av[8];
#pragma unroll
        for (int b = 0; b < 8; b++) av[b] = *(const uint2*)(qrow + 256 * sg + 32 * b);
        uint64_t a[8];
#pragma unroll
        for (int b = 0; b < 8; b++) {
            if constexpr (QT == QT_PLANES)
                a[b] = pack2(perm_b32(av[b].y, av[b].x, 0x06040200u), perm_b32(av[b].y, av[b].x, 0x07050301u));
            else
                a[b] = pack2(av[b].x, av[b].y);
        }
#pragma unroll
        for (int t = 0; t < T; t++) {
            uint64_t code[8];
            float scale[8], off[8];
            q8m_decode(raw[t], g, code, scale, off);
            i4v P[8];
#pragma unroll
            for (int b = 0; b < 8; b++) P[b] = mfma_i8(a[b], code[b]);
#pragma unroll
            for (int b = 0; b < 8; b++) {
                const f4 dd = dsl[(8 * sg + b) * 4 + g], ss = ssl[(8 * sg + b) * 4 + g];   // rows 4g .. 4g + 3
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const float u = __builtin_fmaf(scale[b], (float)P[b][i], -off[b] * ss[i]);
                    acc[t][i] = __builtin_fmaf(dd[i], u, acc[t][i]);
                }
            }
        }
    }
#pragma unroll
    for (int t = 0; t < T; t++)
#pragma unroll
        for (int i = 0; i < 4; i++) red[((wave * T + t) * 16 + 4 * g + i) * 17 + r] = acc[t][i];
    __syncthreads();
    // row rr of the workgroup comes from the tile whose own rows hold it
    for (int x = threadIdx.x; x < R * 16; x += blockDim.x) {
        const int rr = x >> 4, m = x & 15;
        const int t = min(rr >> 4, T - 1), lr = rr - min(16 * t, R - 16);
        float v = 0.f;
        for (int w = 0; w < nwaves; w++) v += red[((w * T + t) * 16 + m) * 17 + lr];
        if (m < M && base + rr < N) {
            if (out_f16) ((_Float16*)C)[(int64_t)m * ldc + base + rr] = (_Float16)v;
            else ((float*)C)[(int64_t)m * ldc + base + rr] = v;
        }
    }
}

namespace {

template <int QT, int MB>
hipError_t launch_q8(const Q8Args& g, hipStream_t st) {
    // waves per workgroup: as few passes over the units as 8 waves allow, then
    // the fewest waves that keep that many passes
    const int n16 = (g.K / 64 + 15) / 16;
    const int passes = (n16 + kQ8MaxWaves - 1) / kQ8MaxWaves;
    const int waves = (n16 + passes - 1) / passes;
    const int8_t* q = (const int8_t*)g.Aq;
    const float* d = (const float*)(q + (int64_t)g.M * g.K);
    const int* s = (const int*)(d + (int64_t)g.M * (g.K / 32));
    const int nx = (g.N + kQ8Rows - 1) / kQ8Rows, ny = (g.M + MB - 1) / MB;
    dim3 grid((unsigned)(((nx + 7) / 8) * 8 * ny));
    hipLaunchKernelGGL((k_gemm_q8<QT, MB>), grid, dim3(64 * waves), 0, st, g.W, g.Waux, q, d, s, g.C, g.ldc,
                       g.out_f16, g.M, g.N, g.K, nx, ny);
    return hipGetLastError();
}

// Waves per workgroup of the MFMA form with T tiles: as many as registers
// allow (more super-groups in flight), 16 up to two tiles, 8 above.
constexpr int q8m_waves(int T) { return T <= 2 ? 16 : 8; }

// LDS of one k_gemm_q8m workgroup: the waves' partial sums, then the batch
// rows' block scales and sums for all of K.
size_t q8m_lds_bytes(int K, int T) {
    return (size_t)q8m_waves(T) * T * 16 * 17 * 4 + (size_t)(K / 32) * 16 * 4 * 2;
}

template <int QT, int T>
hipError_t launch_q8m_t(const Q8Args& g, int R, int G, hipStream_t st) {
    constexpr int NW = q8m_waves(T);
    const int8_t* q = (const int8_t*)g.Aq;
    const float* d = (const float*)(q + (int64_t)g.M * g.K);
    const int* s = (const int*)(d + (int64_t)g.M * (g.K / 32));
    const int waves = std::min(NW, g.K / 256);
    const size_t lds = q8m_lds_bytes(g.K, T);
    if (lds > (size_t)kMaxLds) return hipErrorInvalidValue;     // the dispatcher sends such shapes to k_gemm_q8
    auto k = k_gemm_q8m<QT, T, NW>;
    if (lds > 64 * 1024) {
        // raised once per device to the most any shape may ask for, so the
        // limit does not depend on which K came first
        static std::atomic<uint64_t> attr_set{0};     // one bit per device: LDS limit raised
        int dev = 0;
        hipError_t e = hipGetDevice(&dev);
        if (e != hipSuccess) return e;
        const uint64_t bit = 1ull << (dev & 63);
        if (!(attr_set.load(std::memory_order_acquire) & bit)) {
            e = hipFuncSetAttribute((const void*)k, hipFuncAttributeMaxDynamicSharedMemorySize, kMaxLds);
            if (e != hipSuccess) return e;
            attr_set.fetch_or(bit, std::memory_order_acq_rel);
        }
    }
    hipLaunchKernelGGL(k, dim3((unsigned)G), dim3(64 * waves), lds, st, g.W, g.Waux, q, d, s, g.C, g.ldc, g.out_f16,
                       g.M, g.N, g.K, R);
    return hipGetLastError();
}

// Rows per workgroup: the N rows over one workgroup per CU (at least 16).
int q8m_rows(int N) {
    static std::atomic<int> cus{0};
    int c = cus.load(std::memory_order_relaxed);
    if (c == 0) {
        int dev = 0, v = 0;
        if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) !=
                                                    hipSuccess || v < 1)
            v = 256;
        cus.store(v, std::memory_order_relaxed);
        c = v;
    }
    return std::max(16, (N + c - 1) / c);
}

template <int QT>
hipError_t launch_q8m(const Q8Args& g, hipStream_t st) {
    const int R = q8m_rows(g.N), G = (g.N + R - 1) / R, T = (R + 15) / 16;
    switch (T) {
        case 1: return launch_q8m_t<QT, 1>(g, R, G, st);
        case 2: return launch_q8m_t<QT, 2>(g, R, G, st);
        case 3: return launch_q8m_t<QT, 3>(g, R, G, st);
        case 4:
            if constexpr (QT == QT_Q4_0) return hipErrorNotSupported;
            else return launch_q8m_t<QT, 4>(g, R, G, st);
        default:
            if constexpr (QT == QT_Q4_0) return hipErrorNotSupported;
            else return launch_q8m_t<QT, 5>(g, R, G, st);
    }
}

template <int QT>
hipError_t dispatch_q8_m(const Q8Args& g, hipStream_t st) {
    // The MFMA form from 3 batch rows (below, the v_dot4 form's fixed cost is
    // lower: 7.4 / 8.5 against 9.6 / 10.1 us at 5120^2, M = 1 / 2); Q4_0's
    // 36-byte block pairs take the most registers: up to 3 tiles
    const int R = q8m_rows(g.N);
    if (g.M >= 3 && g.K % 256 == 0 && g.K <= kQ8mMaxK && R <= (QT == QT_Q4_0 ? 48 : 80) &&
        q8m_lds_bytes(g.K, (R + 15) / 16) <= (size_t)kMaxLds)
        return launch_q8m<QT>(g, st);
    // batches above 4 run as groups of 4 rows (more batch rows per workgroup
    // cost registers, and with them the second workgroup per CU)
    if (g.M <= 1) return launch_q8<QT, 1>(g, st);
    if (g.M <= 2) return launch_q8<QT, 2>(g, st);
    return launch_q8<QT, 4>(g, st);
}

}  // namespace

size_t q8_bytes(int M, int K) { return (size_t)M * K + (size_t)8 * M * (K / 32); }

hipError_t quantize_q8(const uint16_t* A, int lda, void* Aq, int M, int K, hipStream_t st) {
    int8_t* q = (int8_t*)Aq;
    float* d = (float*)(q + (int64_t)M * K);
    int* s = (int*)(d + (int64_t)M * (K / 32));
    const int64_t threads = (int64_t)M * (K / 8);
    hipLaunchKernelGGL(k_quantize_q8, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, st, A, lda, q, d, s, M,
                       K);
    return hipGetLastError();
}

bool q8_supports(int M, int K) { return M >= 1 && M <= kQ8MaxM && K % 64 == 0; }

hipError_t gemm_q8(const Q8Args& g, hipStream_t st) {
    if (!q8_supports(g.M, g.K)) return hipErrorNotSupported;
    switch (g.qtype) {
        case QT_Q4_K: return dispatch_q8_m<QT_Q4_K>(g, st);
        case QT_Q4_0: return dispatch_q8_m<QT_Q4_0>(g, st);
        case QT_PLANES: return dispatch_q8_m<QT_PLANES>(g, st);
        default: return hipErrorNotSupported;
    }
}

}  // namespace bf
