// Batched int4-block GEMM on MFMA: C[M][N] = A[M][K] . dequant(W)^T.
//
// Replaces the reference's warp-level mma.m8n8k4 kernel
// (kernels/busfill_v1a.cu:41-104): same math, re-designed for CDNA4.
//
// Work decomposition
//   * one v_mfma_f32_16x16x32_f16 covers 16 batch rows (m) x 16 weight rows (n)
//     x 32 k; a wave owns NT n-tiles (16*NT weight rows) and MT m-tiles;
//   * a workgroup is KW waves that split K: wave w takes the 256-weight
//     super-groups s = w, w+KW, ... and the KW partial tiles are summed through
//     LDS at the end (one launch, no atomics, deterministic);
//   * lane l = (kg = l/16, r = l%16) owns, for every super-group, 64 weights of
//     row n0 + r that lie in ONE contiguous, aligned run of bytes:
//       Q4_K  : chunk kg of qs[128]  (32 B, sub-blocks 2kg and 2kg+1) + header
//       planes: bytes 32kg..32kg+31 of the code row + the two fp16 scales
//       Q4_0  : 18-byte blocks 2kg and 2kg+1 (36 B, 4-byte aligned)
//     and therefore weights k = 256s + 64kg + 8i + j for MFMA i = 0..7, j = 0..7.
//     The activation fragment of lane (r, kg) for MFMA i is A[m][256s+64kg+8i..+7],
//     one 16-byte load in natural order: no LDS staging, no permutation.
//   * weights are decoded by v_perm_b32 / v_and_or_b32 magic bias and scaled in
//     fp16 (v_pk_add_f16 + v_pk_fma_f16/v_pk_mul_f16) before the MFMA, so no
//     per-block fold is needed and the accumulator runs over all of K.  For the
//     Q4_0 formats the fp16 weights equal the bit-exact dequant RN((q-8)*d).
//   * PF super-groups per wave are kept in flight in a register ring.
#include "bf_device.h"
#include "bf_launch.h"

namespace bf {

struct __attribute__((aligned(4))) U4a4 { uint32_t x, y, z, w; };

__device__ __forceinline__ u4 ld16(const uint8_t* p) { return *(const u4*)p; }
__device__ __forceinline__ u4 ld16_a4(const uint8_t* p) {
    U4a4 v = *(const U4a4*)p;
    return u4{v.x, v.y, v.z, v.w};
}
__device__ __forceinline__ h8 ld_act(const uint16_t* p) { return *(const h8*)p; }

// Raw bytes one lane holds for one super-group of one row.
template <int QT> struct Raw;
template <> struct Raw<QT_Q4_K> { u4 hdr, q0, q1; };
template <> struct Raw<QT_PLANES> { u4 q0, q1; uint32_t sc; };
template <> struct Raw<QT_Q4_0> { u4 a, b; uint32_t c; };

template <int QT>
__device__ __forceinline__ void load_raw(Raw<QT>& raw, const uint8_t* W, const uint8_t* Waux,
                                         int64_t n, int s, int kg, int K);

template <>
__device__ __forceinline__ void load_raw<QT_Q4_K>(Raw<QT_Q4_K>& raw, const uint8_t* W, const uint8_t*,
                                                  int64_t n, int s, int kg, int K) {
    const uint8_t* base = W + n * ((int64_t)(K >> 8) * 144) + (int64_t)s * 144;
    raw.hdr = ld16(base);
    raw.q0 = ld16(base + 16 + 32 * kg);
    raw.q1 = ld16(base + 32 + 32 * kg);
}

template <>
__device__ __forceinline__ void load_raw<QT_PLANES>(Raw<QT_PLANES>& raw, const uint8_t* W, const uint8_t* Waux,
                                                    int64_t n, int s, int kg, int K) {
    const uint8_t* base = W + n * (int64_t)(K >> 1) + (int64_t)s * 128 + 32 * kg;
    raw.q0 = ld16(base);
    raw.q1 = ld16(base + 16);
    raw.sc = *(const uint32_t*)(Waux + 2 * (n * (int64_t)(K >> 5) + 8 * s + 2 * kg));
}

template <>
__device__ __forceinline__ void load_raw<QT_Q4_0>(Raw<QT_Q4_0>& raw, const uint8_t* W, const uint8_t*,
                                                  int64_t n, int s, int kg, int K) {
    const uint8_t* base = W + n * ((int64_t)(K >> 8) * 144) + (int64_t)s * 144 + 36 * kg;
    raw.a = ld16_a4(base);
    raw.b = ld16_a4(base + 16);
    raw.c = *(const uint32_t*)(base + 32);
}

// Per-lane scale state derived once per super-group.
template <int QT> struct Scl;
template <> struct Scl<QT_Q4_K> { h2 sa, ma, sb, mb; };   // scale / -min of sub-blocks 2kg, 2kg+1
template <> struct Scl<QT_PLANES> { h2 da, db; };
template <> struct Scl<QT_Q4_0> { h2 da, db; uint32_t qa[4]; };

__device__ __forceinline__ h2 splat(uint32_t hbits) {
    _Float16 v = __builtin_bit_cast(_Float16, (uint16_t)hbits);
    return h2{v, v};
}

__device__ __forceinline__ Scl<QT_Q4_K> scales(const Raw<QT_Q4_K>& raw, int kg) {
    const uint32_t s3[3] = {raw.hdr.y, raw.hdr.z, raw.hdr.w};
    const float d = half_bits_to_float(raw.hdr.x & 0xFFFFu);
    const float dmin = half_bits_to_float(raw.hdr.x >> 16);
    uint32_t sca, mna, scb, mnb;
    // sub-blocks 2kg and 2kg+1 (kg is lane-dependent; both branches are cheap)
    if (kg < 2) {
        sca = (s3[0] >> (16 * kg)) & 63u;       mna = (s3[1] >> (16 * kg)) & 63u;
        scb = (s3[0] >> (16 * kg + 8)) & 63u;   mnb = (s3[1] >> (16 * kg + 8)) & 63u;
    } else {
        q4k_scale_min(s3, 2 * kg, sca, mna);
        q4k_scale_min(s3, 2 * kg + 1, scb, mnb);
    }
    Scl<QT_Q4_K> o;
    _Float16 xa = (_Float16)(d * (float)sca), ya = (_Float16)(-(dmin * (float)mna));
    _Float16 xb = (_Float16)(d * (float)scb), yb = (_Float16)(-(dmin * (float)mnb));
    o.sa = h2{xa, xa}; o.ma = h2{ya, ya};
    o.sb = h2{xb, xb}; o.mb = h2{yb, yb};
    return o;
}

__device__ __forceinline__ Scl<QT_PLANES> scales(const Raw<QT_PLANES>& raw, int) {
    Scl<QT_PLANES> o;
    o.da = splat(raw.sc & 0xFFFFu);
    o.db = splat(raw.sc >> 16);
    return o;
}

__device__ __forceinline__ Scl<QT_Q4_0> scales(const Raw<QT_Q4_0>& raw, int) {
    Scl<QT_Q4_0> o;
    // block 2kg = bytes 0..17: d at 0, qs at 2..17 (realigned by 2 bytes)
    o.da = splat(raw.a.x & 0xFFFFu);
    o.qa[0] = __builtin_amdgcn_alignbit(raw.a.y, raw.a.x, 16);
    o.qa[1] = __builtin_amdgcn_alignbit(raw.a.z, raw.a.y, 16);
    o.qa[2] = __builtin_amdgcn_alignbit(raw.a.w, raw.a.z, 16);
    o.qa[3] = __builtin_amdgcn_alignbit(raw.b.x, raw.a.w, 16);
    // block 2kg+1 = bytes 18..35: d at 18, qs at 20..35 = words 5..8
    o.db = splat(raw.b.x >> 16);
    return o;
}

// Weights of MFMA i (elements 64kg + 8i .. +7 of the lane's run).
__device__ __forceinline__ h8 weights(const Magic& mg, const Raw<QT_Q4_K>& raw, const Scl<QT_Q4_K>& sc, int i) {
    const uint32_t w[8] = {raw.q0.x, raw.q0.y, raw.q0.z, raw.q0.w, raw.q1.x, raw.q1.y, raw.q1.z, raw.q1.w};
    const int t = i & 3;
    if (i < 4) return decode8_fma<false>(mg, w[2 * t], w[2 * t + 1], sc.sa, sc.ma);
    return decode8_fma<true>(mg, w[2 * t], w[2 * t + 1], sc.sb, sc.mb);
}

__device__ __forceinline__ h8 weights(const Magic& mg, const Raw<QT_PLANES>& raw, const Scl<QT_PLANES>& sc, int i) {
    const uint32_t w[8] = {raw.q0.x, raw.q0.y, raw.q0.z, raw.q0.w, raw.q1.x, raw.q1.y, raw.q1.z, raw.q1.w};
    return decode8_planes(mg, w[i], i < 4 ? sc.da : sc.db);
}

__device__ __forceinline__ h8 weights(const Magic& mg, const Raw<QT_Q4_0>& raw, const Scl<QT_Q4_0>& sc, int i) {
    const int t = i & 3;
    if (i < 4) {
        const uint32_t* q = sc.qa;
        return t < 2 ? decode8_q4_0<false>(mg, q[2 * t], q[2 * t + 1], sc.da)
                     : decode8_q4_0<true>(mg, q[2 * (t - 2)], q[2 * (t - 2) + 1], sc.da);
    }
    const uint32_t q[4] = {raw.b.y, raw.b.z, raw.b.w, raw.c};
    return t < 2 ? decode8_q4_0<false>(mg, q[2 * t], q[2 * t + 1], sc.db)
                 : decode8_q4_0<true>(mg, q[2 * (t - 2)], q[2 * (t - 2) + 1], sc.db);
}

template <int QT, int MT, int NT, int KW, int PF>
__global__ __launch_bounds__(64 * KW)
void k_gemm_mfma(const uint8_t* __restrict__ W, const uint8_t* __restrict__ Waux,
                 const uint16_t* __restrict__ A, int lda, void* __restrict__ C, int ldc, int out_f16,
                 int M, int N, int K) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r = lane & 15, kg = lane >> 4;
    const int nsg = K >> 8;
    const int64_t n0 = (int64_t)blockIdx.x * (16 * NT);
    const Magic mg = make_magic();

    int64_t rows[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) {
        int64_t n = n0 + 16 * t + r;
        rows[t] = n < N ? n : (int64_t)N - 1;       // clamp loads; stores are masked
    }
    const uint16_t* arow[MT];
    bool alive[MT];
#pragma unroll
    for (int mt = 0; mt < MT; mt++) {
        int m = 16 * mt + r;
        alive[mt] = m < M;
        arow[mt] = A + (int64_t)(m < M ? m : 0) * lda + 64 * kg;
    }

    f4 acc[MT][NT];
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int t = 0; t < NT; t++) acc[mt][t] = f4{0.f, 0.f, 0.f, 0.f};

    Raw<QT> ring[PF][NT];
#pragma unroll
    for (int p = 0; p < PF; p++) {
        int s = wave + KW * p;
        if (s < nsg) {
#pragma unroll
            for (int t = 0; t < NT; t++) load_raw<QT>(ring[p][t], W, Waux, rows[t], s, kg, K);
        }
    }

    for (int base = wave; base < nsg; base += KW * PF) {
#pragma unroll
        for (int p = 0; p < PF; p++) {
            const int s = base + KW * p;
            if (s < nsg) {
                h8 a[8][MT];
#pragma unroll
                for (int i = 0; i < 8; i++)
#pragma unroll
                    for (int mt = 0; mt < MT; mt++)
                        a[i][mt] = alive[mt] ? ld_act(arow[mt] + 256 * s + 8 * i) : h8{};
#pragma unroll
                for (int t = 0; t < NT; t++) {
                    Raw<QT> raw = ring[p][t];
                    auto sc = scales(raw, kg);
#pragma unroll
                    for (int i = 0; i < 8; i++) {
                        h8 b = weights(mg, raw, sc, i);
#pragma unroll
                        for (int mt = 0; mt < MT; mt++) acc[mt][t] = mfma16x16x32(a[i][mt], b, acc[mt][t]);
                    }
                }
                const int sn = s + KW * PF;
                if (sn < nsg) {
#pragma unroll
                    for (int t = 0; t < NT; t++) load_raw<QT>(ring[p][t], W, Waux, rows[t], sn, kg, K);
                }
            }
        }
    }

    // lane l holds D[m = 16mt + 4kg + i][n = n0 + 16t + r]
    if constexpr (KW == 1) {
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
#pragma unroll
            for (int t = 0; t < NT; t++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    int m = 16 * mt + 4 * kg + i;
                    int64_t n = n0 + 16 * t + r;
                    if (m < M && n < N) {
                        if (out_f16) ((_Float16*)C)[(int64_t)m * ldc + n] = (_Float16)acc[mt][t][i];
                        else ((float*)C)[(int64_t)m * ldc + n] = acc[mt][t][i];
                    }
                }
    } else {
        constexpr int TILE = MT * NT * 256;   // floats of one wave's partial tile
        __shared__ float red[KW * TILE];
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
#pragma unroll
            for (int t = 0; t < NT; t++)
#pragma unroll
                for (int i = 0; i < 4; i++)
                    red[wave * TILE + (((mt * NT + t) * 4 + i) * 64 + lane)] = acc[mt][t][i];
        __syncthreads();
        for (int idx = threadIdx.x; idx < TILE; idx += 64 * KW) {
            float v = 0.f;
#pragma unroll
            for (int w = 0; w < KW; w++) v += red[w * TILE + idx];
            const int ln = idx & 63, i = (idx >> 6) & 3, tt = idx >> 8;
            const int t = tt % NT, mt = tt / NT;
            const int m = 16 * mt + 4 * (ln >> 4) + i;
            const int64_t n = n0 + 16 * t + (ln & 15);
            if (m < M && n < N) {
                if (out_f16) ((_Float16*)C)[(int64_t)m * ldc + n] = (_Float16)v;
                else ((float*)C)[(int64_t)m * ldc + n] = v;
            }
        }
    }
}

// ---------------------------------------------------------------- host side
template <int QT, int MT, int NT, int KW, int PF>
static hipError_t launch_mfma(const GemmArgs& g, hipStream_t st) {
    const int64_t rows_per_block = 16 * NT;
    dim3 grid((unsigned)((g.N + rows_per_block - 1) / rows_per_block));
    hipLaunchKernelGGL((k_gemm_mfma<QT, MT, NT, KW, PF>), grid, dim3(64 * KW), 0, st,
                       g.W, g.Waux, g.A, g.lda, g.C, g.ldc, g.out_f16, g.M, g.N, g.K);
    return hipGetLastError();
}

template <int QT>
static hipError_t dispatch_mfma_qt(const GemmArgs& g, hipStream_t st) {
    const int mt = (g.M + 15) / 16;
    if (mt <= 1) return launch_mfma<QT, 1, 1, 4, 2>(g, st);
    if (mt <= 2) return launch_mfma<QT, 2, 1, 4, 2>(g, st);
    if (mt <= 4) return launch_mfma<QT, 4, 1, 4, 1>(g, st);
    return launch_mfma<QT, 8, 1, 2, 1>(g, st);
}

hipError_t gemm_mfma(const GemmArgs& g, hipStream_t st) {
    switch (g.qtype) {
        case QT_Q4_K: return dispatch_mfma_qt<QT_Q4_K>(g, st);
        case QT_PLANES: return dispatch_mfma_qt<QT_PLANES>(g, st);
        default: return dispatch_mfma_qt<QT_Q4_0>(g, st);
    }
}

}  // namespace bf
