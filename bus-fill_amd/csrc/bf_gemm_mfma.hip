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
#include "bf_formats.h"
#include "bf_launch.h"

namespace bf {

// One wave's share of the K loop: SPW super-groups s = wave, wave + KW, ...
// held in a register ring that is filled before any of it is consumed.
// ALDS: the workgroup first copies A[0:M][0:K] into LDS (rows padded by 16 B so
// the 16 lanes r of one kg group hit different banks) and every wave reads its
// fragments from there; used when M*K is small.  Otherwise fragments come from
// global memory (L2-resident: A is at most 128 x K fp16), one super-group ahead
// when registers allow.
//
// Every load is unconditional with clamped, in-bounds addresses (padding lanes
// read row 0, slots past the end reread the last super-group) and only stores
// and MFMAs are predicated: the compiler's wait counters then stay exact, so a
// slot is consumed as soon as ITS bytes have arrived.
template <int QT, int NT, int KW, int SPW>
__device__ __forceinline__ void ring_load(Raw<QT> (&ring)[SPW][NT], const uint8_t* W, const uint8_t* Waux,
                                          const int64_t (&rows)[NT], int kg, int s_first, int nsg, int K) {
#pragma unroll
    for (int p = 0; p < SPW; p++) {
        const int s = min(s_first + KW * p, nsg - 1);
#pragma unroll
        for (int t = 0; t < NT; t++) load_raw<QT>(ring[p][t], W, Waux, rows[t], s, kg, K);
    }
}

template <int QT, int MT, int NT, int KW, int SPW, bool ALDS>
__device__ __forceinline__ void ring_consume(f4 (&acc)[MT][NT], const Raw<QT> (&ring)[SPW][NT], const Magic& mg,
                                             const uint16_t* const (&arow)[MT], int kg, int s_first, int nsg) {
    constexpr bool APF = !ALDS && MT <= 2;            // prefetch A one super-group ahead
    h8 anext[APF ? 8 : 1][MT];
    if constexpr (APF) {
        const int s0 = min(s_first, nsg - 1);
#pragma unroll
        for (int i = 0; i < 8; i++)
#pragma unroll
            for (int mt = 0; mt < MT; mt++) anext[i][mt] = ld_act(arow[mt] + 256 * s0 + 8 * i);
    }
#pragma unroll
    for (int p = 0; p < SPW; p++) {
        const int s = s_first + KW * p;
        h8 a[8][MT];
        if constexpr (APF) {
#pragma unroll
            for (int i = 0; i < 8; i++)
#pragma unroll
                for (int mt = 0; mt < MT; mt++) a[i][mt] = anext[i][mt];
            if (p + 1 < SPW) {
                const int sa = min(s + KW, nsg - 1);
#pragma unroll
                for (int i = 0; i < 8; i++)
#pragma unroll
                    for (int mt = 0; mt < MT; mt++) anext[i][mt] = ld_act(arow[mt] + 256 * sa + 8 * i);
            }
        }
        if (s < nsg) {
            if constexpr (!APF) {
#pragma unroll
                for (int i = 0; i < 8; i++)
#pragma unroll
                    for (int mt = 0; mt < MT; mt++) a[i][mt] = *(const h8*)(arow[mt] + 256 * s + 8 * i);
            }
#pragma unroll
            for (int t = 0; t < NT; t++) {
                const Raw<QT>& raw = ring[p][t];
                auto sc = scales(raw, kg);
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    h8 b = weights(mg, raw, sc, i);
#pragma unroll
                    for (int mt = 0; mt < MT; mt++) acc[mt][t] = mfma16x16x32(a[i][mt], b, acc[mt][t]);
                }
            }
        }
    }
}

template <int QT, int MT, int NT, int KW, int SPW, bool ALDS>
__global__ __launch_bounds__(64 * KW)
void k_gemm_mfma(const uint8_t* __restrict__ W, const uint8_t* __restrict__ Waux,
                 const uint16_t* __restrict__ A, int lda, void* __restrict__ C, int ldc, int out_f16,
                 int M, int N, int K) {
    extern __shared__ __attribute__((aligned(16))) uint16_t a_lds[];
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
    // padding batch rows (m >= M) read row 0: their outputs are never stored
    const int astride = K + 8;                        // halves per LDS row
    const uint16_t* arow[MT];
#pragma unroll
    for (int mt = 0; mt < MT; mt++) {
        const int m = 16 * mt + r < M ? 16 * mt + r : 0;
        arow[mt] = ALDS ? a_lds + m * astride + 64 * kg : A + (int64_t)m * lda + 64 * kg;
    }

    f4 acc[MT][NT];
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int t = 0; t < NT; t++) acc[mt][t] = f4{0.f, 0.f, 0.f, 0.f};

    // Activations for LDS are loaded first (VMEM loads retire in order, so the
    // LDS writes wait for these only), then the weight ring goes out, then the
    // LDS writes and an LDS-only barrier: the weights stay in flight across it.
    // The one-pass case is a separate straight-line branch so that the compiler
    // does not fold it into the multi-pass loop (which would make it wait for
    // the whole ring before the first MFMA).
    constexpr int NSTAGE = ALDS ? 4 : 1;
    const int per_row = K >> 3, last = M * per_row - 1;
    auto stage_load = [&](h8 (&stage)[NSTAGE]) {
#pragma unroll
        for (int u = 0; u < NSTAGE; u++) {
            const int idx = min((int)threadIdx.x + u * 64 * KW, last);
            stage[u] = ld_act(A + (int64_t)(idx / per_row) * lda + 8 * (idx % per_row));
        }
    };
    auto stage_store = [&](const h8 (&stage)[NSTAGE]) {
#pragma unroll
        for (int u = 0; u < NSTAGE; u++) {
            const int idx = threadIdx.x + u * 64 * KW;
            if (idx <= last) *(h8*)(a_lds + (idx / per_row) * astride + 8 * (idx % per_row)) = stage[u];
        }
        for (int idx = threadIdx.x + NSTAGE * 64 * KW; idx <= last; idx += 64 * KW)
            *(h8*)(a_lds + (idx / per_row) * astride + 8 * (idx % per_row)) =
                ld_act(A + (int64_t)(idx / per_row) * lda + 8 * (idx % per_row));
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    };

    if (nsg <= KW * SPW) {
        h8 stage[NSTAGE];
        if constexpr (ALDS) stage_load(stage);
        Raw<QT> ring[SPW][NT];
        ring_load<QT, NT, KW, SPW>(ring, W, Waux, rows, kg, wave, nsg, K);
        if constexpr (ALDS) stage_store(stage);
        ring_consume<QT, MT, NT, KW, SPW, ALDS>(acc, ring, mg, arow, kg, wave, nsg);
    } else {
        if constexpr (ALDS) {
            h8 stage[NSTAGE];
            stage_load(stage);
            stage_store(stage);
        }
        for (int s_first = wave; s_first < nsg; s_first += KW * SPW) {
            Raw<QT> ring[SPW][NT];
            ring_load<QT, NT, KW, SPW>(ring, W, Waux, rows, kg, s_first, nsg, K);
            ring_consume<QT, MT, NT, KW, SPW, ALDS>(acc, ring, mg, arow, kg, s_first, nsg);
        }
    }

    // lane l holds D[m = 16mt + 4kg + i][n = n0 + 16t + r]; sum the KW split-K
    // partials in a fixed order (deterministic) and store
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
// LDS bytes of the staged activations: M rows of K + 8 halves.
static inline size_t alds_bytes(int M, int K) { return (size_t)M * (K + 8) * 2; }
#ifndef BF_ALDS_MAX
#define BF_ALDS_MAX (48 * 1024)
#endif
constexpr size_t kAldsMax = BF_ALDS_MAX;

template <int QT, int MT, int NT, int KW, int SPW, bool ALDS>
static hipError_t launch_mfma(const GemmArgs& g, hipStream_t st) {
    const int64_t rows_per_block = 16 * NT;
    dim3 grid((unsigned)((g.N + rows_per_block - 1) / rows_per_block));
    const size_t lds = ALDS ? alds_bytes(g.M, g.K) : 0;
    hipLaunchKernelGGL((k_gemm_mfma<QT, MT, NT, KW, SPW, ALDS>), grid, dim3(64 * KW), lds, st,
                       g.W, g.Waux, g.A, g.lda, g.C, g.ldc, g.out_f16, g.M, g.N, g.K);
    return hipGetLastError();
}

#ifndef BF_SMALL_KW
#define BF_SMALL_KW 8
#endif

template <int QT>
static hipError_t dispatch_mfma_qt(const GemmArgs& g, hipStream_t st) {
    const int mt = (g.M + 15) / 16;
    const int nsg = g.K / 256;
    if (mt <= 1 && alds_bytes(g.M, g.K) <= kAldsMax) {
        constexpr int KW = BF_SMALL_KW;
        if (nsg <= KW * 3) return launch_mfma<QT, 1, 1, KW, 3, true>(g, st);
        if (nsg <= KW * 5) return launch_mfma<QT, 1, 1, KW, 5, true>(g, st);
        return launch_mfma<QT, 1, 1, KW, 9, true>(g, st);
    }
    if (mt <= 1) {
        if (nsg <= 20) return launch_mfma<QT, 1, 1, 4, 5, false>(g, st);
        return launch_mfma<QT, 1, 1, 8, 5, false>(g, st);
    }
    if (mt <= 2) {
        if (nsg <= 12) return launch_mfma<QT, 2, 1, 4, 3, false>(g, st);
        return launch_mfma<QT, 2, 1, 8, 3, false>(g, st);
    }
    if (mt <= 4) return launch_mfma<QT, 4, 1, 4, 2, false>(g, st);
    return launch_mfma<QT, 8, 1, 2, 2, false>(g, st);
}

hipError_t gemm_mfma(const GemmArgs& g, hipStream_t st) {
    switch (g.qtype) {
        case QT_Q4_K: return dispatch_mfma_qt<QT_Q4_K>(g, st);
        case QT_PLANES: return dispatch_mfma_qt<QT_PLANES>(g, st);
        default: return dispatch_mfma_qt<QT_Q4_0>(g, st);
    }
}

}  // namespace bf
