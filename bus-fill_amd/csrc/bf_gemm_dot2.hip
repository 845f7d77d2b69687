// Small-batch GEMM (M <= 2) on v_dot2_f32_f16, streaming whole weight rows.
//
// Replaces the reference's busfill_q4 kernel (kernels/busfill_v1a.cu:41-104) for
// decode batches of one or two streams, where an MFMA tile would be 15/16 idle.
//
// Memory layout read as-is (llama.cpp block_q4_K, 144 B per 256 weights): one
// wave streams one weight row.  Each load instruction covers 63 lanes x 16 B =
// 1008 contiguous bytes = exactly seven super-blocks, so every wave-level load
// is contiguous; lane 9j+0 holds super-block j's header (d, dmin, scales[12]),
// lanes 9j+1 .. 9j+8 hold its 128 code bytes, 16 B each; lane 63 idles.
//
// Decode without a magic bias: (w & 0x000F000F) read as fp16 is the exact
// SUBNORMAL pair {q0 * 2^-24, q2 * 2^-24}, and (w & 0x00F000F0) is
// {q0', q2'} * 2^-20 for the high nibbles, so one shift and four v_and_b32
// turn four code bytes into eight fp16 weights that v_dot2_f32_f16 multiplies
// exactly (products of an fp16 activation and a 4-bit integer fit fp32).  The
// pairing {byte0, byte2}, {byte1, byte3} is matched by storing the activations
// in LDS with elements 1 and 2 of every group of four swapped.
//
// Per 16-element half-chunk the lane accumulates p = sum A*q (times 2^-24 or
// 2^-20) and folds it as  acc += (d*sc * 2^24|2^20) * p - (dmin*m) * S, where S
// is the sum of the same 16 activations, computed once per workgroup while the
// activations are staged.  Header lanes decode the eight (d*sc, dmin*m) pairs of
// their super-block into a per-wave LDS table read by the code lanes.
#include "bf_device.h"
#include "bf_launch.h"

namespace bf {

namespace {

constexpr int kWaves = 4;              // waves (= weight rows) per workgroup
constexpr int kSgPerLoad = 7;          // super-blocks per 1008-byte load

__device__ __forceinline__ uint32_t lds_a_index(int k) {    // padded LDS offset (halves) of element k
    return (uint32_t)(k + ((k >> 8) << 3));                 // +16 B after every 256 elements
}

}  // namespace

template <int MB, int NU, int NL>
__global__ __launch_bounds__(64 * kWaves)
void k_gemm_dot2_q4k(const uint8_t* __restrict__ W, const uint16_t* __restrict__ A, int lda,
                     void* __restrict__ C, int ldc, int out_f16, int M, int N, int K) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int nsg = K >> 8;
    const int astride = K + ((K >> 8) << 3);                // padded halves per batch row
    _Float16* a_lds = (_Float16*)lds;                        // [MB][astride]
    float* s_lds = (float*)(lds + (size_t)MB * astride * 2);  // [MB][K/16]
    float* sc_lds = s_lds + MB * (K >> 4);                    // [kWaves][7][4][4]

    // 1. activation staging loads first (VMEM loads retire in order: the LDS
    //    writes below then wait for these only, not for the weight stream)
    const int units = MB * (K >> 4);                         // 16-element units
    u4 st[NU][2];
#pragma unroll
    for (int u = 0; u < NU; u++) {
        int idx = min((int)threadIdx.x + u * 64 * kWaves, units - 1);
        const int m = idx / (K >> 4), kk = (idx - m * (K >> 4)) << 4;
        const uint16_t* src = A + (int64_t)min(m, M - 1) * lda + kk;
        st[u][0] = *(const u4*)src;
        st[u][1] = *(const u4*)(src + 8);
    }

    // 2. this wave's weight row: NL loads of 16 B per lane, all in flight
    const int64_t row = (int64_t)blockIdx.x * kWaves + wave;
    const int64_t rowc = row < N ? row : (int64_t)N - 1;
    const uint8_t* wrow = W + rowc * ((int64_t)nsg * 144);
    const int sgl = lane / 9, piece = lane - 9 * sgl;         // lane 63: sgl = 7 (idle)
    u4 wv[NL];
#pragma unroll
    for (int i = 0; i < NL; i++) {
        int s = min(kSgPerLoad * i + sgl, nsg - 1);
        wv[i] = *(const u4*)(wrow + (int64_t)s * 144 + 16 * piece);
    }

    // 3. activations -> LDS (elements 1,2 of each group of four swapped) and the
    //    16-element sums
#pragma unroll
    for (int u = 0; u < NU; u++) {
        const int idx = threadIdx.x + u * 64 * kWaves;
        if (idx < units) {
            const int m = idx / (K >> 4), kk = (idx - m * (K >> 4)) << 4;
            float s = 0.f;
            uint32_t o[8];
            const uint32_t in[8] = {st[u][0].x, st[u][0].y, st[u][0].z, st[u][0].w,
                                    st[u][1].x, st[u][1].y, st[u][1].z, st[u][1].w};
#pragma unroll
            for (int g = 0; g < 4; g++) {
                // halves {a0,a1},{a2,a3} -> {a0,a2},{a1,a3}
                const uint32_t lo = in[2 * g], hi = in[2 * g + 1];
                o[2 * g] = perm_b32(hi, lo, 0x05040100u);
                o[2 * g + 1] = perm_b32(hi, lo, 0x07060302u);
                h2 x = as_h2(lo), y = as_h2(hi);
                s += (float)x[0] + (float)x[1] + (float)y[0] + (float)y[1];
            }
            _Float16* dst = a_lds + m * astride + lds_a_index(kk);
            *(u4*)dst = u4{o[0], o[1], o[2], o[3]};
            *(u4*)(dst + 8) = u4{o[4], o[5], o[6], o[7]};
            s_lds[m * (K >> 4) + (kk >> 4)] = s;
        }
    }
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");

    // 4. stream the row: for every load, header lanes publish scales, code
    //    lanes dot and fold
    float acc[MB];
#pragma unroll
    for (int m = 0; m < MB; m++) acc[m] = 0.f;
    float* sct = sc_lds + wave * (kSgPerLoad * 16);
    const uint32_t mlo = vreg_const(0x000F000Fu), mhi = vreg_const(0x00F000F0u);
#pragma unroll
    for (int i = 0; i < NL; i++) {
        const int s = kSgPerLoad * i + sgl;
        const bool live = sgl < kSgPerLoad && s < nsg;
        if (live && piece == 0) {
            const u4 h = wv[i];
            const float d = half_bits_to_float(h.x & 0xFFFFu), dmin = half_bits_to_float(h.x >> 16);
            const uint32_t s3[3] = {h.y, h.z, h.w};
#pragma unroll
            for (int c = 0; c < 4; c++) {
                uint32_t sa, ma, sb, mb;
                q4k_scale_min(s3, 2 * c, sa, ma);
                q4k_scale_min(s3, 2 * c + 1, sb, mb);
                *(float4*)(sct + sgl * 16 + 4 * c) =
                    make_float4(d * (float)sa * 16777216.0f, dmin * (float)ma, d * (float)sb * 1048576.0f,
                                dmin * (float)mb);
            }
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        if (live && piece != 0) {
            const int c = (piece - 1) >> 1, hh = (piece - 1) & 1;
            const float4 sc = *(const float4*)(sct + sgl * 16 + 4 * c);
            const int klo = 256 * s + 64 * c + 16 * hh, khi = klo + 32;
            const uint32_t w[4] = {wv[i].x, wv[i].y, wv[i].z, wv[i].w};
#pragma unroll
            for (int m = 0; m < MB; m++) {
                const _Float16* ab = a_lds + m * astride;
                const u4 al0 = *(const u4*)(ab + lds_a_index(klo)), al1 = *(const u4*)(ab + lds_a_index(klo + 8));
                const u4 ah0 = *(const u4*)(ab + lds_a_index(khi)), ah1 = *(const u4*)(ab + lds_a_index(khi + 8));
                const uint32_t al[8] = {al0.x, al0.y, al0.z, al0.w, al1.x, al1.y, al1.z, al1.w};
                const uint32_t ah[8] = {ah0.x, ah0.y, ah0.z, ah0.w, ah1.x, ah1.y, ah1.z, ah1.w};
                float plo = 0.f, phi = 0.f;
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const uint32_t x = w[j], y = w[j] >> 8;
                    plo = __builtin_amdgcn_fdot2(as_h2(al[2 * j]), as_h2(x & mlo), plo, false);
                    plo = __builtin_amdgcn_fdot2(as_h2(al[2 * j + 1]), as_h2(y & mlo), plo, false);
                    phi = __builtin_amdgcn_fdot2(as_h2(ah[2 * j]), as_h2(x & mhi), phi, false);
                    phi = __builtin_amdgcn_fdot2(as_h2(ah[2 * j + 1]), as_h2(y & mhi), phi, false);
                }
                const float slo = s_lds[m * (K >> 4) + (klo >> 4)], shi = s_lds[m * (K >> 4) + (khi >> 4)];
                acc[m] = __builtin_fmaf(sc.x, plo, acc[m]);
                acc[m] = __builtin_fmaf(-sc.y, slo, acc[m]);
                acc[m] = __builtin_fmaf(sc.z, phi, acc[m]);
                acc[m] = __builtin_fmaf(-sc.w, shi, acc[m]);
            }
        }
    }

    // 5. wave reduction (fixed butterfly order) and store
#pragma unroll
    for (int m = 0; m < MB; m++) {
        float v = acc[m];
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
        acc[m] = v;
    }
    if (lane == 0 && row < N) {
#pragma unroll
        for (int m = 0; m < MB; m++) {
            if (m < M) {
                if (out_f16) ((_Float16*)C)[(int64_t)m * ldc + row] = (_Float16)acc[m];
                else ((float*)C)[(int64_t)m * ldc + row] = acc[m];
            }
        }
    }
}

namespace {

size_t dot2_lds_bytes(int MB, int K) {
    const size_t astride = (size_t)K + ((K >> 8) << 3);
    return (size_t)MB * astride * 2 + (size_t)MB * (K >> 4) * 4 + (size_t)kWaves * kSgPerLoad * 16 * 4;
}

template <int MB, int NU, int NL>
hipError_t launch_dot2(const GemmArgs& g, hipStream_t st) {
    dim3 grid((unsigned)((g.N + kWaves - 1) / kWaves));
    hipLaunchKernelGGL((k_gemm_dot2_q4k<MB, NU, NL>), grid, dim3(64 * kWaves), dot2_lds_bytes(MB, g.K), st, g.W,
                       g.A, g.lda, g.C, g.ldc, g.out_f16, g.M, g.N, g.K);
    return hipGetLastError();
}

// NL (loads per lane) covers ceil(K/256 / 7) super-block groups; NU covers the
// staging units MB*K/16 over 256 threads.
template <int MB>
hipError_t dispatch_nl(const GemmArgs& g, hipStream_t st) {
    const int nl = (g.K / 256 + kSgPerLoad - 1) / kSgPerLoad;
    const int nu = (MB * (g.K / 16) + 64 * kWaves - 1) / (64 * kWaves);
    if (nl <= 3 && nu <= 3) return launch_dot2<MB, 3, 3>(g, st);
    if (nl <= 4 && nu <= 4) return launch_dot2<MB, 4, 4>(g, st);
    if (nl <= 10 && nu <= 9) return launch_dot2<MB, 9, 10>(g, st);
    return hipErrorNotSupported;
}

}  // namespace

bool dot2_supports(const GemmArgs& g) {
    if (g.qtype != QT_Q4_K || g.M > 2 || g.K % 256 != 0) return false;
    const int mb = g.M;
    const int nl = (g.K / 256 + kSgPerLoad - 1) / kSgPerLoad;
    const int nu = (mb * (g.K / 16) + 64 * kWaves - 1) / (64 * kWaves);
    return nl <= 10 && nu <= 9 && dot2_lds_bytes(mb, g.K) <= 64 * 1024;
}

hipError_t gemm_dot2(const GemmArgs& g, hipStream_t st) {
    if (!dot2_supports(g)) return hipErrorNotSupported;
    return g.M == 1 ? dispatch_nl<1>(g, st) : dispatch_nl<2>(g, st);
}

}  // namespace bf
