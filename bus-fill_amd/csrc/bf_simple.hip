// Bit-exact fp16 dequant kernels and the shape-generic GEMM fallback.
//
// Dequant contract (one rounding to fp16 of a value formed exactly in fp32):
//   Q4_0 formats: RN_fp16((q - 8) * fp32(d))          kernels/busfill_v0.cu:74,78-81
//   Q4_K        : RN_fp16((d*sc)*q - dmin*m)          ggml dequantize_row_q4_K
// (q - 8) * d and (d*sc)*q are exact products in fp32, so fused and unfused
// evaluation agree and the only rounding is the final v_cvt_f16_f32 (RNE,
// fp16 denormals preserved).
#include "bf_device.h"
#include "bf_launch.h"

namespace bf {

__device__ __forceinline__ uint32_t ld_u8(const uint8_t* p) { return *p; }
__device__ __forceinline__ uint32_t ld_u16_bytes(const uint8_t* p) { return (uint32_t)p[0] | ((uint32_t)p[1] << 8); }

// Element k of row n as fp32 (value before the fp16 rounding).
__device__ __forceinline__ float elem_f32(int qt, const uint8_t* W, const uint8_t* Waux, int64_t n, int k, int K) {
    if (qt == QT_PLANES) {
        uint32_t b = ld_u8(W + n * (int64_t)(K >> 1) + (k >> 1));
        uint32_t q = (k & 1) ? (b >> 4) : (b & 0xF);
        float d = half_bits_to_float(ld_u16_bytes(Waux + 2 * (n * (int64_t)(K >> 5) + (k >> 5))));
        return (float)((int)q - 8) * d;
    }
    if (qt == QT_Q4_0) {
        const uint8_t* blk = W + n * (int64_t)(K >> 5) * 18 + (int64_t)(k >> 5) * 18;
        int e = k & 31;
        uint32_t b = ld_u8(blk + 2 + (e & 15));
        uint32_t q = e < 16 ? (b & 0xF) : (b >> 4);
        return (float)((int)q - 8) * half_bits_to_float(ld_u16_bytes(blk));
    }
    const uint8_t* blk = W + n * (int64_t)(K >> 8) * 144 + (int64_t)(k >> 8) * 144;
    int e = k & 255, c = e >> 6, l = e & 31, hi = (e >> 5) & 1;
    uint32_t s3[3];
    for (int i = 0; i < 3; i++)
        s3[i] = ld_u8(blk + 4 + 4 * i) | (ld_u8(blk + 5 + 4 * i) << 8) | (ld_u8(blk + 6 + 4 * i) << 16) |
                (ld_u8(blk + 7 + 4 * i) << 24);
    uint32_t sc, m;
    q4k_scale_min(s3, 2 * c + hi, sc, m);
    uint32_t b = ld_u8(blk + 16 + 32 * c + l);
    uint32_t q = hi ? (b >> 4) : (b & 0xF);
    float d = half_bits_to_float(ld_u16_bytes(blk)), dmin = half_bits_to_float(ld_u16_bytes(blk + 2));
    return __builtin_fmaf(d * (float)sc, (float)q, -(dmin * (float)m));
}

// One thread per 32-element group (a Q4_0 block or a Q4_K sub-block).
__global__ __launch_bounds__(256) void k_dequant_f16(int qt, const uint8_t* __restrict__ W,
                                                     const uint8_t* __restrict__ Waux,
                                                     uint16_t* __restrict__ out, int N, int K) {
    const int64_t groups = (int64_t)N * (K >> 5);
    for (int64_t g = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; g < groups;
         g += (int64_t)gridDim.x * blockDim.x) {
        const int64_t n = g / (K >> 5);
        const int k0 = (int)(g % (K >> 5)) * 32;
        uint16_t* dst = out + n * (int64_t)K + k0;
#pragma unroll 4
        for (int j = 0; j < 32; j++) {
            _Float16 h = (_Float16)elem_f32(qt, W, Waux, n, k0 + j, K);
            dst[j] = __builtin_bit_cast(uint16_t, h);
        }
    }
}

hipError_t dequant_f16(int qtype, const uint8_t* W, const uint8_t* Waux, uint16_t* out, int N, int K,
                       hipStream_t st) {
    const int64_t groups = (int64_t)N * (K >> 5);
    int64_t blocks = (groups + 255) / 256;
    if (blocks > 8192) blocks = 8192;
    hipLaunchKernelGGL(k_dequant_f16, dim3((unsigned)blocks), dim3(256), 0, st, qtype, W, Waux, out, N, K);
    return hipGetLastError();
}

// Shape-generic GEMM: one thread per output, fp32 accumulation over the exact
// fp32 element values.  Serves legal shapes the fast kernels do not (K not a
// multiple of 256, unaligned operands).
__global__ __launch_bounds__(256) void k_gemm_simple(int qt, const uint8_t* __restrict__ W,
                                                     const uint8_t* __restrict__ Waux,
                                                     const uint16_t* __restrict__ A, int lda,
                                                     void* __restrict__ C, int ldc, int out_f16,
                                                     int M, int N, int K) {
    const int64_t n = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    const int m = blockIdx.y;
    if (n >= N || m >= M) return;
    const uint16_t* a = A + (int64_t)m * lda;
    float acc = 0.f;
    for (int k = 0; k < K; k++) {
        float av = (float)__builtin_bit_cast(_Float16, a[k]);
        acc = __builtin_fmaf(av, elem_f32(qt, W, Waux, n, k, K), acc);
    }
    if (out_f16) ((_Float16*)C)[(int64_t)m * ldc + n] = (_Float16)acc;
    else ((float*)C)[(int64_t)m * ldc + n] = acc;
}

hipError_t gemm_simple(const GemmArgs& g, hipStream_t st) {
    dim3 grid((unsigned)((g.N + 255) / 256), (unsigned)g.M);
    hipLaunchKernelGGL(k_gemm_simple, grid, dim3(256), 0, st, g.qtype, g.W, g.Waux, g.A, g.lda, g.C, g.ldc,
                       g.out_f16, g.M, g.N, g.K);
    return hipGetLastError();
}

// out[m][k] = SiLU(gu[m][k]) * gu[m][K + k] in fp16 (the formula the fused
// down-projection GEMM applies while loading A), eight elements per thread.
// out may be gu itself (in place over the gate half): each thread reads its
// eight gate and eight up values before it writes the eight results.
__global__ __launch_bounds__(256) void k_swiglu_f16(const uint16_t* gu, int ld, uint16_t* out, int ldo, int M,
                                                    int K) {
    const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;   // group of eight in a row
    const int per_row = K >> 3;
    if (i >= (int64_t)M * per_row) return;
    const int m = (int)(i / per_row), k = (int)(i - (int64_t)m * per_row) * 8;
    const uint16_t* g = gu + (int64_t)m * ld + k;
    *(u4*)(out + (int64_t)m * ldo + k) = swiglu8(g, g + K);
}

hipError_t swiglu_f16(const uint16_t* gu, int ld, uint16_t* out, int ldo, int M, int K, hipStream_t st) {
    const int64_t groups = (int64_t)M * (K >> 3);
    hipLaunchKernelGGL(k_swiglu_f16, dim3((unsigned)((groups + 255) / 256)), dim3(256), 0, st, gu, ld, out, ldo, M, K);
    return hipGetLastError();
}

}  // namespace bf
