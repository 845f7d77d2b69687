// Device-side building blocks shared by the busfill kernels (gfx950 only).
//
// Nibble -> fp16 uses the magic-bias construction that the reference builds
// with PRMT + LOP3 (kernels/busfill_v1a.cu:5-21,66-67,82-88), re-expressed with
// v_perm_b32 and v_and_or_b32:
//   v_perm_b32 spreads two code bytes b, b' into the two 16-bit halves
//   ([b, 0, b', 0]); v_and_or_b32 keeps one nibble per half and ORs in an fp16
//   exponent so that the half reads as an exact small integer plus a bias:
//     bits 0-3 | 0x6400  -> 1024 + q   (ulp 1    at 1024)
//     bits 4-7 | 0x5400  ->   64 + q   (ulp 1/16 at 64, nibble worth 16 ulps)
//   Subtracting the bias in fp16 (v_pk_add_f16) is exact, so the weight enters
//   the scale step as the exact integer q (or q - 8).  Unlike the reference's
//   sc/16 trick (kernels/busfill_v1a.cu:78, inexact once sc/16 is subnormal),
//   no scale is ever divided.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace bf {

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef float f16x __attribute__((ext_vector_type(16)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));

enum : int { QT_Q4_0 = 0, QT_PLANES = 1, QT_Q4_K = 2 };

// Bytes of one row of N x K weights: 4.5 bits per weight in every format
// (the planes layout counts only the code plane here; its scale plane is
// K/32 halves per row).
__host__ __device__ inline int64_t row_bytes(int qt, int K) {
    return qt == QT_PLANES ? (int64_t)K / 2 : (int64_t)K / 256 * 144;
}

__device__ __forceinline__ uint32_t perm_b32(uint32_t hi, uint32_t lo, uint32_t sel) {
    return __builtin_amdgcn_perm(hi, lo, sel);
}
__device__ __forceinline__ uint32_t and_or(uint32_t a, uint32_t mask, uint32_t bits) {
    return (a & mask) | bits;
}
__device__ __forceinline__ h2 as_h2(uint32_t x) { return __builtin_bit_cast(h2, x); }
__device__ __forceinline__ uint32_t as_u32(h2 x) { return __builtin_bit_cast(uint32_t, x); }

// byte spreads for v_perm_b32(x, x, sel): [b0,0,b1,0] and [b2,0,b3,0]
constexpr uint32_t SEL_B01 = 0x0C010C00u;
constexpr uint32_t SEL_B23 = 0x0C030C02u;
// [b,0,b,0] for byte b (planes layout: both nibbles of one byte are neighbours)
constexpr uint32_t SEL_BB0 = 0x0C000C00u;
constexpr uint32_t SEL_BB1 = 0x0C010C01u;
constexpr uint32_t SEL_BB2 = 0x0C020C02u;
constexpr uint32_t SEL_BB3 = 0x0C030C03u;

constexpr uint32_t LO_MASK = 0x000F000Fu, LO_BITS = 0x64006400u;   // 1024 + q
constexpr uint32_t HI_MASK = 0x00F000F0u, HI_BITS = 0x54005400u;   //   64 + q
constexpr uint32_t PL_MASK = 0x00F0000Fu, PL_BITS = 0x54006400u;   // {1024 + lo, 64 + hi}

// gfx9 VOP3 encodings take no literal constants, so (x & mask) | bits with two
// literals would become v_and_b32 + v_or_b32.  Holding mask and bits in VGPRs
// (materialised once per kernel, opaque to constant folding) lets the compiler
// select the single v_and_or_b32.
__device__ __forceinline__ uint32_t vreg_const(uint32_t c) {
    uint32_t r;
    asm("v_mov_b32 %0, %1" : "=v"(r) : "i"(c));
    return r;
}

struct Magic {
    uint32_t lo_mask, lo_bits, hi_mask, hi_bits, pl_mask, pl_bits;
};

__device__ __forceinline__ Magic make_magic() {
    return Magic{vreg_const(LO_MASK), vreg_const(LO_BITS), vreg_const(HI_MASK),
                 vreg_const(HI_BITS), vreg_const(PL_MASK), vreg_const(PL_BITS)};
}

__device__ __forceinline__ float half_bits_to_float(uint32_t h) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

// Q4_K scale/min of sub-block j from the 12 scale bytes held as three words
// (ggml get_scale_min_k4).
__device__ __forceinline__ void q4k_scale_min(const uint32_t s[3], int j, uint32_t& sc, uint32_t& m) {
    if (j < 4) {
        sc = (s[0] >> (8 * j)) & 63u;
        m = (s[1] >> (8 * j)) & 63u;
    } else {
        int t = j - 4;
        sc = ((s[2] >> (8 * t)) & 0xFu) | (((s[0] >> (8 * t + 6)) & 3u) << 4);
        m = ((s[2] >> (8 * t + 4)) & 0xFu) | (((s[1] >> (8 * t + 6)) & 3u) << 4);
    }
}

// Eight fp16 weights from eight code bytes (w0 = bytes 0-3, w1 = bytes 4-7),
// one nibble per byte (low nibbles when HI == false), in natural byte order:
// Q4_K, out = RN16(RN32(q*s - dm)), the oracle's (and ggml's) fp16 dequant of
// scale s = d*sc and offset dm = dmin*m, bit for bit.  v_perm_b32 spreads two
// code bytes into the halves of a word and one AND keeps one nibble per half,
// which read as fp16 is an exact subnormal: q * 2^-24 (low nibble) or
// 16 q * 2^-24 (high nibble, masked in place).  v_fma_mix_f32 takes that half
// as its fp16 operand, times s24 = s * 2^24 (low) or s * 2^20 (high), plus
// ndm = -dm, so it forms q*s - dm exactly and rounds it once to fp32;
// v_cvt_pk_f16_f32 then rounds two results to fp16 (RNE).  (v_fma_mix{lo,hi}_f16
// would round the exact value straight to fp16, which differs from the two
// roundings of the dequant in double-rounding cases.)
template <bool HI>
__device__ __forceinline__ h8 decode8_mix(uint32_t w0, uint32_t w1, float s24, float ndm) {
    const uint32_t mask = HI ? 0x00F000F0u : 0x000F000Fu;
    const uint32_t p[4] = {perm_b32(w0, w0, SEL_B01), perm_b32(w0, w0, SEL_B23),
                           perm_b32(w1, w1, SEL_B01), perm_b32(w1, w1, SEL_B23)};
    uint32_t o[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t x = p[i] & mask;                           // {q, q'} as fp16 subnormals
        float lo, hi;
        asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel_hi:[1,0,0]" : "=v"(lo) : "v"(x), "v"(s24), "v"(ndm));
        asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(hi) : "v"(x), "v"(s24), "v"(ndm));
        asm("v_cvt_pk_f16_f32 %0, %1, %2" : "=v"(o[i]) : "v"(lo), "v"(hi));
    }
    return __builtin_bit_cast(h8, u4{o[0], o[1], o[2], o[3]});
}

// Q4_K weights as exact small integers, for the factored product
//   sum_k a_k w_k = d * sum_k a_k (sc_j q_k) - dmin * sum_j m_j (sum_{k in j} a_k):
// (bias + q) * sc - bias * sc = sc * q <= 945 is exact in fp16 (s = {sc, sc},
// c = {-bias * sc, ...} are exact too), so one v_pk_fma_f16 yields two
// weights with no rounding at all.
template <bool HI>
__device__ __forceinline__ h8 decode8_int(const Magic& mg, uint32_t w0, uint32_t w1, h2 s, h2 c) {
    const uint32_t mask = HI ? mg.hi_mask : mg.lo_mask, bits = HI ? mg.hi_bits : mg.lo_bits;
    uint32_t p[4] = {perm_b32(w0, w0, SEL_B01), perm_b32(w0, w0, SEL_B23),
                     perm_b32(w1, w1, SEL_B01), perm_b32(w1, w1, SEL_B23)};
    h8 out;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const h2 v = __builtin_elementwise_fma(as_h2(and_or(p[i], mask, bits)), s, c);   // v_pk_fma_f16
        out[2 * i] = v[0];
        out[2 * i + 1] = v[1];
    }
    return out;
}

// Same for the Q4_0 formats: out = RN((q - 8) * d); (q - 8) is exact, so each
// element is bit-identical to the reference dequant RN_fp16((q-8)*d).
template <bool HI>
__device__ __forceinline__ h8 decode8_q4_0(const Magic& mg, uint32_t w0, uint32_t w1, h2 d) {
    const uint32_t mask = HI ? mg.hi_mask : mg.lo_mask, bits = HI ? mg.hi_bits : mg.lo_bits;
    const h2 unbias = HI ? h2{(_Float16)-72.0f, (_Float16)-72.0f} : h2{(_Float16)-1032.0f, (_Float16)-1032.0f};
    uint32_t p[4] = {perm_b32(w0, w0, SEL_B01), perm_b32(w0, w0, SEL_B23),
                     perm_b32(w1, w1, SEL_B01), perm_b32(w1, w1, SEL_B23)};
    h8 out;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        h2 q = as_h2(and_or(p[i], mask, bits)) + unbias;        // exact q - 8
        h2 v = q * d;                                           // v_pk_mul_f16
        out[2 * i] = v[0];
        out[2 * i + 1] = v[1];
    }
    return out;
}

// Planes layout: byte b holds elements 2b (low nibble) and 2b+1 (high nibble),
// so one v_perm_b32 [b,0,b,0] plus one v_and_or_b32 with mixed mask/bias gives
// the natural-order pair {1024 + lo, 64 + hi}.
__device__ __forceinline__ h8 decode8_planes(const Magic& mg, uint32_t w, h2 d) {
    const uint32_t mask = mg.pl_mask, bits = mg.pl_bits;
    const h2 unbias = h2{(_Float16)-1032.0f, (_Float16)-72.0f};
    uint32_t p[4] = {perm_b32(w, w, SEL_BB0), perm_b32(w, w, SEL_BB1),
                     perm_b32(w, w, SEL_BB2), perm_b32(w, w, SEL_BB3)};
    h8 out;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        h2 q = as_h2(and_or(p[i], mask, bits)) + unbias;        // exact {q0-8, q1-8}
        h2 v = q * d;
        out[2 * i] = v[0];
        out[2 * i + 1] = v[1];
    }
    return out;
}

__device__ __forceinline__ f4 mfma16x16x32(h8 a, h8 b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// 32 x 32 output tile, k = 16: lane l holds row l % 32 of A and column l % 32 of
// B, eight elements each (the same eight k for A and B in lanes l and l + 32k
// alike); D's element (i, j) is register 4 (i / 8) + i % 4 of lane
// j + 32 ((i / 4) % 2).  Per flop the fastest f16 MFMA of gfx950 (2.2 PFLOP/s
// issued back to back, against 1.4 for 16x16x32).
__device__ __forceinline__ f16x mfma32x32x16(h8 a, h8 b, f16x c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// SiLU(g) * u rounded to fp16, computed in fp32 as g * (1 / (1 + e^-g)) * u
// with e^-g = 2^(-g log2 e) on the hardware exp2 and the hardware reciprocal
// (each within about one fp32 ulp; the fused GEMM evaluates this in every
// workgroup, where a correctly rounded exp and division cost several
// microseconds at K = 17408).  The one formula of the fused down-projection
// GEMM and of the standalone kernel, so the two give the same bits.  Very
// negative g: e^-g = inf, reciprocal 0, result -0 or 0; very positive g: g * u.
__device__ __forceinline__ _Float16 swiglu_f16(_Float16 g, _Float16 u) {
    const float gf = (float)g;
    const float e = __builtin_amdgcn_exp2f(gf * -1.44269504088896341f);
    return (_Float16)(gf * __builtin_amdgcn_rcpf(1.0f + e) * (float)u);
}

// Eight fp16 pairs (16 bytes of gate, 16 of up) -> eight fp16 swiglu values.
__device__ __forceinline__ u4 swiglu8v(u4 gv, u4 uv) {
    u4 r;
#pragma unroll
    for (int w = 0; w < 4; w++) {
        const uint32_t gw = gv[w], uw = uv[w];
        const _Float16 lo = swiglu_f16(__builtin_bit_cast(_Float16, (uint16_t)(gw & 0xFFFF)),
                                       __builtin_bit_cast(_Float16, (uint16_t)(uw & 0xFFFF)));
        const _Float16 hi = swiglu_f16(__builtin_bit_cast(_Float16, (uint16_t)(gw >> 16)),
                                       __builtin_bit_cast(_Float16, (uint16_t)(uw >> 16)));
        r[w] = (uint32_t)__builtin_bit_cast(uint16_t, lo) | ((uint32_t)__builtin_bit_cast(uint16_t, hi) << 16);
    }
    return r;
}

__device__ __forceinline__ u4 swiglu8(const uint16_t* g, const uint16_t* u) {
    return swiglu8v(*(const u4*)g, *(const u4*)u);
}

// Eight fp32 activations (32 bytes, 16-byte aligned) rounded to fp16 (nearest
// even: the conversion instruction's rounding, as an fp32 -> fp16 copy does).
__device__ __forceinline__ u4 f32x8_to_f16(const float* x) {
    typedef float f4v __attribute__((ext_vector_type(4)));
    const f4v a = *(const f4v*)x, b = *(const f4v*)(x + 4);
    auto pk = [](float lo, float hi) {
        return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)lo) |
               ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)hi) << 16);
    };
    return u4{pk(a[0], a[1]), pk(a[2], a[3]), pk(b[0], b[1]), pk(b[2], b[3])};
}

}  // namespace bf
