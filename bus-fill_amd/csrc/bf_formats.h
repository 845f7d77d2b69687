// Per-format register image of one lane's 64-weight run of a 256-weight
// super-group, and its decode into pre-scaled fp16 MFMA operands.  Shared by
// the register-streaming and the LDS-staged MFMA kernels.
//
// Lane (r = l%16, kg = l/16) owns, for super-group s of row r, the 64 weights
// k = 256s + 64kg + 8i + j (i = 0..7 selects the MFMA, j the element):
//   Q4_K  : chunk kg of qs[128] (32 B, sub-blocks 2kg and 2kg+1) + the header
//   planes: code bytes 32kg..32kg+31 of the row + the two fp16 block scales
//   Q4_0  : 18-byte blocks 2kg and 2kg+1 (36 B)
#pragma once

#include "bf_device.h"

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
// Q4_K: d*sc * 2^24 (sub-block 2kg, low nibbles) and d*sc * 2^20 (2kg+1, high
// nibbles), and -dmin*m of each: the operands of decode8_mix
template <> struct Scl<QT_Q4_K> { float sa, ca, sb, cb; };
template <> struct Scl<QT_PLANES> { h2 da, db; };
template <> struct Scl<QT_Q4_0> { h2 da, db; uint32_t qa[4]; };

__device__ __forceinline__ h2 splat(uint32_t hbits) {
    _Float16 v = __builtin_bit_cast(_Float16, (uint16_t)hbits);
    return h2{v, v};
}

__device__ __forceinline__ Scl<QT_Q4_K> scales(const Raw<QT_Q4_K>& raw, int kg) {
    // (scale, min) codes of sub-blocks 2kg and 2kg+1, two bytes at a time and
    // without branches: for kg < 2 they are the low six bits of scale bytes
    // 2kg, 2kg+1 and 2kg+4, 2kg+5; for kg >= 2 they are assembled from the
    // nibbles of bytes 8..11 and the top two bits of bytes 0..7.
    const uint32_t s0 = raw.hdr.y, s1 = raw.hdr.z, s2 = raw.hdr.w;
    const uint32_t sh = 16u * (uint32_t)(kg & 1);
    const uint32_t sc_lo = (s0 >> sh) & 0x3F3Fu, mn_lo = (s1 >> sh) & 0x3F3Fu;
    const uint32_t sc_hi = ((s2 >> sh) & 0x0F0Fu) | ((s0 >> (sh + 2)) & 0x3030u);
    const uint32_t mn_hi = ((s2 >> (sh + 4)) & 0x0F0Fu) | ((s1 >> (sh + 2)) & 0x3030u);
    const uint32_t sc = kg < 2 ? sc_lo : sc_hi, mn = kg < 2 ? mn_lo : mn_hi;
    const float d = half_bits_to_float(raw.hdr.x & 0xFFFFu);
    const float dmin = half_bits_to_float(raw.hdr.x >> 16);
    Scl<QT_Q4_K> o;
    // d*sc and dmin*m are exact in fp32 (at most 17 significant bits), and so
    // are their power-of-two multiples (d*sc < 2^22: no overflow)
    o.sa = d * (float)(sc & 0xFFu) * 16777216.0f;
    o.ca = -(dmin * (float)(mn & 0xFFu));
    o.sb = d * (float)(sc >> 8) * 1048576.0f;
    o.cb = -(dmin * (float)(mn >> 8));
    return o;
}

// Per-lane state of the factored Q4_K product (integer weights sc * q, the
// scales and mins applied per super-group outside the MFMA):
//   s_lo/c_lo, s_hi/c_hi: fp16 {sc, sc} and {-bias*sc, ...} of sub-blocks 2kg
//     (low nibbles, bias 1024) and 2kg+1 (high nibbles, bias 64);
//   min_hi, min_lo: fp16 {32 m, 32 m'} and {m / 64, m' / 64} of the same two
//     sub-blocks, the MFMA operand that meets the activation block sums;
//   d, dmin: the super-block's fp32 scales.
struct SclK {
    h2 s_lo, c_lo, s_hi, c_hi;
    uint32_t min_hi, min_lo;
    float d, dmin;
};

__device__ __forceinline__ SclK scales_int(const Raw<QT_Q4_K>& raw, int kg) {
    const uint32_t s0 = raw.hdr.y, s1 = raw.hdr.z, s2 = raw.hdr.w;
    const uint32_t sh = 16u * (uint32_t)(kg & 1);
    const uint32_t sc_lo = (s0 >> sh) & 0x3F3Fu, mn_lo = (s1 >> sh) & 0x3F3Fu;
    const uint32_t sc_hi = ((s2 >> sh) & 0x0F0Fu) | ((s0 >> (sh + 2)) & 0x3030u);
    const uint32_t mn_hi = ((s2 >> (sh + 4)) & 0x0F0Fu) | ((s1 >> (sh + 2)) & 0x3030u);
    const uint32_t sc = kg < 2 ? sc_lo : sc_hi, mn = kg < 2 ? mn_lo : mn_hi;
    // six-bit codes v to fp16 through the exponent of 1024: bits 0x6400 | v are 1024 + v
    const uint32_t e1024 = 0x64646464u;
    const h2 k1024 = {(_Float16)1024.0f, (_Float16)1024.0f};
    SclK o;
    o.s_lo = as_h2(perm_b32(e1024, sc, 0x04000400u)) - k1024;        // {sc, sc} of sub-block 2kg
    o.s_hi = as_h2(perm_b32(e1024, sc, 0x04010401u)) - k1024;        // of sub-block 2kg+1
    o.c_lo = o.s_lo * h2{(_Float16)-1024.0f, (_Float16)-1024.0f};
    o.c_hi = o.s_hi * h2{(_Float16)-64.0f, (_Float16)-64.0f};
    const h2 mb = as_h2(perm_b32(e1024, mn, 0x04010400u));            // {1024 + m, 1024 + m'}
    o.min_hi = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(
        mb, h2{(_Float16)32.0f, (_Float16)32.0f}, h2{(_Float16)-32768.0f, (_Float16)-32768.0f}));
    o.min_lo = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(
        mb, h2{(_Float16)0.015625f, (_Float16)0.015625f}, h2{(_Float16)-16.0f, (_Float16)-16.0f}));
    o.d = half_bits_to_float(raw.hdr.x & 0xFFFFu);
    o.dmin = half_bits_to_float(raw.hdr.x >> 16);
    return o;
}

// Per-lane state of the sub-block rows form (codes enter the MFMA as fp16
// subnormals; scales applied to the per-sub-block sums afterwards):
//   c_lo16 = 16 sc and c_hi = sc of sub-blocks 2kg and 2kg+1 (the low codes are
//   q * 2^-24, the high ones 16 q * 2^-24, so d20 * c * P recovers d sc sum a q),
//   m_lo, m_hi their mins, d20 = d * 2^20, dmin.
struct BdScl {
    float c_lo16, c_hi, m_lo, m_hi, d20, dmin;
};

__device__ __forceinline__ BdScl scales_bd(const Raw<QT_Q4_K>& raw, int kg) {
    const uint32_t s0 = raw.hdr.y, s1 = raw.hdr.z, s2 = raw.hdr.w;
    const uint32_t sh = 16u * (uint32_t)(kg & 1);
    const uint32_t sc_lo = (s0 >> sh) & 0x3F3Fu, mn_lo = (s1 >> sh) & 0x3F3Fu;
    const uint32_t sc_hi = ((s2 >> sh) & 0x0F0Fu) | ((s0 >> (sh + 2)) & 0x3030u);
    const uint32_t mn_hi = ((s2 >> (sh + 4)) & 0x0F0Fu) | ((s1 >> (sh + 2)) & 0x3030u);
    const uint32_t sc = kg < 2 ? sc_lo : sc_hi, mn = kg < 2 ? mn_lo : mn_hi;
    BdScl o;
    o.c_lo16 = (float)(sc & 0xFFu) * 16.0f;
    o.c_hi = (float)(sc >> 8);
    o.m_lo = (float)(mn & 0xFFu);
    o.m_hi = (float)(mn >> 8);
    o.d20 = half_bits_to_float(raw.hdr.x & 0xFFFFu) * 1048576.0f;
    o.dmin = half_bits_to_float(raw.hdr.x >> 16);
    return o;
}

// The lane's 32 code bytes for the sub-block rows form, as eight words: Q4_K
// the run of sub-blocks 2kg (low nibbles) and 2kg+1 (high nibbles); Q4_0 and
// planes the code bytes of blocks 2kg (words 0-3) and 2kg+1 (words 4-7).
__device__ __forceinline__ void bd_code_words(const Raw<QT_Q4_K>& raw, uint32_t w[8]) {
    const uint32_t v[8] = {raw.q0.x, raw.q0.y, raw.q0.z, raw.q0.w, raw.q1.x, raw.q1.y, raw.q1.z, raw.q1.w};
#pragma unroll
    for (int i = 0; i < 8; i++) w[i] = v[i];
}

__device__ __forceinline__ void bd_code_words(const Raw<QT_PLANES>& raw, uint32_t w[8]) {
    const uint32_t v[8] = {raw.q0.x, raw.q0.y, raw.q0.z, raw.q0.w, raw.q1.x, raw.q1.y, raw.q1.z, raw.q1.w};
#pragma unroll
    for (int i = 0; i < 8; i++) w[i] = v[i];
}

__device__ __forceinline__ void bd_code_words(const Raw<QT_Q4_0>& raw, uint32_t w[8]) {
    // block 2kg: d at bytes 0-1, codes at 2..17 (realigned by two bytes);
    // block 2kg+1: d at 18-19, codes at 20..35 (words 5..8, aligned)
    w[0] = __builtin_amdgcn_alignbit(raw.a.y, raw.a.x, 16);
    w[1] = __builtin_amdgcn_alignbit(raw.a.z, raw.a.y, 16);
    w[2] = __builtin_amdgcn_alignbit(raw.a.w, raw.a.z, 16);
    w[3] = __builtin_amdgcn_alignbit(raw.b.x, raw.a.w, 16);
    w[4] = raw.b.y;
    w[5] = raw.b.z;
    w[6] = raw.b.w;
    w[7] = raw.c;
}

// fp32 scales d of the lane's two blocks (Q4_0 formats), times 2^20.
__device__ __forceinline__ void bd_block_scales(const Raw<QT_Q4_0>& raw, float& da20, float& db20) {
    da20 = half_bits_to_float(raw.a.x & 0xFFFFu) * 1048576.0f;
    db20 = half_bits_to_float(raw.b.x >> 16) * 1048576.0f;
}

__device__ __forceinline__ void bd_block_scales(const Raw<QT_PLANES>& raw, float& da20, float& db20) {
    da20 = half_bits_to_float(raw.sc & 0xFFFFu) * 1048576.0f;
    db20 = half_bits_to_float(raw.sc >> 16) * 1048576.0f;
}

// Codes of bytes 8t .. 8t+7 of the lane's code words as MFMA operands, in the
// order b0 b2 b1 b3 b4 b6 b5 b7: `lo` the low nibbles as the fp16 bit patterns
// q (value q * 2^-24), `hi` the high nibbles masked in place (16 q * 2^-24).
// One v_alignbit_b32 and four v_and_b32 per word.
__device__ __forceinline__ void codes_subnormal(const uint32_t w[8], int t, h8& lo, h8& hi) {
    const uint32_t x0 = w[2 * t], x1 = w[2 * t + 1];
    const uint32_t r0 = __builtin_amdgcn_alignbit(x0, x0, 8), r1 = __builtin_amdgcn_alignbit(x1, x1, 8);
    lo = __builtin_bit_cast(h8, u4{x0 & 0x000F000Fu, r0 & 0x000F000Fu, x1 & 0x000F000Fu, r1 & 0x000F000Fu});
    hi = __builtin_bit_cast(h8, u4{x0 & 0x00F000F0u, r0 & 0x00F000F0u, x1 & 0x00F000F0u, r1 & 0x00F000F0u});
}

// Integer weights sc * q of MFMA i (the same elements as weights() below).
__device__ __forceinline__ h8 weights_int(const Magic& mg, const Raw<QT_Q4_K>& raw, const SclK& sc, int i) {
    const uint32_t w[8] = {raw.q0.x, raw.q0.y, raw.q0.z, raw.q0.w, raw.q1.x, raw.q1.y, raw.q1.z, raw.q1.w};
    const int t = i & 3;
    if (i < 4) return decode8_int<false>(mg, w[2 * t], w[2 * t + 1], sc.s_lo, sc.c_lo);
    return decode8_int<true>(mg, w[2 * t], w[2 * t + 1], sc.s_hi, sc.c_hi);
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
    if (i < 4) return decode8_mix<false>(w[2 * t], w[2 * t + 1], sc.sa, sc.ca);
    return decode8_mix<true>(w[2 * t], w[2 * t + 1], sc.sb, sc.cb);
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

}  // namespace bf
