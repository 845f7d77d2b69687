// Building blocks of the LDS-staged kernels (bf_gemm_lds.hip, bf_gemm_slab.hip):
// direct-to-LDS loads, completion markers, LDS flag waits, per-format LDS
// readers and the loader address pattern.
#pragma once

#include "bf_formats.h"
#include "bf_lds_plan.h"

namespace bf {
namespace {

constexpr int kASg = 528;                // LDS bytes of one super-group of one activation row (512 + 16)

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint8_t*)p;
}

// Lane l copies the 16 bytes at `src` to LDS byte address m0 + 16*l.
// (One wait state is required between the M0 write and the LDS-DMA.)
__device__ __forceinline__ void dma16(const void* src, uint32_t m0) {
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off" :: "v"(src), "{m0}"(m0) : "memory");
}

// Completion marker: lane 0 copies the nonzero word at `src` to LDS byte address
// m0 (a one-dword direct-to-LDS load; the other lanes are masked off).  A wave's
// loads return in issue order, so once the marker is visible in LDS every load
// this wave issued before it has landed as well.
__device__ __forceinline__ void dma_marker(const void* src, uint32_t m0, int lane) {
    if (lane == 0)
        asm volatile("s_nop 0\n\tglobal_load_lds_dword %0, off" :: "v"(src), "{m0}"(m0) : "memory");
}

__device__ const uint32_t g_marker_src[64] = {
    1u, 1u, 1u, 1u, 1u, 1u, 1u, 1u, 1u, 1u, 1u, 1u, 1u, 1u, 1u, 1u, 1u, 1u, 1u, 1u, 1u, 1u,
    1u, 1u, 1u, 1u, 1u, 1u, 1u, 1u, 1u, 1u, 1u, 1u, 1u, 1u, 1u, 1u, 1u, 1u, 1u, 1u, 1u, 1u,
    1u, 1u, 1u, 1u, 1u, 1u, 1u, 1u, 1u, 1u, 1u, 1u, 1u, 1u, 1u, 1u, 1u, 1u, 1u, 1u};

// Barrier that waits for this wave's LDS traffic only (the LDS-DMA loads of
// later steps stay in flight across it).
__device__ __forceinline__ void barrier_lds() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// One column's image of one super-group, read from LDS.
template <int QT>
__device__ __forceinline__ void lds_raw(Raw<QT>& raw, const uint8_t* u, int kg);

template <>
__device__ __forceinline__ void lds_raw<QT_Q4_K>(Raw<QT_Q4_K>& raw, const uint8_t* u, int kg) {
    raw.hdr = *(const u4*)u;
    raw.q0 = *(const u4*)(u + 16 + 32 * kg);
    raw.q1 = *(const u4*)(u + 32 + 32 * kg);
}

template <>
__device__ __forceinline__ void lds_raw<QT_PLANES>(Raw<QT_PLANES>& raw, const uint8_t* u, int kg) {
    raw.q0 = *(const u4*)(u + 16 + 32 * kg);
    raw.q1 = *(const u4*)(u + 32 + 32 * kg);
    raw.sc = *(const uint32_t*)(u + 4 * kg);
}

template <>
__device__ __forceinline__ void lds_raw<QT_Q4_0>(Raw<QT_Q4_0>& raw, const uint8_t* u, int kg) {
    raw.a = ld16_a4(u + 36 * kg);
    raw.b = ld16_a4(u + 36 * kg + 16);
    raw.c = *(const uint32_t*)(u + 36 * kg + 32);
}

// Global address of 16-byte piece c (0..8) of the super-group image of (row, sg).
template <int QT>
__device__ __forceinline__ const uint8_t* w_piece(const uint8_t* W, const uint8_t* Waux, int64_t row, int sg,
                                                  int c, int K) {
    if constexpr (QT == QT_PLANES) {
        if (c == 0) return Waux + 2 * (row * (int64_t)(K >> 5) + 8 * sg);
        return W + row * (int64_t)(K >> 1) + 128 * sg + 16 * (c - 1);
    } else {
        return W + row * ((int64_t)(K >> 8) * 144) + 144 * sg + 16 * c;
    }
}

// Bounded waits.  A wait ends when its producer signals; the bound only
// guards against a hang if a producer were ever missing (a protocol bug: no
// launch comes close to it).  A wait that reaches the bound marks the
// workgroup poisoned before the wave goes on: it sets the LDS word `poison`
// and waits for that write, so every LDS write the wave makes afterwards (and
// every load it issues afterwards) is ordered behind it.  Each store of a
// result first reads the poison word (poisoned()) and stores NaN instead of a
// value if it is set, so a missing producer shows as a failed result, never as
// a plausible wrong one.
constexpr int kWaitBound = 1 << 20;

__device__ __forceinline__ void mark_poison(int* poison) {
    asm volatile("ds_write_b32 %0, %1\n\ts_waitcnt lgkmcnt(0)" :: "v"(lds_addr(poison)), "v"(1) : "memory");
}

__device__ __forceinline__ bool poisoned(const int* poison) {
    int v;
    asm volatile("ds_read_b32 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(lds_addr(poison)) : "memory");
    return __builtin_amdgcn_readfirstlane(v) != 0;
}

// Spin (with s_sleep) until the LDS word at `flag` is nonzero.
__device__ __forceinline__ void wait_flag(const int* flag, int* poison) {
    const uint32_t a = lds_addr(flag);
    for (int it = 0; it < kWaitBound; it++) {
        int v;
        asm volatile("ds_read_b32 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(a) : "memory");
        if (__builtin_amdgcn_readfirstlane(v) != 0) return;
        __builtin_amdgcn_s_sleep(1);
    }
    mark_poison(poison);
}

// Spin until the LDS word at `flag` equals v.
__device__ __forceinline__ void wait_flag_value(const int* flag, int v, int* poison) {
    const uint32_t a = lds_addr(flag);
    for (int it = 0; it < kWaitBound; it++) {
        int x;
        asm volatile("ds_read_b32 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(x) : "v"(a) : "memory");
        if (__builtin_amdgcn_readfirstlane(x) == v) return;
        __builtin_amdgcn_s_sleep(1);
    }
    mark_poison(poison);
}

// Spin until the LDS word at `flag` is at least n.
__device__ __forceinline__ void wait_count(const int* flag, int n, int* poison) {
    const uint32_t a = lds_addr(flag);
    for (int it = 0; it < kWaitBound; it++) {
        int v;
        asm volatile("ds_read_b32 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(a) : "memory");
        if (__builtin_amdgcn_readfirstlane(v) >= n) return;
        __builtin_amdgcn_s_sleep(1);
    }
    mark_poison(poison);
}

// Spin until the n <= 64 consecutive LDS words from `flags` are all >= v0:
// lane l polls word l, so one LDS read per round covers all of them.
__device__ __forceinline__ void wait_flags(const int* flags, int n, int lane, int* poison, int v0 = 1) {
    const uint32_t a = lds_addr(flags + (lane < n ? lane : 0));
    for (int it = 0; it < kWaitBound; it++) {
        int v;
        asm volatile("ds_read_b32 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(a) : "memory");
        if (__builtin_amdgcn_ballot_w64(v < v0) == 0) return;
        __builtin_amdgcn_s_sleep(1);
    }
    mark_poison(poison);
}

// Spin until the LDS word each lane names is nonzero in every lane with
// `need`: one LDS read per round for up to 64 flags anywhere in LDS.
__device__ __forceinline__ void wait_lanes(const int* flag, bool need, int* poison) {
    const uint32_t a = lds_addr(flag);
    for (int it = 0; it < kWaitBound; it++) {
        int v;
        asm volatile("ds_read_b32 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(a) : "memory");
        if (__builtin_amdgcn_ballot_w64(need && v == 0) == 0) return;
        __builtin_amdgcn_s_sleep(1);
    }
    mark_poison(poison);
}

// A free partial slot word of the counter-free exchanges: a signaling NaN,
// which no arithmetic result is (results that are NaN are quiet NaNs), so a
// written partial never looks free.
constexpr unsigned kSlotFree = 0x7FA5A5A5u;

// The XCC (XCD) this wave runs on.
__device__ __forceinline__ int xcc_id() {
    int x;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(x));
    return x & 0xF;
}

// Buffer access cache policy sc1: device scope.  Such a store is written
// through the XCD's L2 to the point of coherence of all XCDs; such a load
// misses the L1 and the XCD's L2 for lines another XCD may have written.
constexpr int kDeviceScope = 16;

// A dependency between the workgroups of one launch, in device memory (one
// 256-byte line per word): word 0 counts the producers that have stored their
// results; word 64 counts the consumers that are past their wait; the last
// producer raises kDepLines release flags (words kDepLine0 + 64 i), which the
// consumers poll round robin, so that no one line takes every consumer's polls
// (polls of a single line from every CU queue behind each other for several
// microseconds).  The last consumer past its wait clears everything.  Word
// kDepPoison is sticky: a consumer whose wait gave up sets it (a producer that
// arrives after the clear would leave the release flags raised for the next
// launch), and every later consumer that finds it set writes NaN.
constexpr int kDepLines = 32, kDepLine0 = 128;
constexpr int kDepPoison = kDepLine0 + 64 * kDepLines;
constexpr int kDepWords = kDepPoison + 64;

// Spin until the device-scope word *cnt is at least n (lane 0 polls with
// agent-scope atomic loads, which bypass the XCD's L2; a short s_sleep
// between polls).  The bound (2^15 polls of about a microsecond each) stays
// below the LDS waits' so that the poller, not a waiter, is the one to give up.
constexpr int kDeviceWaitBound = 1 << 15;

__device__ __forceinline__ void wait_device_count(const unsigned* cnt, unsigned n, int lane, int* poison) {
    for (int it = 0; it < kDeviceWaitBound; it++) {
        unsigned v = 0;
        if (lane == 0) v = __hip_atomic_load(cnt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if ((unsigned)__builtin_amdgcn_readfirstlane(v) >= n) return;
        __builtin_amdgcn_s_sleep(2);
    }
    mark_poison(poison);
}

// Sets the LDS word at `flag` to 1 once every load this wave has issued has
// completed; for direct-to-LDS loads completion includes the LDS write.
__device__ __forceinline__ void signal_own_loads(int* flag, int lane) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    if (lane == 0) asm volatile("ds_write_b32 %0, %1" :: "v"(lds_addr(flag)), "v"(1) : "memory");
}

// v + (v of lane ^ 16) and v + (v of lane ^ 32), the same value in both lanes.
// v_permlane{16,32}_swap exchanges the odd rows (of 16 or 32 lanes) of its
// first operand with the even rows of its second; with v in both, the two
// results hold the lane's and its partner's value.  Written as inline asm with
// two distinct registers: the builtin form has been compiled to add the first
// result to itself.
__device__ __forceinline__ float sum_lane_xor16(float v) {
    uint32_t a = __builtin_bit_cast(uint32_t, v), b = a;
    asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(a), "+v"(b));
    return __builtin_bit_cast(float, a) + __builtin_bit_cast(float, b);
}

__device__ __forceinline__ float sum_lane_xor32(float v) {
    uint32_t a = __builtin_bit_cast(uint32_t, v), b = a;
    asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
    return __builtin_bit_cast(float, a) + __builtin_bit_cast(float, b);
}

__device__ __forceinline__ float dpp_xor(float v, int ctrl_sel) {
    // quad_perm [1,0,3,2] (xor 1) or [2,3,0,1] (xor 2)
    const int x = __builtin_bit_cast(int, v);
    return __builtin_bit_cast(float, ctrl_sel == 1 ? __builtin_amdgcn_mov_dpp(x, 0xB1, 0xF, 0xF, false)
                                                   : __builtin_amdgcn_mov_dpp(x, 0x4E, 0xF, 0xF, false));
}

// Loader address pattern: the offset of piece c of column (rowl, g) inside one
// step image, relative to the step's base (bit 28 set: the piece comes from
// the planes layout's scale array), and the scalar bases of a step.
template <int QT>
__device__ __forceinline__ uint32_t step_piece_offset(int rowl, int g, int c, int K) {
    // rowl < 16, and K < 81920 (the activations fit in LDS), so the row strides
    // stay far below 2^24 bytes: 24-bit multiplies
    if constexpr (QT == QT_PLANES) {
        if (c == 0) return (__umul24((uint32_t)rowl, (uint32_t)(K >> 4)) + 16u * g) | (1u << 28);
        return __umul24((uint32_t)rowl, (uint32_t)(K >> 1)) + 128u * g + 16u * (c - 1);
    } else {
        return __umul24((uint32_t)rowl, (uint32_t)((K >> 8) * 144)) + 144u * g + 16u * c;
    }
}

template <int QT> struct StepBase { int64_t w; };
template <> struct StepBase<QT_PLANES> { int64_t w, aux; };

template <int QT>
__device__ __forceinline__ StepBase<QT> step_base(int64_t row0, int sg0, int K) {
    if constexpr (QT == QT_PLANES) {
        return StepBase<QT>{row0 * (K >> 1) + 128 * sg0, row0 * (K >> 4) + 16 * sg0};
    } else {
        return StepBase<QT>{row0 * ((K >> 8) * 144) + 144 * sg0};
    }
}

template <int QT>
__device__ __forceinline__ const uint8_t* piece_addr(const uint8_t* W, const uint8_t* Waux, const StepBase<QT>& b,
                                                     uint32_t off) {
    if constexpr (QT == QT_PLANES) {
        const uint32_t o = off & 0x0FFFFFFFu;
        return (off >> 28) & 1u ? Waux + b.aux + o : W + b.w + o;
    } else {
        return W + b.w + off;
    }
}

}  // namespace
}  // namespace bf
