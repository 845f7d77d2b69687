// K-split LDS-resident MFMA GEMM for batches of up to 32 rows (k_gemm_split).
//
//   C[m][n] = sum_k A[m][k] * dequant(W)[n][k]      (fp32 accumulation)
//
// At batch 9-32 the activations, not the weights, decide the time: a
// workgroup that covers all of K needs all of A (328 KB at M = 32, K = 5120),
// far more than its share of the weights, and 256 such copies cross the L2.
// Splitting K in S parts divides both the activations each workgroup reads and
// the total activation traffic by S:
//
// * Workgroup (row group rg, split s) owns nt 16-row tiles and the super-groups
//   [s * nsgS, (s + 1) * nsgS).  At N = K = 5120, M = 32: S = 4, nt = 5, 256
//   workgroups, each with 57.6 KB of weights and 82 KB of activations, all of it
//   resident in LDS at once (no ring, no slot reuse).
// * The data of one local super-group i (the activation slab A[0:M][256 i ..
//   256 i + 256) followed by the nt tiles' 144-byte weight images) is one
//   contiguous LDS "unit" of 16-byte pieces.  Four loader waves split each
//   unit's 1 KB direct-to-LDS instructions round robin (per-lane addresses are
//   computed once; a unit only adds a per-piece stride) and each ends its share
//   of a unit with a one-dword marker load; a unit has landed when its four
//   markers are visible (a wave's loads return in order).
// * Compute wave c owns tile c % nt and the super-groups u, u + U, ... of it
//   (u = c / nt, U = number of waves on that tile), accumulating all batch rows
//   (MT m-tiles of 16) in registers.  The other waves of a tile park their sums
//   in LDS and the tile's first wave adds them in wave order.
// * XCD-local exchange: the dispatcher hands the workgroups of a launch to
//   the nx XCDs round robin, starting from an XCD that depends on the
//   hardware queue of the stream (measured: 0 on the null stream, 6 and 7 on
//   two created streams), so each round of nx consecutive workgroups covers
//   every XCD once.  A workgroup takes its row group from the XCD it finds
//   itself on (XCC id x) and its round (b / nx): XCD x holds row groups x,
//   x + nx, ..., each as S consecutive rounds, so all S splits of a row group
//   share one L2 whatever the starting XCD.
// * Exchange through free slots (S > 1): the tile sums go to workspace slots
//   that hold kSlotFree (a signaling NaN, never an arithmetic result) between
//   launches, as plain (L2 write-back) stores; the row group's last split
//   reads every split's slots of each of its elements from its XCD's L2 until
//   no word is free, adds them in split order, writes C and frees the slots.
//   No counter and no store acknowledgement.  The order never depends on
//   timing, so results are deterministic (k_split_sum, the second-launch sum,
//   adds in the same order).  The row group's reader swaps its tag from free
//   to taken at its start and frees it at its end, so a placement that is not
//   round robin (a moved workgroup keeps its split: a row group then misses a
//   split, or has a second reader) shows as NaN in C and a poison word in the
//   workspace that makes every later launch on it NaN (split_body); a
//   poisoned split (a bounded LDS wait gave up) writes NaN sums, and so NaN C.
#include <algorithm>
#include <atomic>
#include <map>
#include <mutex>
#include <thread>
#include <tuple>
#include <utility>
#include <vector>

#include "bf_launch.h"
#include "bf_lds.h"

namespace bf {
namespace {
__global__ void k_zero_u32(unsigned* p, int n) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) p[i] = 0u;
}

// A new workspace: counters at zero, free partial slots (kSlotFree) after them.
__global__ void k_init_workspace(unsigned* p, int nzero, int nfree) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < nzero + nfree; i += gridDim.x * blockDim.x)
        p[i] = i < nzero ? 0u : kSlotFree;
}
}  // namespace

// Bytes before a launch's partial slots: the poison word and padding.
constexpr size_t kSlotHeader = 256;

// XCDs of the current device: the workgroup round robin the XCD-local exchange
// lays its grid out for (1 on a device with one XCD per agent).
int device_xcds() {
    static std::atomic<int> cache[64];                 // 0: not queried yet
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
    int n = cache[dev].load(std::memory_order_relaxed);
    if (n == 0) {
        int v = 0;
        if (hipDeviceGetAttribute(&v, hipDeviceAttributeNumberOfXccs, dev) != hipSuccess || v < 1 || v > 16) v = -1;
        cache[dev].store(v, std::memory_order_relaxed);
        n = v;
    }
    return n > 0 ? n : 0;                                // unknown: device-scope exchange
}

// CUs of the current device (the dense kernel runs one workgroup on each), 0 if unknown.
int device_cus() {
    static std::atomic<int> cache[64];                 // 0: not queried yet
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
    int n = cache[dev].load(std::memory_order_relaxed);
    if (n == 0) {
        int v = 0;
        if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v < 1) v = -1;
        cache[dev].store(v, std::memory_order_relaxed);
        n = v;
    }
    return n > 0 ? n : 0;
}

// The library's own workspaces, one per (device, stream): launches on one
// stream are ordered, so they can share it.  hipStreamPerThread names a
// different stream in every host thread, so it is keyed by the thread too.
// Three regions: counters (kept zero between launches by the kernels that use
// them), partial slots (kept free, every word kSlotFree, between launches by
// the K-split exchange that uses them) and partials (no state between
// launches).  Grown on demand, each region that is too small to at least
// twice its old size, so a stream holds at most about twice its largest
// need.  A buffer that has been replaced is retired, never freed: launches
// already queued may use it, so may a graph captured from the stream, and so
// may a call that another host thread is enqueueing on the same stream with
// the pointer it was handed before the growth (every launch leaves its
// buffer in the state the next one expects, so a retired buffer stays
// usable).  Retired buffers are released when the process ends.  Never
// allocated while the stream is being captured into a graph (an allocation
// cannot be captured): such a call fails with
// hipErrorStreamCaptureUnsupported unless a large enough workspace exists.
hipError_t library_workspace(hipStream_t st, size_t cbytes, size_t sbytes, size_t pbytes, unsigned** counters,
                             float** slots, float** parts) {
    struct Slot {
        uint8_t* p = nullptr;
        size_t cb = 0, sb = 0, pb = 0;
    };
    static std::mutex mu;
    static std::map<std::tuple<int, uintptr_t, std::thread::id>, Slot> cache;
    static std::vector<uint8_t*> retired;
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    const std::thread::id tid = st == hipStreamPerThread ? std::this_thread::get_id() : std::thread::id();
    std::lock_guard<std::mutex> lock(mu);
    Slot& slot = cache[{dev, (uintptr_t)st, tid}];
    if (!slot.p || slot.cb < cbytes || slot.sb < sbytes || slot.pb < pbytes) {
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        e = hipStreamIsCapturing(st, &cs);
        if (e != hipSuccess) return e;
        if (cs != hipStreamCaptureStatusNone) return hipErrorStreamCaptureUnsupported;
        auto grow = [](size_t have, size_t need) {
            return need <= have ? have : std::max(need, 2 * have);
        };
        const size_t cb = grow(slot.cb, cbytes), sb = grow(slot.sb, sbytes), pb = grow(slot.pb, pbytes);
        uint8_t* p = nullptr;
        e = hipMalloc((void**)&p, cb + sb + pb);
        if (e != hipSuccess) return e;
        hipLaunchKernelGGL(k_init_workspace, dim3(256), dim3(256), 0, st, (unsigned*)p, (int)(cb / 4), (int)(sb / 4));
        e = hipGetLastError();
        if (e != hipSuccess) {
            (void)hipFree(p);
            return e;
        }
        if (slot.p) retired.push_back(slot.p);
        slot = Slot{p, cb, sb, pb};
    }
    *counters = (unsigned*)slot.p;
    *slots = (float*)(slot.p + slot.cb);
    *parts = (float*)(slot.p + slot.cb + slot.sb);
    return hipSuccess;
}

hipError_t reserve_workspace(hipStream_t st, const WsNeed& need) {
    if (!need.c && !need.s && !need.p) return hipSuccess;
    unsigned* counters = nullptr;
    float *slots = nullptr, *parts = nullptr;
    return library_workspace(st, need.c, need.s, need.p, &counters, &slots, &parts);
}

// Partial slots of one launch of the shared exchange, behind a 256-byte
// header whose first word is the workspace's poison word (kSlotFree while
// clean).  In the library's workspace for the stream the region is free
// between launches (every launch frees each slot it fills); a caller's
// scratch may hold anything, so there it is filled with kSlotFree by a small
// kernel on the stream before each launch (a kernel, not a memset node, so
// that a captured call replays correctly).
hipError_t slot_workspace(const Scratch* scratch, hipStream_t st, size_t sbytes, float** slots) {
    if (!scratch) {
        unsigned* counters = nullptr;
        float *region = nullptr, *parts = nullptr;
        const hipError_t e = library_workspace(st, 0, kSlotHeader + sbytes, 0, &counters, &region, &parts);
        if (e != hipSuccess) return e;
        *slots = (float*)((uint8_t*)region + kSlotHeader);
        return hipSuccess;
    }
    if (kSlotHeader + sbytes > scratch->bytes) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_init_workspace, dim3(256), dim3(256), 0, st, (unsigned*)scratch->base, 0,
                       (int)((kSlotHeader + sbytes) / 4));
    *slots = (float*)(scratch->base + kSlotHeader);
    return hipGetLastError();
}

hipError_t split_workspace(const Scratch* scratch, hipStream_t st, size_t cbytes, size_t pbytes,
                            unsigned** counters, float** parts) {
    float* slots = nullptr;
    if (!scratch) return library_workspace(st, cbytes, 0, pbytes, counters, &slots, parts);
    if (cbytes + pbytes > scratch->bytes) return hipErrorInvalidValue;
    *counters = (unsigned*)scratch->base;
    *parts = (float*)(scratch->base + cbytes);
    // the counters must start at zero: cleared by a kernel on the stream
    // (not a memset node, so a captured call replays correctly)
    if (cbytes == 0) return hipSuccess;
    hipLaunchKernelGGL(k_zero_u32, dim3(16), dim3(256), 0, st, *counters, (int)(cbytes / 4));
    return hipGetLastError();
}

// Partials that a second launch sums (no state between launches).
hipError_t partial_workspace(const Scratch* scratch, hipStream_t st, size_t pbytes, float** parts) {
    unsigned* counters = nullptr;
    return split_workspace(scratch, st, 0, pbytes, &counters, parts);
}

namespace {

// LDS: [0, 2048) flags: tag-check word at 4, tag-check count at 8, poison
// word at 12 (a bounded wait gave up), unit
// markers of loader j for unit i at 64 + 16 i + 4 j, park flag of compute wave
// c at 1024 + 4 c; then the units; then the parked sums.
constexpr int kSpTagCheck = 1;                          // the reader's own tag swap: 1 free, 2 taken
constexpr int kSpTagCount = 2;                          // the reader's compute waves done with the tags
constexpr int kSpPoison = 3;
constexpr int kSpMaxS = 56;                             // splits of a row group
constexpr int kSpRq = 4;                                // quads a reader wave keeps summed before the tag check
constexpr int kSpFlags = 2048;
constexpr int kSpMaxUnits = (1024 - 64) / 16;
constexpr int kSpNC = 12, kSpNL = 4;    // compute and loader waves per workgroup
constexpr int kSpQS = 12;               // instruction slots per loader and unit
constexpr int kSpMaxPieces = 64 * kSpNL * kSpQS;
constexpr int kCoherent = 16;           // buffer access cache policy: sc1 (device scope: misses the L1)

// Byte offset of the exchange's tags (one dword per row group: its reader's)
// after the partial slots [S][N][Mp] fp32, at a 256-byte boundary.
__host__ __device__ __forceinline__ int tag_offset(int S, int N, int Mp) {
    return (int)(((int64_t)S * N * Mp * 4 + 255) & ~(int64_t)255);
}

// Buffer resource over the split partials [S][N][Mp] (fp32).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t workspace_rsrc(float* ws, int S, int N, int Mp) {
    return __builtin_amdgcn_make_buffer_rsrc(ws, (short)0, (int)((int64_t)S * N * Mp * 4), 0x00020000);
}

// One GEMM's share of a launch: workgroup `bid` of its grid.  SUM2: the
// splits' partials are left for k_split_sum (a second launch); otherwise
// (slots) the row group's splits exchange them through the workspace's free
// slots, each split summing a share of the row group (poison: the
// workspace's poison word).
template <int QT, int MT, bool SUM2>
__device__ __forceinline__ void split_body(int bid, uint8_t* lds, const uint8_t* __restrict__ W,
                                           const uint16_t* __restrict__ A, int lda, int M, int N, int K, int nt,
                                           int S, int nsgS, int unit_bytes, const uint8_t* __restrict__ Waux,
                                           void* __restrict__ C, int ldc, int out_f16, float* __restrict__ ws,
                                           unsigned* __restrict__ poison, int nx, int slots) {
    constexpr int NC = kSpNC, NL = kSpNL;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    int rg, s;
    if (nx > 0) {
        // XCD x holds row groups x, x + nx, ..., each as S consecutive rounds;
        // with the exchange x is the XCD this workgroup runs on (the same
        // bijection for any starting XCD of the round robin)
        const int x = !SUM2 && S > 1 && nx > 1 ? xcc_id() % nx : bid % nx;
        const int jx = bid / nx, q = jx / S;
        rg = x + nx * q;
        s = jx - q * S;
        if ((int64_t)rg * nt * 16 >= N) return;          // padding of the last XCD round
    } else {
        rg = bid / S;
        s = bid - rg * S;
    }
    const int sg0 = s * nsgS;
    int* const flags = (int*)lds;
    const uint32_t lds0 = lds_addr(lds);
    const int PA = M * 33, PW = nt * 144;                // activation and weight pieces of a unit
    const int I = (PA + PW + 63) >> 6;                   // 1 KB instructions per unit
    const int Mp = (M + 3) & ~3;                         // workspace rows, whole quads

    auto clear_flags_and_meet = [&]() {
        static_assert((NC + NL) * 128 == kSpFlags, "each wave clears 32 flags");
        if (lane < 32) flags[32 * wave + lane] = 0;
        barrier_lds();
    };

    if (wave < NL) {
        // ------------------------------------------------------------ loader wave
        __builtin_amdgcn_s_setprio(3);
        const int j = wave;
        // instruction q = j + 4 * slot covers pieces 64 q + lane of every unit;
        // the piece's address in unit i is src + i * step (step 0: lane idle).
        // Unit 0's load of each slot goes out as soon as its address is known
        // (all slots' addresses take a few hundred cycles of instruction issue).
        const uint8_t* src[kSpQS];
        uint32_t step[kSpQS];
#pragma unroll
        for (int q2 = 0; q2 < kSpQS; q2++) {
            const uint32_t P = 64u * (j + 4 * q2) + lane;
            src[q2] = W;
            step[q2] = 0;
            if (P < (uint32_t)PA) {
                // activation piece: row m, 16-byte part c (part 32 is the row's bank padding)
                const uint32_t m = __umul24(P, 1986u) >> 16, c = P - 33u * m;     // P < 3072
                if (c < 32) {
                    src[q2] = (const uint8_t*)(A + (int64_t)m * lda + 256 * sg0 + 8 * c);
                    step[q2] = 512;
                }
            } else if (P < (uint32_t)(PA + PW)) {
                // weight piece: tile t, row n of the tile, part c of its 144-byte image
                const uint32_t pw = P - PA, t = __umul24(pw, 7282u) >> 20, rem = pw - 144u * t;
                const uint32_t n = __umul24(rem, 7282u) >> 16, c = rem - 9u * n;
                const int64_t row = min((int64_t)(rg * nt + (int)t) * 16 + (int)n, (int64_t)N - 1);
                src[q2] = w_piece<QT>(W, Waux, row, sg0, (int)c, K);
                step[q2] = QT == QT_PLANES ? (c == 0 ? 16u : 128u) : 144u;
            }
            const int q = j + 4 * q2;
            if (q < I && step[q2]) dma16(src[q2], lds0 + (uint32_t)(kSpFlags + (q << 10)));
        }
        for (int i = 0; i < nsgS; i++) {
            const uint32_t ub = lds0 + (uint32_t)(kSpFlags + i * unit_bytes);
#pragma unroll
            for (int q2 = 0; q2 < kSpQS; q2++) {
                const int q = j + 4 * q2;
                if (i == 0 || q >= I) break;
                if (step[q2]) dma16(src[q2] + (uint32_t)i * step[q2], ub + (uint32_t)(q << 10));
            }
            if (i == 0) clear_flags_and_meet();
            dma_marker(g_marker_src + lane, lds0 + (uint32_t)(64 + 16 * i + 4 * j), lane);
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        return;
    }

    // ---------------------------------------------------------------- compute wave
    clear_flags_and_meet();
    const int c = wave - NL;
    const bool exchange = !SUM2 && S > 1 && slots;
    // the row group's last split (wave 0) swaps its tag from free to taken
    // now and loads the workspace's poison word (an earlier launch's exchange
    // that gave up leaves it set); both answers are looked at after the
    // compute
    uint32_t* const tags = exchange ? (uint32_t*)((uint8_t*)ws + tag_offset(S, N, Mp)) : nullptr;
    uint32_t tag_old = kSlotFree, pword = kSlotFree;
    if (exchange && s == S - 1 && c == 0 && lane == 0) {
        tag_old = __hip_atomic_exchange(tags + rg, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        pword = __hip_atomic_load(poison, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    const int t = c % nt, u = c / nt;
    const int U = (NC - 1 - t) / nt + 1;                 // waves on tile t
    const Magic mg = make_magic();
    const int r = lane & 15, kg = lane >> 4;
    int arow[MT];
#pragma unroll
    for (int mt = 0; mt < MT; mt++) arow[mt] = min(mt * 16 + r, M - 1) * 528 + 128 * kg;   // pad rows reread M-1
    f4 acc[MT];
#pragma unroll
    for (int mt = 0; mt < MT; mt++) acc[mt] = f4{0.f, 0.f, 0.f, 0.f};

    for (int i = u; i < nsgS; i += U) {
        wait_flags(flags + 16 + 4 * i, NL, lane, flags + kSpPoison);
        const uint8_t* unit = lds + kSpFlags + i * unit_bytes;
        Raw<QT> raw;
        lds_raw<QT>(raw, unit + PA * 16 + t * 2304 + r * 144, kg);
        const auto sc = scales(raw, kg);
#pragma unroll
        for (int ii = 0; ii < 8; ii++) {
            const h8 b = weights(mg, raw, sc, ii);
#pragma unroll
            for (int mt = 0; mt < MT; mt++) acc[mt] = mfma16x16x32(*(const h8*)(unit + arow[mt] + 16 * ii), b, acc[mt]);
        }
    }

    // the tile's first wave adds the others' sums (in wave order) and writes the tile
    float* const park = (float*)(lds + kSpFlags + nsgS * unit_bytes);
    if (u > 0) {
        float* mine = park + (c - nt) * MT * 256;
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
#pragma unroll
            for (int i = 0; i < 4; i++) mine[(mt * 4 + i) * 64 + lane] = acc[mt][i];
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        if (lane == 0) asm volatile("ds_write_b32 %0, %1" :: "v"(lds_addr(&flags[256 + c])), "v"(1) : "memory");
    } else {
        for (int u2 = 1; u2 < U; u2++) {
            const int c2 = t + nt * u2;
            wait_flag(&flags[256 + c2], flags + kSpPoison);
            const float* theirs = park + (c2 - nt) * MT * 256;
#pragma unroll
            for (int mt = 0; mt < MT; mt++)
#pragma unroll
                for (int i = 0; i < 4; i++) acc[mt][i] += theirs[(mt * 4 + i) * 64 + lane];
        }
        const int64_t n = (int64_t)(rg * nt + t) * 16 + r;
        if (poisoned(flags + kSpPoison)) {
#pragma unroll
            for (int mt = 0; mt < MT; mt++) acc[mt] = f4{1.f, 1.f, 1.f, 1.f} * __builtin_nanf("");
        }
        if (S > 1) {
            // workspace [s][n][Mp]: this lane's four rows of an m-tile are one 16-byte store
            const __amdgpu_buffer_rsrc_t wr = workspace_rsrc(ws, S, N, Mp);
#pragma unroll
            for (int mt = 0; mt < MT; mt++) {
                const int m4 = mt * 16 + 4 * kg;
                if (m4 < Mp && n < N) {
                    const int off = (int)((((int64_t)s * N + n) * Mp + m4) * 4);
                    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u4, acc[mt]), wr, off, 0, 0);
                }
            }
        } else {
#pragma unroll
            for (int mt = 0; mt < MT; mt++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int m = mt * 16 + 4 * kg + i;
                    if (m < M && n < N) {
                        if (out_f16) ((_Float16*)C)[(int64_t)m * ldc + n] = (_Float16)acc[mt][i];
                        else ((float*)C)[(int64_t)m * ldc + n] = acc[mt][i];
                    }
                }
        }
    }
    if (!exchange) return;

    // -------------------------------------------------------- the exchange
    // The row group's last split (s = S - 1, dispatched after the others,
    // so it waits only for workgroups that started before it) reads every
    // split's slots of each of its elements from its XCD's L2 until no word
    // is free (bounded), adds them in split order (k_split_sum's order: the
    // same bits), writes C and frees the slots for the next launch.  Each
    // reader swapped its row group's tag from free to taken at its start: it
    // writes C only if the swap found the tag free (a second reader of the row
    // group does not, while the first still runs) and the workspace is not
    // poisoned.  A missing split leaves its slots free, so the reader gives
    // up; so does a second reader that starts after the first has freed the
    // slots.  A reader that gives up writes NaN over all of C (a row group
    // whose reader went missing to a duplicate's role has no other writer)
    // and sets the workspace's poison word, after which every launch on the
    // workspace writes NaN (a duplicated split may refill slots after the
    // reader freed them).  Exchange plans fill whole XCD rounds (no padding
    // workgroups), and a workgroup moved off its XCD keeps its split, so it
    // lands on the role of another row group's same split: a missing split,
    // or a missing reader beside a second one.
    {
        const int rows = nt * 16, nq = rows * (Mp / 4);
        const int64_t n0 = (int64_t)rg * rows;
        bool late = false;                               // give up: NaN over C
        if (s == S - 1) {
            const __amdgpu_buffer_rsrc_t wr = workspace_rsrc(ws, S, N, Mp);
            const int sstride = N * Mp * 4;              // bytes between two splits' slots
            const u4 freev = u4{kSlotFree, kSlotFree, kSlotFree, kSlotFree};
            // wave 0 publishes its own swap's answer and the poison word (1: the
            // tag was free and the workspace clean, 2: not) to the other waves
            if (c == 0 && lane == 0)
                asm volatile("ds_write_b32 %0, %1" :: "v"(lds_addr(&flags[kSpTagCheck])),
                             "v"(tag_old == kSlotFree && pword == kSlotFree ? 1 : 2) : "memory");
            // the quads this wave sums: up to kSpRq in registers, the rest written as summed
            f4 kept[kSpRq];
            int koff[kSpRq];
            auto poll_sum = [&, S](int off, bool ok, f4& sum) __attribute__((always_inline)) {
                sum = f4{0.f, 0.f, 0.f, 0.f};
                if (late) return;
                for (int s0 = 0; s0 < S; s0 += 4) {
                    u4 x[4];
                    for (int it = 0;; it++) {
                        bool miss = false;
#pragma unroll
                        for (int k = 0; k < 4; k++)
                            x[k] = ok && s0 + k < S ? __builtin_amdgcn_raw_buffer_load_b128(wr, off + (s0 + k) * sstride,
                                                                                              0, kCoherent)
                                                    : u4{0u, 0u, 0u, 0u};
#pragma unroll
                        for (int k = 0; k < 4; k++) {
                            const u4 w = x[k];
                            miss = miss || w[0] == kSlotFree || w[1] == kSlotFree || w[2] == kSlotFree ||
                                   w[3] == kSlotFree;
                        }
                        if (__builtin_amdgcn_ballot_w64(miss) == 0) break;
                        if (it == kDeviceWaitBound) {
                            late = true;
                            break;
                        }
                        __builtin_amdgcn_s_sleep(2);
                    }
                    if (late) break;
#pragma unroll
                    for (int k = 0; k < 4; k++)
                        if (s0 + k < S) sum += __builtin_bit_cast(f4, x[k]);   // splits in order
                }
            };
            bool checked = false;
            auto check_tag = [&]() __attribute__((always_inline)) {
                if (checked) return;
                checked = true;
                wait_flag(&flags[kSpTagCheck], flags + kSpPoison);
                if (flags[kSpTagCheck] != 1) late = true;
            };
            auto write_c = [&, S, M](int off, const f4& sum) __attribute__((always_inline)) {
                const int q = off / 16, n = q / (Mp / 4), m4 = 4 * (q - n * (Mp / 4));
                for (int k = 0; k < S; k++) __builtin_amdgcn_raw_buffer_store_b128(freev, wr, off + k * sstride, 0, 0);
                const bool bad = late || poisoned(flags + kSpPoison);
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    if (m4 + i >= M) break;
                    const float y = bad ? __builtin_nanf("") : sum[i];
                    if (out_f16) ((_Float16*)C)[(int64_t)(m4 + i) * ldc + n] = (_Float16)y;
                    else ((float*)C)[(int64_t)(m4 + i) * ldc + n] = y;
                }
            };
            // the first kSpRq quads of this wave, summed in registers (unrolled:
            // fixed register slots), then every quad beyond them summed and
            // written one by one after the check
            auto quad_off = [&, nq, N](int b, bool& ok) __attribute__((always_inline)) {
                const int v = b + lane;
                const int nl = v / (Mp / 4), m4 = 4 * (v - nl * (Mp / 4));
                ok = v < nq && n0 + nl < N;
                return ok ? (int)(((n0 + nl) * Mp + m4) * 4) : 0;
            };
#pragma unroll
            for (int r = 0; r < kSpRq; r++) {
                const int b = c * 64 + r * NC * 64;
                koff[r] = -1;
                if (b < nq) {
                    bool ok;
                    const int off = quad_off(b, ok);
                    poll_sum(off, ok, kept[r]);
                    if (ok) koff[r] = off;
                }
            }
            for (int b = c * 64 + kSpRq * NC * 64; b < nq; b += NC * 64) {
                bool ok;
                const int off = quad_off(b, ok);
                f4 sum;
                poll_sum(off, ok, sum);
                check_tag();
                if (ok) write_c(off, sum);
            }
            check_tag();
#pragma unroll
            for (int r = 0; r < kSpRq; r++)
                if (koff[r] >= 0) write_c(koff[r], kept[r]);
            // the last wave done frees the row group's tag
            uint32_t seen = 0;
            if (lane == 0)
                asm volatile("ds_add_rtn_u32 %0, %1, %2\n\ts_waitcnt lgkmcnt(0)"
                             : "=v"(seen) : "v"(lds_addr(&flags[kSpTagCount])), "v"(1u) : "memory");
            if ((uint32_t)__builtin_amdgcn_readfirstlane(seen) == (uint32_t)(NC - 1) && lane == 0)
                __hip_atomic_store(tags + rg, kSlotFree, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        if (late) {
            // NaN over all of C: a row group whose reader went missing has no other writer
            for (int64_t e = lane; e < (int64_t)M * N; e += 64) {
                const int64_t m = e / N, n = e - m * N;
                if (out_f16) ((_Float16*)C)[m * ldc + n] = (_Float16)__builtin_nanf("");
                else ((float*)C)[m * ldc + n] = __builtin_nanf("");
            }
            if (lane == 0) __hip_atomic_store(poison, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

// The single-launch kernel's arguments fit in the 14 dwords preloaded into
// SGPRs at wave launch (no scalar load of an argument, which the first wait
// for the flags' LDS writes would also wait for, queued behind the weight
// stream): X = N | (M - 1) << 24 | out_f16 << 29 | slots << 30, Y = K / 256 |
// nt << 12 | S << 16 | nx << 22 (split_packed_args); the workspace's poison
// word sits kSlotHeader bytes before the slots.
template <int QT, int MT, bool SUM2>
__global__ __launch_bounds__(64 * (kSpNC + kSpNL)) __attribute__((amdgpu_waves_per_eu(1, 4)))
void k_gemm_split(const uint8_t* __restrict__ W, const uint16_t* __restrict__ A, const uint8_t* __restrict__ Waux,
                  void* __restrict__ C, float* __restrict__ ws, int lda, int ldc, uint32_t X, uint32_t Y) {
    extern __shared__ __attribute__((aligned(1024))) uint8_t lds[];
    const int N = (int)(X & 0xFFFFFFu), M = (int)((X >> 24) & 31u) + 1, out_f16 = (int)((X >> 29) & 1u);
    const int slots = (int)((X >> 30) & 1u);
    const int nsg = (int)(Y & 0xFFFu), nt = (int)((Y >> 12) & 15u), S = (int)((Y >> 16) & 63u), nx = (int)((Y >> 22) & 31u);
    unsigned* const poison = slots ? (unsigned*)((uint8_t*)ws - kSlotHeader) : nullptr;
    split_body<QT, MT, SUM2>((int)blockIdx.x, lds, W, A, lda, M, N, nsg << 8, nt, S, nsg / S, (M * 33 + nt * 144) * 16,
                             Waux, C, ldc, out_f16, ws, poison, nx, slots);
}

// C of a single K-split launch: the S partials [s][n][Mp] of each element
// added in split order (the order the batched launch's last split uses, so
// both give the same bits).  Block b: rows 32 b .. 32 b + 31 and all batch
// rows (M <= 32: at most 256 quads, one per thread); coalesced partial loads,
// an LDS transpose, C stored along its rows.
__global__ __launch_bounds__(256) void k_split_sum(const float* __restrict__ ws, void* __restrict__ C, int ldc,
                                                   int out_f16, int M, int N, int S) {
    __shared__ float tr[32 * 33];
    const int Mp = (M + 3) & ~3, nq = 32 * (Mp / 4);
    const int n0 = 32 * (int)blockIdx.x, tid = (int)threadIdx.x;
    if (tid < nq) {
        const int nl = tid / (Mp / 4), m4 = 4 * (tid - nl * (Mp / 4));
        f4 s = f4{0.f, 0.f, 0.f, 0.f};
        if (n0 + nl < N)
            // up to eight splits' loads in flight before the first add (splits in order)
            for (int k0 = 0; k0 < S; k0 += 8) {
                f4 x[8];
#pragma unroll
                for (int k = 0; k < 8; k++)
                    x[k] = k0 + k < S ? *(const f4*)(ws + ((size_t)(k0 + k) * N + n0 + nl) * Mp + m4)
                                      : f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int k = 0; k < 8; k++)
                    if (k0 + k < S) s += x[k];
            }
#pragma unroll
        for (int i = 0; i < 4; i++) tr[(m4 + i) * 33 + nl] = s[i];
    }
    __syncthreads();
    for (int y = tid; y < M * 32; y += 256) {
        const int m = y >> 5, nl = y & 31;
        if (n0 + nl >= N) continue;
        const float x = tr[m * 33 + nl];
        if (out_f16) ((_Float16*)C)[(int64_t)m * ldc + n0 + nl] = (_Float16)x;
        else ((float*)C)[(int64_t)m * ldc + n0 + nl] = x;
    }
}

// Several independent GEMMs in one launch (their grids back to back): a
// workgroup finds its GEMM by its id.  Workgroups of a later GEMM start as
// those of an earlier one retire, so one GEMM's cross-split exchange overlaps
// the next one's weight stream, and the launch gaps between them disappear.
constexpr int kSpMaxJobs = 8;
struct SplitJob {
    const uint8_t* W;
    const uint8_t* Waux;
    const uint16_t* A;
    void* C;
    float* ws;
    int lda, ldc, M, N, K, nt, S, nsgS, unit_bytes, grid0;
};
struct SplitJobs {
    SplitJob job[kSpMaxJobs];
    unsigned* poison;                    // the workspace's poison word (the slots' header)
    int n, out_f16, nx;                  // nx: XCD-local exchange (every job's grid0 a multiple of nx)
    int slots;                           // the shared exchange through free slots
};

template <int QT, int MT>
__global__ __launch_bounds__(64 * (kSpNC + kSpNL)) __attribute__((amdgpu_waves_per_eu(1, 4)))
void k_gemm_split_batched(const SplitJobs jobs) {
    extern __shared__ __attribute__((aligned(1024))) uint8_t lds[];
    // the last job whose grid starts at or before this workgroup (uniform
    // selects over the kernel arguments: no dynamic indexing)
    SplitJob j = jobs.job[0];
#pragma unroll
    for (int i = 1; i < kSpMaxJobs; i++)
        if (i < jobs.n && (int)blockIdx.x >= jobs.job[i].grid0) j = jobs.job[i];
    // (read into SGPRs one by one: kept as a struct, a field was once
    // spilled to scratch and reloaded through a selected address)
    const auto u = [](int v) { return __builtin_amdgcn_readfirstlane(v); };
    split_body<QT, MT, false>((int)blockIdx.x - u(j.grid0), lds, j.W, j.A, u(j.lda), u(j.M), u(j.N), u(j.K), u(j.nt),
                              u(j.S), u(j.nsgS), u(j.unit_bytes), j.Waux, j.C, u(j.ldc), jobs.out_f16, j.ws,
                              jobs.poison, jobs.nx, jobs.slots);
}


struct SplitPlan {
    int S, nt, nsgS, MT, grid, unit_bytes, lds, nx, rgs;
};

int split_lds_bytes(int M, int nt, int nsgS, int MT) {
    const int unit = (M * 33 + nt * 144) * 16;
    const int parks = (kSpNC > nt ? kSpNC - nt : 0) * MT * 1024;
    return kSpFlags + nsgS * unit + parks;
}

// S divides the super-groups; nt tiles per workgroup (<= the compute waves);
// the estimate is rounds of 256 workgroups times the bytes each one loads,
// plus the partials' round trip when S > 1.  With nx XCDs the grid holds
// ceil(rgs / nx) * nx row groups (whole rounds of the XCD round robin).
bool plan_split(const GemmArgs& g, SplitPlan& p, int nx) {
    if (g.M > 32 || g.K % 256) return false;
    if (g.N >= (1 << 24) || g.K / 256 > 0xFFF) return false;            // the packed kernel arguments
    if (nx > 31) nx = 0;
    if ((int64_t)g.K / 256 * g.N * 32 * 4 >= (1LL << 31)) return false;   // partials addressed by 32-bit offsets
    const int nsg = g.K / 256, T = (g.N + 15) / 16;
    const int MT = g.M <= 16 ? 1 : 2;
    double best = 1e300;
    for (int S = 1; S <= nsg && S <= kSpMaxS; S++) {
        if (nsg % S) continue;
        const int nsgS = nsg / S;
        if (nsgS > kSpMaxUnits) continue;
        for (int rounds = 1; rounds <= 16; rounds++) {
            const int nt = (int)(((int64_t)T * S + 256LL * rounds - 1) / (256LL * rounds));
            if (nt > kSpNC || g.M * 33 + nt * 144 > kSpMaxPieces) continue;
            if (split_lds_bytes(g.M, nt, nsgS, MT) > kMaxLds) continue;
            const int rgs = (T + nt - 1) / nt;
            const int sx = S > 1 && nx > 0 ? nx : 0;
            const int grid = (sx ? (rgs + sx - 1) / sx * sx : rgs) * S;
            const double per_wg = (double)nt * nsgS * 2304 + (double)g.M * nsgS * 512 +
                                  (S > 1 ? 3.0 * nt * 16 * g.M * 4 : 0.0);
            const double est = (double)((grid + 255) / 256) * per_wg;
            if (est < best) {
                best = est;
                p = SplitPlan{S, nt, nsgS, MT, grid, (g.M * 33 + nt * 144) * 16, split_lds_bytes(g.M, nt, nsgS, MT),
                              sx, rgs};
            }
            break;                                       // fewer rounds fit first: more would only add rounds
        }
    }
    return best < 1e300;
}

// Partials of one K-split GEMM, [S][N][Mp] fp32 (0 when the plan does not
// split K), rounded up to 256 bytes.
size_t partial_bytes(const GemmArgs& g, const SplitPlan& p) {
    return p.S > 1 ? ((size_t)p.S * g.N * ((g.M + 3) & ~3) * 4 + 255) & ~(size_t)255 : 0;
}

// The exchange's slots of one K-split GEMM: its partials, then its readers' tags.
size_t slot_bytes(const GemmArgs& g, const SplitPlan& p) {
    if (p.S <= 1) return 0;
    return (size_t)tag_offset(p.S, g.N, (g.M + 3) & ~3) + (((size_t)p.rgs * 4 + 255) & ~(size_t)255);
}

// A single launch's splits are summed by k_split_sum (a second launch) where
// the XCD count is unknown (no XCD-local exchange), where the row groups do not
// fill whole XCD rounds (the exchange's placement check needs every workgroup
// to hold a role: no padding), and where the grid takes two or more full
// rounds of one workgroup per CU: the row groups' readers then
// run after everyone else (17408x5120 at M = 16, 512 workgroups: 23.1 against
// 23.8-24.3 us in the kernel).  A grid of more than one round but less than two
// keeps the exchange in the kernel (7168x5120 at M = 32, 448 workgroups: 17.9
// -> 17.1 us), and so does one round (5120^2 at M = 16-32: the second launch
// cost 0.4-1 us).
bool split_second_launch(const SplitPlan& p) {
    const int cus = device_cus() > 0 ? device_cus() : 256;
    return p.S > 1 && (p.nx == 0 || p.rgs % p.nx != 0 || p.grid >= 2 * cus);
}

// The single-launch kernel's packed arguments (k_gemm_split).
bool split_packed_args(const GemmArgs& g, const SplitPlan& p, int slots, uint32_t& X, uint32_t& Y) {
    if (g.N < 1 || g.N >= (1 << 24) || g.M < 1 || g.M > 32 || g.K / 256 > 0xFFF || p.nt > 15 || p.S > 63 ||
        p.nx > 31)
        return false;
    X = (uint32_t)g.N | (uint32_t)(g.M - 1) << 24 | (uint32_t)(g.out_f16 ? 1 : 0) << 29 | (uint32_t)(slots ? 1 : 0) << 30;
    Y = (uint32_t)(g.K / 256) | (uint32_t)p.nt << 12 | (uint32_t)p.S << 16 | (uint32_t)p.nx << 22;
    return true;
}

template <int QT, int MT, bool SUM2>
hipError_t launch_split_k(const GemmArgs& g, const SplitPlan& p, const Scratch* scratch, hipStream_t st) {
    auto k = k_gemm_split<QT, MT, SUM2>;
    static std::atomic<uint64_t> attr_set{0};          // one bit per device: LDS limit raised
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    const uint64_t bit = 1ull << (dev & 63);
    if (!(attr_set.load(std::memory_order_acquire) & bit)) {
        e = hipFuncSetAttribute((const void*)k, hipFuncAttributeMaxDynamicSharedMemorySize, kMaxLds);
        if (e != hipSuccess) return e;
        attr_set.fetch_or(bit, std::memory_order_acq_rel);
    }
    float* parts = nullptr;
    const int slots = !SUM2 && p.S > 1;
    if (p.S > 1) {
        e = slots ? slot_workspace(scratch, st, slot_bytes(g, p), &parts)
                  : partial_workspace(scratch, st, partial_bytes(g, p), &parts);
        if (e != hipSuccess) return e;
    }
    uint32_t X = 0, Y = 0;
    if (!split_packed_args(g, p, slots, X, Y)) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k, dim3(p.grid), dim3(64 * (kSpNC + kSpNL)), p.lds, st, g.W, g.A, g.Waux, g.C, parts, g.lda,
                       g.ldc, X, Y);
    e = hipGetLastError();
    if (e != hipSuccess || !SUM2) return e;
    hipLaunchKernelGGL(k_split_sum, dim3((g.N + 31) / 32), dim3(256), 0, st, (const float*)parts, g.C, g.ldc,
                       g.out_f16, g.M, g.N, p.S);
    return hipGetLastError();
}

template <int QT, int MT>
hipError_t launch_split(const GemmArgs& g, const SplitPlan& p, const Scratch* scratch, hipStream_t st) {
    return split_second_launch(p) ? launch_split_k<QT, MT, true>(g, p, scratch, st)
                                  : launch_split_k<QT, MT, false>(g, p, scratch, st);
}

template <int QT>
hipError_t dispatch_split(const GemmArgs& g, const SplitPlan& p, const Scratch* scratch, hipStream_t st) {
    return p.MT == 1 ? launch_split<QT, 1>(g, p, scratch, st) : launch_split<QT, 2>(g, p, scratch, st);
}

// Up to kSpMaxJobs GEMMs of one format and one m-tile count in one launch.
template <int QT, int MT>
hipError_t launch_split_batched(const GemmArgs* gs, const SplitPlan* ps, int n, int nx, const Scratch* scratch,
                                hipStream_t st) {
    auto k = k_gemm_split_batched<QT, MT>;
    static std::atomic<uint64_t> attr_set{0};          // one bit per device: LDS limit raised
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    const uint64_t bit = 1ull << (dev & 63);
    if (!(attr_set.load(std::memory_order_acquire) & bit)) {
        e = hipFuncSetAttribute((const void*)k, hipFuncAttributeMaxDynamicSharedMemorySize, kMaxLds);
        if (e != hipSuccess) return e;
        attr_set.fetch_or(bit, std::memory_order_acq_rel);
    }
    // one workspace for the launch: the poison word's header, then every
    // job's partial slots at 256-byte offsets
    size_t pb[kSpMaxJobs] = {}, ptot = 0;
    bool any = false;
    for (int i = 0; i < n; i++) {
        pb[i] = slot_bytes(gs[i], ps[i]);
        ptot += pb[i];
        any = any || ps[i].S > 1;
    }
    float* parts = nullptr;
    unsigned* poison = nullptr;
    if (any) {
        if (nx == 0) return hipErrorInvalidValue;        // no XCD-local exchange: split_batched_supports refuses
        e = slot_workspace(scratch, st, ptot, &parts);
        if (e != hipSuccess) return e;
        poison = (unsigned*)((uint8_t*)parts - kSlotHeader);
    }
    SplitJobs jobs = {};
    jobs.n = n;
    jobs.out_f16 = gs[0].out_f16;
    jobs.nx = nx;
    jobs.slots = any;
    jobs.poison = poison;
    int grid = 0, lds = 0;
    size_t po = 0;
    for (int i = 0; i < n; i++) {
        const GemmArgs& g = gs[i];
        const SplitPlan& p = ps[i];
        jobs.job[i] = SplitJob{g.W, g.Waux, g.A, g.C, p.S > 1 ? (float*)((uint8_t*)parts + po) : nullptr,
                               g.lda, g.ldc, g.M, g.N, g.K, p.nt, p.S, p.nsgS, p.unit_bytes, grid};
        po += pb[i];
        // with the XCD-local exchange every job starts on XCD 0 (its grid is
        // padded to whole rounds of the XCD round robin; for S = 1 the padding
        // workgroups exit at once)
        grid += nx > 0 ? (p.grid + nx - 1) / nx * nx : p.grid;
        lds = std::max(lds, p.lds);
    }
    hipLaunchKernelGGL(k, dim3(grid), dim3(64 * (kSpNC + kSpNL)), lds, st, jobs);
    return hipGetLastError();
}

}  // namespace

bool split_supports(const GemmArgs& g) {
    SplitPlan p;
    if (g.qtype == QT_PLANES && ((uintptr_t)g.Waux & 15)) return false;
    return plan_split(g, p, device_xcds());
}

bool split_multi_round(const GemmArgs& g) {
    SplitPlan p;
    const int cus = device_cus();
    return plan_split(g, p, device_xcds()) && cus > 0 && p.grid > cus;
}

size_t split_scratch_bytes(const GemmArgs& g) {
    SplitPlan p;
    if (!plan_split(g, p, device_xcds()) || p.S <= 1) return 0;
    return split_second_launch(p) ? partial_bytes(g, p) : kSlotHeader + slot_bytes(g, p);
}

WsNeed split_ws_need(const GemmArgs& g) {
    WsNeed w;
    SplitPlan p;
    if (!plan_split(g, p, device_xcds()) || p.S <= 1) return w;
    if (split_second_launch(p)) w.p = partial_bytes(g, p);
    else w.s = kSlotHeader + slot_bytes(g, p);
    return w;
}

// The slots one launch of gemm_split_batched takes for each launch of up to
// kSpMaxJobs GEMMs (the header, then every job's partials side by side); the
// largest of them.
size_t split_batched_slot_bytes(const GemmArgs* gs, int n) {
    const int nx = device_xcds();
    size_t worst = 0;
    for (int i0 = 0; i0 < n; i0 += kSpMaxJobs) {
        size_t tot = 0;
        bool any = false;
        for (int i = i0; i < std::min(n, i0 + kSpMaxJobs); i++) {
            SplitPlan p;
            if (!plan_split(gs[i], p, nx)) continue;
            tot += slot_bytes(gs[i], p);
            any = any || p.S > 1;
        }
        if (any) worst = std::max(worst, kSlotHeader + tot);
    }
    return worst;
}

WsNeed split_batched_ws_need(const GemmArgs* gs, int n) {
    WsNeed w;
    w.s = split_batched_slot_bytes(gs, n);
    return w;
}

bool split_batched_supports(const GemmArgs* gs, int n) {
    if (n < 1) return false;
    const int nx = device_xcds();
    for (int i = 0; i < n; i++) {
        SplitPlan p;
        if (gs[i].qtype != gs[0].qtype || gs[i].out_f16 != gs[0].out_f16) return false;
        if ((gs[i].M <= 16) != (gs[0].M <= 16)) return false;      // one m-tile count per launch
        if (gs[i].qtype == QT_PLANES && ((uintptr_t)gs[i].Waux & 15)) return false;
        if (!plan_split(gs[i], p, nx)) return false;
        // the exchange needs the XCD round robin, and whole rounds of row groups
        if (p.S > 1 && (p.nx == 0 || p.rgs % p.nx != 0)) return false;
    }
    return true;
}

size_t split_batched_scratch_bytes(const GemmArgs* gs, int n) { return split_batched_slot_bytes(gs, n); }

hipError_t gemm_split_batched(const GemmArgs* gs, int n, const Scratch* scratch, hipStream_t st) {
    if (!split_batched_supports(gs, n)) return hipErrorInvalidValue;
    const int nx = device_xcds();
    for (int i0 = 0; i0 < n; i0 += kSpMaxJobs) {
        const int m = std::min(kSpMaxJobs, n - i0);
        SplitPlan ps[kSpMaxJobs];
        int bnx = 0;                                     // XCD-local exchange if any job splits K
        for (int i = 0; i < m; i++) {
            plan_split(gs[i0 + i], ps[i], nx);
            if (ps[i].nx) bnx = ps[i].nx;
        }
        const bool mt1 = gs[0].M <= 16;
        hipError_t e;
        switch (gs[0].qtype) {
            case QT_Q4_K:
                e = mt1 ? launch_split_batched<QT_Q4_K, 1>(gs + i0, ps, m, bnx, scratch, st)
                        : launch_split_batched<QT_Q4_K, 2>(gs + i0, ps, m, bnx, scratch, st);
                break;
            case QT_PLANES:
                e = mt1 ? launch_split_batched<QT_PLANES, 1>(gs + i0, ps, m, bnx, scratch, st)
                        : launch_split_batched<QT_PLANES, 2>(gs + i0, ps, m, bnx, scratch, st);
                break;
            default:
                e = mt1 ? launch_split_batched<QT_Q4_0, 1>(gs + i0, ps, m, bnx, scratch, st)
                        : launch_split_batched<QT_Q4_0, 2>(gs + i0, ps, m, bnx, scratch, st);
                break;
        }
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

hipError_t gemm_split(const GemmArgs& g, const Scratch* scratch, hipStream_t st) {
    SplitPlan p;
    if (!plan_split(g, p, device_xcds())) return hipErrorInvalidValue;
    switch (g.qtype) {
        case QT_Q4_K: return dispatch_split<QT_Q4_K>(g, p, scratch, st);
        case QT_PLANES: return dispatch_split<QT_PLANES>(g, p, scratch, st);
        default: return dispatch_split<QT_Q4_0>(g, p, scratch, st);
    }
}

}  // namespace bf
