// C-ABI front end of libbusfill: validation, dispatch, error reporting.
// Declarations and the reference interfaces they replace: include/busfill.h.
#include "busfill.h"

#include <atomic>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <algorithm>
#include <map>
#include <memory>
#include <mutex>
#include <thread>
#include <tuple>
#include <vector>

#include "bf_device.h"
#include "bf_launch.h"

namespace {

thread_local char g_last_error[512] = "";

bf_status fail(bf_status st, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_last_error, sizeof g_last_error, fmt, ap);
    va_end(ap);
    return st;
}

bf_status from_hip(hipError_t e, const char* what) {
    if (e == hipSuccess) return BF_OK;
    return fail(BF_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

bool aligned(const void* p, uintptr_t a) { return ((uintptr_t)p & (a - 1)) == 0; }

// Held while a call plans, secures its workspace and enqueues its launches:
// one lock per (device, stream; per host thread for hipStreamPerThread), so
// the launches of one call stay together on the stream when several host
// threads call on it.  A call of two or more launches (a kernel and its
// second-launch sum, a slot fill and its kernel, the ggml hook's staging and
// its GEMMs) shares the stream's workspace between them; another call's
// launches in between would overwrite it.  Recursive: an entry point that
// calls another takes it again.
std::unique_lock<std::recursive_mutex> stream_lock(void* stream) {
    static std::mutex mu;
    static std::map<std::tuple<int, uintptr_t, std::thread::id>, std::unique_ptr<std::recursive_mutex>> locks;
    const hipStream_t st = (hipStream_t)stream;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) dev = -1;
    const std::thread::id tid = st == hipStreamPerThread ? std::this_thread::get_id() : std::thread::id();
    std::recursive_mutex* m = nullptr;
    {
        std::lock_guard<std::mutex> g(mu);
        std::unique_ptr<std::recursive_mutex>& slot = locks[{dev, (uintptr_t)st, tid}];
        if (!slot) slot.reset(new std::recursive_mutex);
        m = slot.get();
    }
    return std::unique_lock<std::recursive_mutex>(*m);
}

// A K-split launch: the one error of its own is a first use of a stream's
// workspace while the stream is being captured.
bf_status from_split(hipError_t e, const char* what) {
    if (e == hipErrorStreamCaptureUnsupported)
        return fail(BF_ERR_UNSUPPORTED, "%s: the K-split kernel's workspace for this stream is allocated on its first "
                                        "use, which cannot happen during stream capture; make one uncaptured call of "
                                        "this shape (or a larger one) on the stream first", what);
    return from_hip(e, what);
}

constexpr int kMaxMPerLaunch = 128;   // MFMA kernels cover up to 8 batch tiles of 16
constexpr int kDot2MaxM = 4;          // crossover dot2 -> MFMA (see the batch sweep)
constexpr int kSplitMaxM = 32;        // batch rows of one K-split launch

bf_status check_weights(bf_qtype qt, const void* W, const void* W_aux, int N, int K) {
    if (qt != BF_Q4_0 && qt != BF_Q4_0_PLANES && qt != BF_Q4_K)
        return fail(BF_ERR_INVALID, "unknown qtype %d", (int)qt);
    if (!W) return fail(BF_ERR_INVALID, "W is NULL");
    if (qt == BF_Q4_0_PLANES) {
        if (!W_aux) return fail(BF_ERR_INVALID, "W_aux (Ws scale plane) is NULL for BF_Q4_0_PLANES");
        if (!aligned(W_aux, 2)) return fail(BF_ERR_INVALID, "Ws is not 2-byte aligned");
    } else if (W_aux) {
        return fail(BF_ERR_INVALID, "W_aux must be NULL for qtype %d", (int)qt);
    }
    if (N < 1 || K < 1) return fail(BF_ERR_INVALID, "N=%d K=%d must be >= 1", N, K);
    if (qt == BF_Q4_K && K % 256 != 0) return fail(BF_ERR_INVALID, "K=%d is not a multiple of 256 (Q4_K)", K);
    if (K % 32 != 0) return fail(BF_ERR_INVALID, "K=%d is not a multiple of 32", K);
    if (qt == BF_Q4_0 && !aligned(W, 2)) return fail(BF_ERR_INVALID, "W is not 2-byte aligned");
    return BF_OK;
}

// Batches of 9-32 rows on large matrices (3 * 2^24 weights or more, 28 MB of
// Q4_K), measured per kernel: the dense kernel (one workgroup per CU over
// equal shares of the units, sums in a second launch) beats the K-split
// kernel at every batch when K >= N (4096x13824, 8192x8192, 6144x16384,
// 5120x17408: 19.9-28.8 us against 21-42 us at M = 9-32) and from 17 rows
// when N > K; below that the K-split kernel is faster there (17408x5120 at
// M = 9-16: 25 against 28-31 us; 13824x4096: 19 against 21 us) and the LDS
// kernel's all-of-A form is not (31 us at M = 9).  Smaller matrices keep the
// automatic order (7168x5120 at M = 16: K-split 11.7 against dense 18.5 us).
bf_algo mid_batch_choice(const bf::GemmArgs& g) {
    if (g.M < 9 || g.M > kSplitMaxM) return BF_ALGO_AUTO;
    // 17-32 rows whose K-split plan takes more than one round of workgroups
    // (the activations leave room for fewer tiles per workgroup): the dense
    // kernel (7168 x 5120 at M = 32: 15.1 against 17.3 us; at M = 24 the
    // split plan fits one round and stays, 12.1 against 14.9)
    if (g.M > 16 && (int64_t)g.N * g.K < 3 * (int64_t(1) << 24))
        return bf::split_multi_round(g) && bf::dense_supports(g) ? BF_ALGO_DENSE : BF_ALGO_AUTO;
    if ((int64_t)g.N * g.K < 3 * (int64_t(1) << 24)) return BF_ALGO_AUTO;
    if (g.N > g.K && g.M <= 16) return bf::split_supports(g) ? BF_ALGO_SPLIT : BF_ALGO_AUTO;
    return bf::dense_supports(g) ? BF_ALGO_DENSE : BF_ALGO_AUTO;
}

bool fast_eligible(const bf::GemmArgs& g) {
    if (g.K % 256 != 0) return false;
    if (!aligned(g.A, 16) || g.lda % 8 != 0) return false;
    if (!aligned(g.W, 16)) return false;
    if (g.qtype == bf::QT_PLANES && !aligned(g.Waux, 4)) return false;
    return true;
}

// The kernel bf_gemm launches for g when it takes one launch of a kernel that
// has a batched form (BF_ALGO_LDS, _SPLIT or _DENSE); BF_ALGO_AUTO otherwise
// (several launches, or another kernel).
bf_algo one_launch_algo(const bf::GemmArgs& g) {
    if (!fast_eligible(g) || g.M > kMaxMPerLaunch) return BF_ALGO_AUTO;
    // above 32 rows bf_gemm takes one launch only where the dense kernel serves g
    if (g.M > kSplitMaxM && !bf::dense_supports(g)) return BF_ALGO_AUTO;
    const bf_algo mid = mid_batch_choice(g);
    if (mid != BF_ALGO_AUTO) return mid;
    if (bf::lds_supports(g)) return BF_ALGO_LDS;
    if (bf::split_supports(g)) return BF_ALGO_SPLIT;
    return g.M > kSplitMaxM ? BF_ALGO_DENSE : BF_ALGO_AUTO;
}

bf_status check_gemm(bf_qtype qtype, const void* W, const void* W_aux, const uint16_t* A, int lda, void* C,
                     int ldc, bf_otype otype, int M, int N, int K) {
    bf_status st = check_weights(qtype, W, W_aux, N, K);
    if (st != BF_OK) return st;
    if (!A || !C) return fail(BF_ERR_INVALID, "A or C is NULL");
    if (M < 1) return fail(BF_ERR_INVALID, "M=%d must be >= 1", M);
    if (lda < K) return fail(BF_ERR_INVALID, "lda=%d < K=%d", lda, K);
    if (ldc < N) return fail(BF_ERR_INVALID, "ldc=%d < N=%d", ldc, N);
    if (otype != BF_OUT_F32 && otype != BF_OUT_F16) return fail(BF_ERR_INVALID, "unknown otype %d", (int)otype);
    if (!aligned(A, 2)) return fail(BF_ERR_INVALID, "A is not 2-byte aligned");
    if (!aligned(C, otype == BF_OUT_F32 ? 4 : 2)) return fail(BF_ERR_INVALID, "C is not aligned to its element");
    return BF_OK;
}

// One launch of a bf_gemm call: a slice of batch rows and its kernel.
struct Planned {
    bf::GemmArgs g;
    bf_algo use;
};

// The launches a call makes, each checked against its kernel's limits before
// anything is enqueued (BF_ERR_UNSUPPORTED for an explicit kernel family that
// cannot serve a slice).
bf_status plan_gemm(bf_qtype qtype, const void* W, const void* W_aux, const uint16_t* A, int lda, void* C, int ldc,
                    bf_otype otype, int M, int N, int K, bf_algo algo, std::vector<Planned>& out) {
    const size_t csize = otype == BF_OUT_F32 ? 4 : 2;
    // Batches above 32 rows: the dense kernel, all batch rows of a launch per
    // workgroup (the weights streamed once per 128 rows); where it cannot
    // serve the shape, the K-split kernel over slices of 32 rows (the weights
    // streamed once per slice), which beats the register-streaming MFMA
    // kernel, whose activation traffic grows with every 16-row tile.
    int slice = kMaxMPerLaunch;
    bool dense_slices = false;
    auto args = [&](int m0, int rows) {
        bf::GemmArgs g;
        g.qtype = (int)qtype;
        g.W = (const uint8_t*)W;
        g.Waux = (const uint8_t*)W_aux;
        g.A = A + (int64_t)m0 * lda;
        g.lda = lda;
        g.C = (char*)C + (size_t)m0 * ldc * csize;
        g.ldc = ldc;
        g.out_f16 = otype == BF_OUT_F16;
        g.M = rows;
        g.N = N;
        g.K = K;
        return g;
    };
    if (algo == BF_ALGO_AUTO && M > kSplitMaxM) {
        bf::GemmArgs probe = args(0, M < kMaxMPerLaunch ? M : kMaxMPerLaunch);
        dense_slices = fast_eligible(probe) && bf::dense_supports(probe);
        probe.M = kSplitMaxM;
        if (!dense_slices && fast_eligible(probe) && bf::split_supports(probe)) slice = kSplitMaxM;
    }
    for (int m0 = 0; m0 < M; m0 += slice) {
        const bf::GemmArgs g = args(m0, M - m0 < slice ? M - m0 : slice);
        const bool fast = fast_eligible(g);
        bf_algo use = algo;
        if (use == BF_ALGO_AUTO) {
            const bf_algo mid = mid_batch_choice(g);
            if (!fast) use = BF_ALGO_SIMPLE;
            else if (mid != BF_ALGO_AUTO) use = mid;
            else if (bf::lds_supports(g)) use = BF_ALGO_LDS;
            else if (bf::split_supports(g)) use = BF_ALGO_SPLIT;
            else if (dense_slices && bf::dense_supports(g)) use = BF_ALGO_DENSE;
            else if (bf::slab_supports(g)) use = BF_ALGO_SLAB;
            else if (g.M <= kDot2MaxM && bf::dot2_supports(g)) use = BF_ALGO_DOT2;
            else use = BF_ALGO_MFMA;
        }
        switch (use) {
            case BF_ALGO_MFMA:
                if (!fast) return fail(BF_ERR_UNSUPPORTED, "MFMA path needs K %% 256 == 0, 16-byte aligned A/W, lda %% 8 == 0");
                break;
            case BF_ALGO_DOT2:
                if (!fast || !bf::dot2_supports(g))
                    return fail(BF_ERR_UNSUPPORTED, "dot2 path does not serve M=%d K=%d with these alignments", g.M, K);
                break;
            case BF_ALGO_SLAB:
                if (!fast || !bf::slab_supports(g))
                    return fail(BF_ERR_UNSUPPORTED, "slab path does not serve qtype %d M=%d N=%d K=%d",
                                (int)qtype, g.M, N, K);
                break;
            case BF_ALGO_SPLIT:
                if (!fast || !bf::split_supports(g))
                    return fail(BF_ERR_UNSUPPORTED, "K-split path does not serve qtype %d M=%d N=%d K=%d",
                                (int)qtype, g.M, N, K);
                break;
            case BF_ALGO_DENSE:
                if (!fast || !bf::dense_supports(g))
                    return fail(BF_ERR_UNSUPPORTED, "dense path does not serve qtype %d M=%d N=%d K=%d",
                                (int)qtype, g.M, N, K);
                break;
            case BF_ALGO_LDS:
                if (!fast || !bf::lds_supports(g))
                    return fail(BF_ERR_UNSUPPORTED, "LDS-staged path does not serve M=%d N=%d K=%d with these alignments",
                                g.M, N, K);
                break;
            default:
                use = BF_ALGO_SIMPLE;
                break;
        }
        out.push_back(Planned{g, use});
    }
    return BF_OK;
}

// Workspace bytes one launch takes from a caller's buffer (the exchange's
// counters, cleared on the stream by each launch, and partial sums).
size_t scratch_need(const Planned& l) {
    if (l.use == BF_ALGO_SPLIT) return bf::split_scratch_bytes(l.g);
    if (l.use == BF_ALGO_DENSE) return bf::dense_scratch_bytes(l.g);
    return 0;
}

// ... or from the library's workspace for the stream.
bf::WsNeed ws_need(const Planned& l) {
    if (l.use == BF_ALGO_SPLIT) return bf::split_ws_need(l.g);
    if (l.use == BF_ALGO_DENSE) return bf::dense_ws_need(l.g);
    return bf::WsNeed{};
}

const char* kernel_name(bf_algo a) { return a == BF_ALGO_SPLIT ? "K-split" : a == BF_ALGO_DENSE ? "dense" : "other"; }

// Before anything is enqueued: a caller's buffer must hold every launch's
// need (the launches run in stream order, so they share it); otherwise the
// stream's workspace is made large enough for all of them now, so that no
// launch of the call can fail for want of it.
bf_status secure_workspace(const std::vector<Planned>& ls, const bf::Scratch* scratch, hipStream_t hs,
                           const char* who, const char* holder) {
    if (scratch) {
        for (const Planned& l : ls) {
            const size_t need = scratch_need(l);
            if (need > scratch->bytes)
                return fail(BF_ERR_INVALID, "%s: M=%d N=%d K=%d needs %zu bytes for the %s kernel's exchange, "
                            "more than the %zu bytes of %s", who, l.g.M, l.g.N, l.g.K, need, kernel_name(l.use),
                            scratch->bytes, holder);
        }
        return BF_OK;
    }
    bf::WsNeed w;
    for (const Planned& l : ls) w.merge(ws_need(l));
    return from_split(bf::reserve_workspace(hs, w), who);
}

bf_status launch_planned(const Planned& l, const bf::Scratch* scratch, hipStream_t hs) {
    hipError_t e;
    switch (l.use) {
        case BF_ALGO_MFMA: e = bf::gemm_mfma(l.g, hs); break;
        case BF_ALGO_DOT2: e = bf::gemm_dot2(l.g, hs); break;
        case BF_ALGO_SLAB: e = bf::gemm_slab(l.g, hs); break;
        case BF_ALGO_SPLIT: e = bf::gemm_split(l.g, scratch, hs); break;
        case BF_ALGO_DENSE: e = bf::gemm_dense(l.g, scratch, hs); break;
        case BF_ALGO_LDS: e = bf::gemm_lds(l.g, hs); break;
        default: e = bf::gemm_simple(l.g, hs); break;
    }
    return l.use == BF_ALGO_SPLIT || l.use == BF_ALGO_DENSE ? from_split(e, "kernel launch") : from_hip(e, "kernel launch");
}

// scratch: the caller's workspace (bf_gemm_ws, bf_gemm_noalloc) or nullptr
// (the library's workspace for the stream).
bf_status run_gemm(bf_qtype qtype, const void* W, const void* W_aux, const uint16_t* A, int lda, void* C,
                   int ldc, bf_otype otype, int M, int N, int K, bf_algo algo, void* stream,
                   const bf::Scratch* scratch = nullptr, const char* who = "bf_gemm",
                   const char* holder = "workspace given") {
    g_last_error[0] = '\0';
    bf_status st = check_gemm(qtype, W, W_aux, A, lda, C, ldc, otype, M, N, K);
    if (st != BF_OK) return st;
    if (algo < BF_ALGO_AUTO || algo > BF_ALGO_DENSE) return fail(BF_ERR_INVALID, "unknown algo %d", (int)algo);
    std::vector<Planned> ls;
    st = plan_gemm(qtype, W, W_aux, A, lda, C, ldc, otype, M, N, K, algo, ls);
    if (st != BF_OK) return st;
    hipStream_t hs = (hipStream_t)stream;
    // calls on the LDS-staged and other single-launch kernels share nothing
    // between launches: no lock on the batch 1-8 path
    bool shares = scratch != nullptr;
    for (const Planned& l : ls) shares = shares || l.use == BF_ALGO_SPLIT || l.use == BF_ALGO_DENSE;
    std::unique_lock<std::recursive_mutex> held;
    if (shares) held = stream_lock(stream);
    st = secure_workspace(ls, scratch, hs, who, holder);
    if (st != BF_OK) return st;
    for (const Planned& l : ls) {
        st = launch_planned(l, scratch, hs);
        if (st != BF_OK) return st;
    }
    return BF_OK;
}

// Workspace bytes of a call with lda = K, ldc = N and aligned operands (the
// operands' addresses only decide between the fast kernels and the simple one,
// which needs none).
size_t gemm_workspace_bytes(bf_qtype qtype, bf_otype otype, int M, int N, int K) {
    uint8_t* const fake = (uint8_t*)(uintptr_t)4096;      // aligned placeholders, never dereferenced
    if (check_gemm(qtype, fake, qtype == BF_Q4_0_PLANES ? fake : nullptr, (const uint16_t*)fake, K, fake, N, otype,
                   M, N, K) != BF_OK)
        return 0;
    std::vector<Planned> ls;
    if (plan_gemm(qtype, fake, qtype == BF_Q4_0_PLANES ? fake : nullptr, (const uint16_t*)fake, K, fake, N, otype, M,
                  N, K, BF_ALGO_AUTO, ls) != BF_OK)
        return 0;
    size_t need = 0;
    for (const Planned& l : ls) need = std::max(need, scratch_need(l));
    return need;
}

// Scratch of bf_gemm_noalloc: the K-split and dense kernels' row-group
// counters and partial sums, in place of the workspace bf_gemm allocates per
// stream (34 MiB: the dense kernel's 256 workgroups x two 128 x 128 fp32
// pieces plus counters for up to 8192 row groups).  Each
// GPU the library runs on holds its own copy until the process ends.  In host
// code `scratch` only names the symbol: its device address comes from
// hipGetSymbolAddress (noalloc_scratch), once per device.
constexpr size_t kNoallocScratch = 34u << 20;
static __device__ __align__(256) uint8_t scratch[kNoallocScratch];

constexpr int kMaxDevices = 64;
std::atomic<uint8_t*> g_scratch_ptr[kMaxDevices];

// The current device's copy of `scratch`: looked up on the first call on each
// device (with that device current) and kept.
bf_status noalloc_scratch(uint8_t** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return fail(BF_ERR_HIP, "hipGetDevice: %s", hipGetErrorString(e));
    if (dev < 0 || dev >= kMaxDevices)
        return fail(BF_ERR_UNSUPPORTED, "device %d: bf_gemm_noalloc serves devices 0-%d", dev, kMaxDevices - 1);
    uint8_t* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
    if (!p) {
        void* addr = nullptr;
        e = hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !addr) return fail(BF_ERR_HIP, "hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
        p = (uint8_t*)addr;
        g_scratch_ptr[dev].store(p, std::memory_order_release);
    }
    *out = p;
    return BF_OK;
}

// A bf_gemm_batched call: its GEMMs grouped by the kernel bf_gemm would give
// each (the results are then the same bits) -- every group of two or more
// shares launches: the LDS-staged kernel at batch 1-8 (one batch size, so one
// kernel shape), the K-split kernel at 9-32 rows (one m-tile count), the
// dense kernel (one batch size) -- and the launches of the rest, which run
// one by one as bf_gemm runs them.
struct BatchedPlan {
    std::vector<std::pair<int, std::vector<bf::GemmArgs>>> groups;   // 0 LDS / 1 K-split / 2 dense
    std::vector<Planned> singles;
};

bf_status plan_batched(bf_qtype qtype, bf_otype otype, int count, const bf_gemm_desc* descs, BatchedPlan& bp) {
    if (count < 0) return fail(BF_ERR_INVALID, "count=%d must be >= 0", count);
    if (count > 0 && !descs) return fail(BF_ERR_INVALID, "descs is NULL");
    for (int i = 0; i < count; i++) {
        const bf_gemm_desc& d = descs[i];
        const bf_status st = check_gemm(qtype, d.W, d.W_aux, d.A, d.lda, d.C, d.ldc, otype, d.M, d.N, d.K);
        if (st != BF_OK) return st;
    }
    std::vector<bf::GemmArgs> gs(count);
    std::map<std::pair<int, int>, std::vector<int>> grp;   // (kind, batch key)
    std::vector<int> single;
    for (int i = 0; i < count; i++) {
        const bf_gemm_desc& d = descs[i];
        bf::GemmArgs& g = gs[i];
        g.qtype = (int)qtype;
        g.W = (const uint8_t*)d.W;
        g.Waux = (const uint8_t*)d.W_aux;
        g.A = d.A;
        g.lda = d.lda;
        g.C = d.C;
        g.ldc = d.ldc;
        g.out_f16 = otype == BF_OUT_F16;
        g.M = d.M;
        g.N = d.N;
        g.K = d.K;
        const bf_algo a = one_launch_algo(g);
        if (a == BF_ALGO_LDS) grp[{0, g.M}].push_back(i);
        else if (a == BF_ALGO_SPLIT) grp[{1, g.M <= 16}].push_back(i);
        else if (a == BF_ALGO_DENSE) grp[{2, g.M}].push_back(i);
        else single.push_back(i);
    }
    for (const auto& kv : grp) {
        const int k = kv.first.first;
        std::vector<bf::GemmArgs> sub;
        for (int i : kv.second) sub.push_back(gs[i]);
        const int n = (int)sub.size();
        const bool ok = n > 1 && (k == 0   ? bf::lds_batched_supports(sub.data(), n)
                                  : k == 1 ? bf::split_batched_supports(sub.data(), n)
                                           : bf::dense_batched_supports(sub.data(), n));
        if (ok) bp.groups.emplace_back(k, std::move(sub));
        else single.insert(single.end(), kv.second.begin(), kv.second.end());
    }
    for (int i : single) {
        const bf_gemm_desc& d = descs[i];
        const bf_status st =
            plan_gemm(qtype, d.W, d.W_aux, d.A, d.lda, d.C, d.ldc, otype, d.M, d.N, d.K, BF_ALGO_AUTO, bp.singles);
        if (st != BF_OK) return st;
    }
    return BF_OK;
}

// The most workspace any one launch of the call takes from a caller's buffer
// (the launches run in stream order, so they share it).
size_t batched_scratch_need(const BatchedPlan& bp) {
    size_t need = 0;
    for (const auto& gr : bp.groups) {
        const int n = (int)gr.second.size();
        if (gr.first == 1) need = std::max(need, bf::split_batched_scratch_bytes(gr.second.data(), n));
        if (gr.first == 2) need = std::max(need, bf::dense_batched_scratch_bytes(gr.second.data(), n));
    }
    for (const Planned& l : bp.singles) need = std::max(need, scratch_need(l));
    return need;
}

bf::WsNeed batched_ws_need(const BatchedPlan& bp) {
    bf::WsNeed w;
    for (const auto& gr : bp.groups) {
        const int n = (int)gr.second.size();
        if (gr.first == 1) w.merge(bf::split_batched_ws_need(gr.second.data(), n));
        if (gr.first == 2) w.merge(bf::dense_batched_ws_need(gr.second.data(), n));
    }
    for (const Planned& l : bp.singles) w.merge(ws_need(l));
    return w;
}

bf_status launch_batched(const BatchedPlan& bp, const bf::Scratch* scratch, hipStream_t hs) {
    for (const auto& gr : bp.groups) {
        const bf::GemmArgs* sub = gr.second.data();
        const int n = (int)gr.second.size();
        const bf_status st = gr.first == 0   ? from_hip(bf::gemm_lds_batched(sub, n, hs), "batched launch")
                             : gr.first == 1 ? from_split(bf::gemm_split_batched(sub, n, scratch, hs), "batched launch")
                                             : from_split(bf::gemm_dense_batched(sub, n, scratch, hs), "batched launch");
        if (st != BF_OK) return st;
    }
    for (const Planned& l : bp.singles) {
        const bf_status st = launch_planned(l, scratch, hs);
        if (st != BF_OK) return st;
    }
    return BF_OK;
}

// A caller's workspace: NULL with 0 bytes (for calls that need none), or a
// 256-byte aligned buffer.
bf_status check_workspace(const void* ws, size_t bytes) {
    if (!ws && bytes) return fail(BF_ERR_INVALID, "workspace is NULL but workspace_bytes is %zu", bytes);
    if (ws && !aligned(ws, 256)) return fail(BF_ERR_INVALID, "workspace is not 256-byte aligned");
    return BF_OK;
}


// ------------------------------------------------------------ ggml mul_mat hook
// ggml_mul_mat's operands checked and cut into one GEMM per (i2, i3) slice of
// dst (ggml.c's ggml_can_mul_mat and ggml_mul_mat fix the shapes; src0 is
// broadcast over src1's outer dimensions by i02 = i2 / r2, i03 = i3 / r3).
struct GgmlCall {
    bf_qtype qt = BF_Q4_0;
    int64_t K = 0, N = 0, M = 0, ne2 = 1, ne3 = 1, r2 = 1, r3 = 1;
    bool stage = false;            // src1 goes through the fp16 staging buffer
    size_t stage_bytes = 0;
    bool fused = false;            // one fp32 row on the batch-1 LDS kernel, rounded as it loads (fg)
    bf::GemmArgs fg;
};

constexpr size_t align256(size_t b) { return (b + 255) & ~(size_t)255; }

bf_status check_ggml(const bf_ggml_tensor* s0, const bf_ggml_tensor* s1, const bf_ggml_tensor* d, GgmlCall& c) {
    if (!s0 || !s1 || !d) return fail(BF_ERR_INVALID, "ggml mul_mat: a tensor is NULL");
    const bf_ggml_tensor* ts[3] = {s0, s1, d};
    const char* nm[3] = {"src0", "src1", "dst"};
    for (int t = 0; t < 3; t++) {
        if (!ts[t]->data) return fail(BF_ERR_INVALID, "ggml mul_mat: %s data is NULL", nm[t]);
        for (int i = 0; i < 4; i++)
            if (ts[t]->ne[i] < 1) return fail(BF_ERR_INVALID, "ggml mul_mat: %s ne[%d]=%lld must be >= 1", nm[t], i,
                                              (long long)ts[t]->ne[i]);
    }
    if (s0->type != BF_GGML_Q4_0 && s0->type != BF_GGML_Q4_K)
        return fail(BF_ERR_UNSUPPORTED, "ggml mul_mat: src0 type %d (the hook serves Q4_0 = 2 and Q4_K = 12)",
                    (int)s0->type);
    if (s1->type != BF_GGML_F32 && s1->type != BF_GGML_F16)
        return fail(BF_ERR_UNSUPPORTED, "ggml mul_mat: src1 type %d (the hook serves F32 and F16)", (int)s1->type);
    if (d->type != BF_GGML_F32)
        return fail(BF_ERR_UNSUPPORTED, "ggml mul_mat: dst type %d (the hook writes F32)", (int)d->type);
    // the shapes ggml_mul_mat accepts and the one it gives dst
    if (s0->ne[0] != s1->ne[0])
        return fail(BF_ERR_INVALID, "ggml mul_mat: src0 ne[0]=%lld != src1 ne[0]=%lld", (long long)s0->ne[0],
                    (long long)s1->ne[0]);
    if (s1->ne[2] % s0->ne[2] || s1->ne[3] % s0->ne[3])
        return fail(BF_ERR_INVALID, "ggml mul_mat: src1 ne[2], ne[3] must be multiples of src0's (broadcast)");
    if (d->ne[0] != s0->ne[1] || d->ne[1] != s1->ne[1] || d->ne[2] != s1->ne[2] || d->ne[3] != s1->ne[3])
        return fail(BF_ERR_INVALID, "ggml mul_mat: dst ne must be {src0 ne[1], src1 ne[1], src1 ne[2], src1 ne[3]}");
    c.qt = s0->type == BF_GGML_Q4_K ? BF_Q4_K : BF_Q4_0;
    const int64_t blk = c.qt == BF_Q4_K ? 256 : 32, bb = c.qt == BF_Q4_K ? 144 : 18;
    c.K = s0->ne[0];
    c.N = s0->ne[1];
    c.M = s1->ne[1];
    c.ne2 = s1->ne[2];
    c.ne3 = s1->ne[3];
    c.r2 = s1->ne[2] / s0->ne[2];
    c.r3 = s1->ne[3] / s0->ne[3];
    if (c.K % blk) return fail(BF_ERR_INVALID, "ggml mul_mat: src0 ne[0]=%lld is not whole blocks", (long long)c.K);
    if (c.K > INT32_MAX || c.N > INT32_MAX || c.M > INT32_MAX || c.ne2 > (1 << 20) || c.ne3 > (1 << 20) ||
        c.ne2 * c.ne3 > (1 << 20) || c.M * c.ne2 * c.ne3 > (int64_t(1) << 40) / c.K)
        return fail(BF_ERR_UNSUPPORTED, "ggml mul_mat: a dimension exceeds 2^31 - 1, more than 2^20 slices, or more "
                                        "than 2^40 activations");
    // src0: whole rows of blocks, one after the other (a matrix per slice)
    if (s0->nb[0] != (uint64_t)bb || s0->nb[1] != (uint64_t)(c.K / blk * bb))
        return fail(BF_ERR_UNSUPPORTED, "ggml mul_mat: src0 rows must be contiguous blocks (nb[0]=%lld, nb[1]=%lld)",
                    (long long)bb, (long long)(c.K / blk * bb));
    if (c.qt == BF_Q4_0 && (((uintptr_t)s0->data | s0->nb[2] | s0->nb[3]) & 1))
        return fail(BF_ERR_UNSUPPORTED, "ggml mul_mat: Q4_0 matrices must start 2-byte aligned");
    // dst: F32 rows, slices that do not overlap
    const uint64_t ldc = d->nb[1] / 4;
    if (d->nb[0] != 4 || d->nb[1] % 4 || ldc < (uint64_t)c.N || ldc > INT32_MAX ||
        (((uintptr_t)d->data | d->nb[2] | d->nb[3]) & 3))
        return fail(BF_ERR_UNSUPPORTED, "ggml mul_mat: dst must be F32 rows (nb[0] = 4, nb[1] >= 4 ne[0])");
    if ((c.ne2 > 1 && d->nb[2] < (uint64_t)c.M * d->nb[1]) || (c.ne3 > 1 && d->nb[3] < (uint64_t)c.ne2 * d->nb[2]))
        return fail(BF_ERR_UNSUPPORTED, "ggml mul_mat: dst slices overlap");
    // src1: element-aligned strides; fp16 rows the GEMM reads in place, or staging
    const uint64_t es = s1->type == BF_GGML_F32 ? 4 : 2;
    if (((uintptr_t)s1->data | s1->nb[0] | s1->nb[1] | s1->nb[2] | s1->nb[3]) & (es - 1))
        return fail(BF_ERR_UNSUPPORTED, "ggml mul_mat: src1 strides must be multiples of its element size");
    c.stage = !(s1->type == BF_GGML_F16 && s1->nb[0] == 2 &&
                (((uintptr_t)s1->data | s1->nb[1] | s1->nb[2] | s1->nb[3]) & 15) == 0 &&
                s1->nb[1] / 2 >= (uint64_t)c.K && s1->nb[1] / 2 <= INT32_MAX);
    c.stage_bytes = c.stage ? align256((size_t)(c.M * c.ne2 * c.ne3) * (size_t)c.K * 2) : 0;
    // One or two fp32 rows (decode steps) where bf_gemm would run the LDS
    // kernel on their fp16 copy in a form whose compute waves load all of A:
    // that kernel rounds the rows as it loads them (the same rounding, so the
    // same bits), and no staging launch runs.
    if (s1->type == BF_GGML_F32 && c.M <= 2 && c.ne2 * c.ne3 == 1 && s1->nb[0] == 4 &&
        (((uintptr_t)s1->data | s1->nb[1]) & 15) == 0 && s1->nb[1] / 4 >= (uint64_t)c.K &&
        s1->nb[1] / 4 <= INT32_MAX) {
        const uint16_t* const fake = (const uint16_t*)(uintptr_t)0x100000;   // aligned fp16 rows (the plan's view)
        std::vector<Planned> ls;
        const bf_status st = plan_gemm(c.qt, s0->data, nullptr, fake, (int)c.K, d->data, (int)(d->nb[1] / 4),
                                       BF_OUT_F32, (int)c.M, (int)c.N, (int)c.K, BF_ALGO_AUTO, ls);
        if (st == BF_OK && ls.size() == 1 && ls[0].use == BF_ALGO_LDS) {
            bf::GemmArgs g = ls[0].g;
            g.A = (const uint16_t*)s1->data;
            g.lda = (int)(s1->nb[1] / 4);
            g.a_f32 = 1;
            if (bf::lds_f32_supports(g)) {
                c.fused = true;
                c.fg = g;
                c.stage = false;
                c.stage_bytes = 0;
            }
        }
        g_last_error[0] = '\0';
    }
    return BF_OK;
}

// The slices' GEMMs, src1 read from `staged` (fp16 rows of K, slice-major) or
// in place, planned as bf_gemm_batched plans them.
bf_status plan_ggml(const GgmlCall& c, const bf_ggml_tensor* s0, const bf_ggml_tensor* s1, const bf_ggml_tensor* d,
                    const uint16_t* staged, BatchedPlan& bp) {
    std::vector<bf_gemm_desc> descs;
    descs.reserve((size_t)(c.ne2 * c.ne3));
    for (int64_t i3 = 0; i3 < c.ne3; i3++)
        for (int64_t i2 = 0; i2 < c.ne2; i2++) {
            bf_gemm_desc g;
            g.W = (const uint8_t*)s0->data + (i3 / c.r3) * s0->nb[3] + (i2 / c.r2) * s0->nb[2];
            g.W_aux = nullptr;
            if (c.stage) {
                g.A = staged + (size_t)((i3 * c.ne2 + i2) * c.M) * (size_t)c.K;
                g.lda = (int)c.K;
            } else {
                g.A = (const uint16_t*)((const uint8_t*)s1->data + i3 * s1->nb[3] + i2 * s1->nb[2]);
                g.lda = (int)(s1->nb[1] / 2);
            }
            g.C = (uint8_t*)d->data + i3 * d->nb[3] + i2 * d->nb[2];
            g.ldc = (int)(d->nb[1] / 4);
            g.M = (int)c.M;
            g.N = (int)c.N;
            g.K = (int)c.K;
            descs.push_back(g);
        }
    return plan_batched(c.qt, BF_OUT_F32, (int)descs.size(), descs.data(), bp);
}

// Any 256-byte aligned address: a plan's kernels depend on A's alignment only.
const uint16_t* const kStagePlaceholder = (const uint16_t*)(uintptr_t)0x100000;

bf_status enqueue_ggml(const GgmlCall& c, const bf_ggml_tensor* s1, uint16_t* staged, const BatchedPlan& bp,
                       const bf::Scratch* scratch, hipStream_t hs) {
    if (c.stage) {
        const bf_status st = from_hip(bf::stage_rows_f16(s1->data, s1->type == BF_GGML_F32, s1->ne, s1->nb, staged, hs),
                                      "ggml mul_mat: staging src1");
        if (st != BF_OK) return st;
    }
    return launch_batched(bp, scratch, hs);
}
}  // namespace

extern "C" {

bf_status bf_gemm(bf_qtype qtype, const void* W, const void* W_aux, const uint16_t* A, int lda, void* C, int ldc,
                  bf_otype otype, int M, int N, int K, void* stream) {
    return run_gemm(qtype, W, W_aux, A, lda, C, ldc, otype, M, N, K, BF_ALGO_AUTO, stream);
}

bf_status bf_gemm_ex(bf_qtype qtype, const void* W, const void* W_aux, const uint16_t* A, int lda, void* C,
                     int ldc, bf_otype otype, int M, int N, int K, bf_algo algo, void* stream) {
    return run_gemm(qtype, W, W_aux, A, lda, C, ldc, otype, M, N, K, algo, stream);
}

bf_status bf_gemm_noalloc(bf_qtype qtype, const void* W, const void* W_aux, const uint16_t* A, int lda, void* C,
                          int ldc, bf_otype otype, int M, int N, int K, void* stream) {
    g_last_error[0] = '\0';
    uint8_t* p = nullptr;
    const bf_status st = noalloc_scratch(&p);
    if (st != BF_OK) return st;
    const bf::Scratch sc{p, kNoallocScratch};
    return run_gemm(qtype, W, W_aux, A, lda, C, ldc, otype, M, N, K, BF_ALGO_AUTO, stream, &sc, "bf_gemm_noalloc",
                    "scratch bf_gemm_noalloc holds per GPU");
}

size_t bf_gemm_workspace_bytes(bf_qtype qtype, bf_otype otype, int M, int N, int K) {
    g_last_error[0] = '\0';
    return gemm_workspace_bytes(qtype, otype, M, N, K);
}

bf_status bf_gemm_ws(bf_qtype qtype, const void* W, const void* W_aux, const uint16_t* A, int lda, void* C, int ldc,
                     bf_otype otype, int M, int N, int K, void* workspace, size_t workspace_bytes, void* stream) {
    g_last_error[0] = '\0';
    const bf_status st = check_workspace(workspace, workspace_bytes);
    if (st != BF_OK) return st;
    const bf::Scratch sc{(uint8_t*)workspace, workspace_bytes};
    return run_gemm(qtype, W, W_aux, A, lda, C, ldc, otype, M, N, K, BF_ALGO_AUTO, stream, &sc, "bf_gemm_ws");
}

bf_status bf_busfill_q4_ws(const uint16_t* A, const uint8_t* Wq, const uint16_t* Ws, float* C, int Bsz, int K, int N,
                           void* workspace, size_t workspace_bytes, void* stream) {
    return bf_gemm_ws(BF_Q4_0_PLANES, Wq, Ws, A, K, C, N, BF_OUT_F32, Bsz, N, K, workspace, workspace_bytes, stream);
}

bf_status bf_gemm_batched(bf_qtype qtype, bf_otype otype, int count, const bf_gemm_desc* descs, void* stream) {
    g_last_error[0] = '\0';
    BatchedPlan bp;
    bf_status st = plan_batched(qtype, otype, count, descs, bp);
    if (st != BF_OK) return st;
    hipStream_t hs = (hipStream_t)stream;
    const auto held = stream_lock(stream);
    st = from_split(bf::reserve_workspace(hs, batched_ws_need(bp)), "bf_gemm_batched");
    if (st != BF_OK) return st;
    return launch_batched(bp, nullptr, hs);
}

size_t bf_gemm_batched_workspace_bytes(bf_qtype qtype, bf_otype otype, int count, const bf_gemm_desc* descs) {
    g_last_error[0] = '\0';
    BatchedPlan bp;
    if (plan_batched(qtype, otype, count, descs, bp) != BF_OK) return 0;
    return batched_scratch_need(bp);
}

bf_status bf_gemm_batched_ws(bf_qtype qtype, bf_otype otype, int count, const bf_gemm_desc* descs, void* workspace,
                             size_t workspace_bytes, void* stream) {
    g_last_error[0] = '\0';
    bf_status st = check_workspace(workspace, workspace_bytes);
    if (st != BF_OK) return st;
    BatchedPlan bp;
    st = plan_batched(qtype, otype, count, descs, bp);
    if (st != BF_OK) return st;
    const size_t need = batched_scratch_need(bp);
    if (need > workspace_bytes)
        return fail(BF_ERR_INVALID, "bf_gemm_batched_ws: the call needs %zu bytes of workspace, %zu given", need,
                    workspace_bytes);
    const bf::Scratch sc{(uint8_t*)workspace, workspace_bytes};
    const auto held = stream_lock(stream);
    return launch_batched(bp, need ? &sc : nullptr, (hipStream_t)stream);
}

bf_status bf_gemm_swiglu(bf_qtype qtype, const void* W, const void* W_aux, const uint16_t* gate_up, int ld,
                         void* C, int ldc, bf_otype otype, int M, int N, int K, void* stream) {
    g_last_error[0] = '\0';
    if (ld < 2 * (int64_t)K) return fail(BF_ERR_INVALID, "ld=%d < 2K=%lld", ld, 2 * (long long)K);
    bf_status st = check_gemm(qtype, W, W_aux, gate_up, ld, C, ldc, otype, M, N, K);
    if (st != BF_OK) return st;
    if (!aligned(gate_up, 16) || ld % 8) return fail(BF_ERR_INVALID, "gate_up rows must be 16-byte aligned (ld %% 8 == 0)");
    bf::GemmArgs g;
    g.qtype = (int)qtype;
    g.W = (const uint8_t*)W;
    g.Waux = (const uint8_t*)W_aux;
    g.A = gate_up;
    g.lda = ld;
    g.C = C;
    g.ldc = ldc;
    g.out_f16 = otype == BF_OUT_F16;
    g.M = M;
    g.N = N;
    g.K = K;
    if (!fast_eligible(g) || !bf::lds_swiglu_supports(g))
        return fail(BF_ERR_UNSUPPORTED, "fused SiLU*up GEMM: batch 1-2 with the activations resident in LDS "
                                        "(M=%d N=%d K=%d); use bf_swiglu_f16 then bf_gemm", M, N, K);
    return from_hip(bf::gemm_lds_swiglu(g, (hipStream_t)stream), "kernel launch");
}

bf_status bf_ffn_swiglu_ex(bf_qtype qtype, bf_qweights gate, bf_qweights up, bf_qweights down, const uint16_t* A,
                           int lda, uint16_t* gate_up, int ldgu, void* C, int ldc, bf_otype otype, int M, int K,
                           int F, int N, bf_ffn_form form, void* stream) {
    g_last_error[0] = '\0';
    if (form < BF_FFN_AUTO || form > BF_FFN_CALLS) return fail(BF_ERR_INVALID, "unknown form %d", (int)form);
    if (!gate_up) return fail(BF_ERR_INVALID, "gate_up is NULL");
    if (F < 8 || F % 8) return fail(BF_ERR_INVALID, "F=%d must be a positive multiple of 8", F);
    if (ldgu < 2 * (int64_t)F) return fail(BF_ERR_INVALID, "ldgu=%d < 2F=%lld", ldgu, 2 * (long long)F);
    if (!aligned(gate_up, 16) || ldgu % 8) return fail(BF_ERR_INVALID, "gate_up rows must be 16-byte aligned (ldgu %% 8 == 0)");
    bf_status st = check_gemm(qtype, gate.W, gate.W_aux, A, lda, gate_up, ldgu, BF_OUT_F16, M, F, K);
    if (st == BF_OK) st = check_gemm(qtype, up.W, up.W_aux, A, lda, gate_up + F, ldgu, BF_OUT_F16, M, F, K);
    if (st == BF_OK) st = check_gemm(qtype, down.W, down.W_aux, gate_up, ldgu, C, ldc, otype, M, N, F);
    if (st != BF_OK) return st;
    hipStream_t hs = (hipStream_t)stream;
    bf::GemmArgs gs[3];
    const bf_qweights* w[3] = {&gate, &up, &down};
    for (int i = 0; i < 3; i++) {
        bf::GemmArgs& g = gs[i];
        g.qtype = (int)qtype;
        g.W = (const uint8_t*)w[i]->W;
        g.Waux = (const uint8_t*)w[i]->W_aux;
        g.A = i < 2 ? A : gate_up;
        g.lda = i < 2 ? lda : ldgu;
        g.C = i == 0 ? (void*)gate_up : i == 1 ? (void*)(gate_up + F) : C;
        g.ldc = i < 2 ? ldgu : ldc;
        g.out_f16 = i < 2 ? 1 : otype == BF_OUT_F16;
        g.M = M;
        g.N = i < 2 ? F : N;
        g.K = i < 2 ? K : F;
    }
    const bool fast = fast_eligible(gs[0]) && fast_eligible(gs[1]) && fast_eligible(gs[2]);
    const auto held = stream_lock(stream);
    if (form == BF_FFN_ONE_LAUNCH) {
        if (!fast || !bf::ffn_lds_supports(gs))
            return fail(BF_ERR_UNSUPPORTED, "one-launch feed-forward block: batch 1-2 with every GEMM on the LDS-staged "
                                            "kernel's batch-1 or all-of-A form (M=%d K=%d F=%d N=%d)", M, K, F, N);
        return from_split(bf::ffn_lds(gs, hs), "feed-forward launch");
    }
    const bf_gemm_desc d[2] = {{gate.W, gate.W_aux, A, lda, gate_up, ldgu, M, F, K},
                               {up.W, up.W_aux, A, lda, gate_up + F, ldgu, M, F, K}};
    const bool two = fast && bf::lds_swiglu_supports(gs[2]);
    if (form == BF_FFN_TWO_LAUNCHES && !two)
        return fail(BF_ERR_UNSUPPORTED, "two-launch feed-forward block: batch 1-2 with the down projection's "
                                        "activations resident in LDS (M=%d F=%d)", M, F);
    const bool fused_down = two && form != BF_FFN_CALLS;
    // every launch of the block is planned, and the stream's workspace made
    // large enough for all of them, before the first is enqueued
    BatchedPlan bp;
    st = plan_batched(qtype, BF_OUT_F16, 2, d, bp);
    if (st != BF_OK) return st;
    bf::WsNeed need = batched_ws_need(bp);
    std::vector<Planned> down_l;
    if (!fused_down) {
        st = plan_gemm(qtype, down.W, down.W_aux, gate_up, ldgu, C, ldc, otype, M, N, F, BF_ALGO_AUTO, down_l);
        if (st != BF_OK) return st;
        for (const Planned& l : down_l) need.merge(ws_need(l));
    }
    st = from_split(bf::reserve_workspace(hs, need), "bf_ffn_swiglu");
    if (st != BF_OK) return st;
    st = launch_batched(bp, nullptr, hs);
    if (st != BF_OK) return st;
    if (fused_down) return from_hip(bf::gemm_lds_swiglu(gs[2], hs), "kernel launch");
    // SiLU(gate) * up in place over the gate half, then the down GEMM
    st = from_hip(bf::swiglu_f16(gate_up, ldgu, gate_up, ldgu, M, F, hs), "kernel launch");
    if (st != BF_OK) return st;
    for (const Planned& l : down_l) {
        st = launch_planned(l, nullptr, hs);
        if (st != BF_OK) return st;
    }
    return BF_OK;
}

bf_status bf_ffn_swiglu(bf_qtype qtype, bf_qweights gate, bf_qweights up, bf_qweights down, const uint16_t* A,
                        int lda, uint16_t* gate_up, int ldgu, void* C, int ldc, bf_otype otype, int M, int K, int F,
                        int N, void* stream) {
    return bf_ffn_swiglu_ex(qtype, gate, up, down, A, lda, gate_up, ldgu, C, ldc, otype, M, K, F, N, BF_FFN_AUTO,
                            stream);
}

bf_status bf_swiglu_f16(const uint16_t* gate_up, int ld, uint16_t* out, int ldo, int M, int K, void* stream) {
    g_last_error[0] = '\0';
    if (!gate_up || !out) return fail(BF_ERR_INVALID, "gate_up or out is NULL");
    if (M < 1 || K < 8 || K % 8) return fail(BF_ERR_INVALID, "M=%d must be >= 1 and K=%d a multiple of 8", M, K);
    if (ld < 2 * (int64_t)K || ldo < K) return fail(BF_ERR_INVALID, "ld=%d < 2K or ldo=%d < K=%d", ld, ldo, K);
    if (!aligned(gate_up, 16) || !aligned(out, 16) || ld % 8 || ldo % 8)
        return fail(BF_ERR_INVALID, "gate_up and out rows must be 16-byte aligned");
    return from_hip(bf::swiglu_f16(gate_up, ld, out, ldo, M, K, (hipStream_t)stream), "kernel launch");
}

size_t bf_q8_bytes(int M, int K) { return M < 1 || K < 32 || K % 32 ? 0 : bf::q8_bytes(M, K); }

bf_status bf_quantize_q8(const uint16_t* A, int lda, void* Aq, int M, int K, void* stream) {
    g_last_error[0] = '\0';
    if (!A || !Aq) return fail(BF_ERR_INVALID, "A or Aq is NULL");
    if (M < 1 || K < 32 || K % 32) return fail(BF_ERR_INVALID, "M=%d must be >= 1 and K=%d a multiple of 32", M, K);
    if (lda < K) return fail(BF_ERR_INVALID, "lda=%d < K=%d", lda, K);
    if (!aligned(A, 16) || lda % 8 || !aligned(Aq, 16))
        return fail(BF_ERR_INVALID, "A rows and Aq must be 16-byte aligned (lda %% 8 == 0)");
    return from_hip(bf::quantize_q8(A, lda, Aq, M, K, (hipStream_t)stream), "kernel launch");
}

bf_status bf_gemm_q8(bf_qtype qtype, const void* W, const void* W_aux, const void* Aq, void* C, int ldc,
                     bf_otype otype, int M, int N, int K, void* stream) {
    g_last_error[0] = '\0';
    bf_status st = check_weights(qtype, W, W_aux, N, K);
    if (st != BF_OK) return st;
    if (!Aq || !C) return fail(BF_ERR_INVALID, "Aq or C is NULL");
    if (otype != BF_OUT_F32 && otype != BF_OUT_F16) return fail(BF_ERR_INVALID, "unknown otype %d", (int)otype);
    if (M < 1) return fail(BF_ERR_INVALID, "M=%d must be >= 1", M);
    if (ldc < N) return fail(BF_ERR_INVALID, "ldc=%d < N=%d", ldc, N);
    if (!aligned(C, otype == BF_OUT_F32 ? 4 : 2)) return fail(BF_ERR_INVALID, "C is not aligned to its element");
    if (!aligned(Aq, 16) || !aligned(W, 16) || (W_aux && !aligned(W_aux, 4)))
        return fail(BF_ERR_INVALID, "Aq and W must be 16-byte aligned, W_aux 4-byte aligned");
    if (!bf::q8_supports(M, K))
        return fail(BF_ERR_UNSUPPORTED, "integer-dot GEMM: batch 1-16 and K %% 64 == 0 (M=%d K=%d)", M, K);
    bf::Q8Args g;
    g.qtype = (int)qtype;
    g.W = (const uint8_t*)W;
    g.Waux = (const uint8_t*)W_aux;
    g.Aq = Aq;
    g.C = C;
    g.ldc = ldc;
    g.out_f16 = otype == BF_OUT_F16;
    g.M = M;
    g.N = N;
    g.K = K;
    return from_hip(bf::gemm_q8(g, (hipStream_t)stream), "kernel launch");
}

bf_status bf_busfill_q4(const uint16_t* A, const uint8_t* Wq, const uint16_t* Ws, float* C, int Bsz, int K, int N,
                        void* stream) {
    return run_gemm(BF_Q4_0_PLANES, Wq, Ws, A, K, C, N, BF_OUT_F32, Bsz, N, K, BF_ALGO_AUTO, stream);
}

bf_status bf_dequant_f16(bf_qtype qtype, const void* W, const void* W_aux, uint16_t* W_f16, int N, int K,
                         void* stream) {
    g_last_error[0] = '\0';
    bf_status st = check_weights(qtype, W, W_aux, N, K);
    if (st != BF_OK) return st;
    if (!W_f16) return fail(BF_ERR_INVALID, "W_f16 is NULL");
    if (!aligned(W_f16, 2)) return fail(BF_ERR_INVALID, "W_f16 is not 2-byte aligned");
    return from_hip(bf::dequant_f16((int)qtype, (const uint8_t*)W, (const uint8_t*)W_aux, W_f16, N, K,
                                    (hipStream_t)stream),
                    "dequant launch");
}


bf_status bf_ggml_mul_mat(const bf_ggml_tensor* src0, const bf_ggml_tensor* src1, const bf_ggml_tensor* dst,
                          void* stream) {
    g_last_error[0] = '\0';
    GgmlCall c;
    bf_status st = check_ggml(src0, src1, dst, c);
    if (st != BF_OK) return st;
    hipStream_t hs = (hipStream_t)stream;
    if (c.fused) return from_hip(bf::gemm_lds(c.fg, hs), "ggml mul_mat: kernel launch");
    const auto held = stream_lock(stream);
    uint16_t* staged = nullptr;
    if (c.stage) {
        const hipError_t e = bf::staging_buffer(hs, c.stage_bytes, &staged);
        if (e == hipErrorStreamCaptureUnsupported)
            return fail(BF_ERR_UNSUPPORTED, "ggml mul_mat: the staging buffer for this stream is allocated on first "
                                            "use, which cannot happen during stream capture; make one uncaptured call "
                                            "of this size (or a larger one) on the stream first");
        st = from_hip(e, "ggml mul_mat: staging buffer");
        if (st != BF_OK) return st;
    }
    BatchedPlan bp;
    st = plan_ggml(c, src0, src1, dst, staged, bp);
    if (st != BF_OK) return st;
    st = from_split(bf::reserve_workspace(hs, batched_ws_need(bp)), "bf_ggml_mul_mat");
    if (st != BF_OK) return st;
    return enqueue_ggml(c, src1, staged, bp, nullptr, hs);
}

size_t bf_ggml_mul_mat_workspace_bytes(const bf_ggml_tensor* src0, const bf_ggml_tensor* src1,
                                       const bf_ggml_tensor* dst) {
    g_last_error[0] = '\0';
    GgmlCall c;
    BatchedPlan bp;
    if (check_ggml(src0, src1, dst, c) != BF_OK || c.fused ||
        plan_ggml(c, src0, src1, dst, kStagePlaceholder, bp) != BF_OK)
        return 0;
    const size_t need = batched_scratch_need(bp);
    return need || c.stage_bytes ? align256(need) + c.stage_bytes : 0;
}

bf_status bf_ggml_mul_mat_ws(const bf_ggml_tensor* src0, const bf_ggml_tensor* src1, const bf_ggml_tensor* dst,
                             void* workspace, size_t workspace_bytes, void* stream) {
    g_last_error[0] = '\0';
    bf_status st = check_workspace(workspace, workspace_bytes);
    if (st != BF_OK) return st;
    GgmlCall c;
    st = check_ggml(src0, src1, dst, c);
    if (st != BF_OK) return st;
    if (c.fused) return from_hip(bf::gemm_lds(c.fg, (hipStream_t)stream), "ggml mul_mat: kernel launch");
    // the GEMMs' workspace first, the staging buffer behind it
    BatchedPlan probe;
    st = plan_ggml(c, src0, src1, dst, kStagePlaceholder, probe);
    if (st != BF_OK) return st;
    const size_t need = align256(batched_scratch_need(probe));
    if (need + c.stage_bytes > workspace_bytes)
        return fail(BF_ERR_INVALID, "bf_ggml_mul_mat_ws: the call needs %zu bytes of workspace, %zu given",
                    need + c.stage_bytes, workspace_bytes);
    uint16_t* staged = c.stage ? (uint16_t*)((uint8_t*)workspace + need) : nullptr;
    BatchedPlan bp;
    st = plan_ggml(c, src0, src1, dst, staged, bp);
    if (st != BF_OK) return st;
    const bf::Scratch sc{(uint8_t*)workspace, need};
    const auto held = stream_lock(stream);
    return enqueue_ggml(c, src1, staged, bp, need ? &sc : nullptr, (hipStream_t)stream);
}

const char* bf_status_str(bf_status s) {
    switch (s) {
        case BF_OK: return "BF_OK";
        case BF_ERR_INVALID: return "BF_ERR_INVALID";
        case BF_ERR_UNSUPPORTED: return "BF_ERR_UNSUPPORTED";
        case BF_ERR_HIP: return "BF_ERR_HIP";
    }
    return "BF_UNKNOWN_STATUS";
}

const char* bf_last_error(void) { return g_last_error; }

}  // extern "C"

namespace bf {
void set_last_error(const char* text) { snprintf(g_last_error, sizeof g_last_error, "%s", text); }

bool copy_to_device(void* dst, const void* src, size_t n, void* stream) {
    hipStream_t st = (hipStream_t)stream;
    const hipError_t e = hipMemcpyAsync(dst, src, n, hipMemcpyHostToDevice, st);
    const hipError_t e2 = e == hipSuccess ? hipStreamSynchronize(st) : e;
    if (e2 == hipSuccess) return true;
    snprintf(g_last_error, sizeof g_last_error, "copy of %zu bytes to the device failed: %s", n, hipGetErrorString(e2));
    return false;
}
}  // namespace bf

extern "C" {

int bf_version(void) { return 100; }

}  // extern "C"
