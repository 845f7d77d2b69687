// ggml mul_mat hook, device side: src1's rows rounded to fp16 into a
// contiguous staging buffer, and that buffer for the library's own calls.
// The hook itself (validation, slices, GEMMs) is in bf_api.hip.
//
// ggml_mul_mat reads src1 through its byte strides (a permuted or transposed
// view works as well as a contiguous one), so each element is fetched at
// i0 nb[0] + i1 nb[1] + i2 nb[2] + i3 nb[3]; rows whose elements are
// contiguous and 16-byte aligned take 16- or 32-byte loads.  fp32 -> fp16 is
// the conversion instruction's round to nearest even, the rounding of ggml's
// own fp32 -> fp16 copies (so the activations the GEMM sees are the ones a
// ggml fp16 path would see).
#include <map>
#include <mutex>
#include <thread>
#include <tuple>
#include <vector>

#include "bf_launch.h"

namespace bf {
namespace {

typedef float f4v __attribute__((ext_vector_type(4)));
typedef _Float16 h8v __attribute__((ext_vector_type(8)));

// Block r of the grid (stride gridDim.x) takes row r; thread t elements
// 8t .. 8t + 7 of it (stride 8 blockDim.x).  vec: the row's elements are
// contiguous and every row starts 16-byte aligned.
__global__ __launch_bounds__(256) void k_stage_f16(const uint8_t* __restrict__ src, int f32, int64_t ne0, int64_t ne1,
                                                   int64_t ne2, uint64_t nb0, uint64_t nb1, uint64_t nb2, uint64_t nb3,
                                                   int64_t rows, int vec, uint16_t* __restrict__ dst) {
    for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
        const int64_t i1 = r % ne1, i2 = (r / ne1) % ne2, i3 = r / (ne1 * ne2);
        const uint8_t* row = src + i1 * nb1 + i2 * nb2 + i3 * nb3;
        h8v* out = (h8v*)(dst + r * ne0);
        for (int64_t k = 8 * (int64_t)threadIdx.x; k < ne0; k += 8 * (int64_t)blockDim.x) {
            h8v h;
            if (vec && f32) {
                const f4v a = *(const f4v*)(row + 4 * k), b = *(const f4v*)(row + 4 * k + 16);
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    h[j] = (_Float16)a[j];
                    h[4 + j] = (_Float16)b[j];
                }
            } else if (vec) {
                h = *(const h8v*)(row + 2 * k);
            } else {
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    const uint8_t* e = row + (uint64_t)(k + j) * nb0;
                    h[j] = f32 ? (_Float16)*(const float*)e : *(const _Float16*)e;
                }
            }
            out[k / 8] = h;
        }
    }
}

}  // namespace

hipError_t stage_rows_f16(const void* src, int f32, const int64_t ne[4], const uint64_t nb[4], uint16_t* dst,
                          hipStream_t st) {
    const int64_t rows = ne[1] * ne[2] * ne[3];
    const uint64_t es = f32 ? 4 : 2;
    const bool vec = nb[0] == es && (((uintptr_t)src | nb[1] | nb[2] | nb[3]) & 15) == 0;
    const int grid = (int)std::min<int64_t>(rows, 4096);
    hipLaunchKernelGGL(k_stage_f16, dim3(grid), dim3(256), 0, st, (const uint8_t*)src, f32, ne[0], ne[1], ne[2],
                       nb[0], nb[1], nb[2], nb[3], rows, vec ? 1 : 0, dst);
    return hipGetLastError();
}

hipError_t staging_buffer(hipStream_t st, size_t bytes, uint16_t** out) {
    struct Buf {
        uint8_t* p = nullptr;
        size_t bytes = 0;
    };
    static std::mutex mu;
    static std::map<std::tuple<int, uintptr_t, std::thread::id>, Buf> cache;
    static std::vector<uint8_t*> retired;
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    const std::thread::id tid = st == hipStreamPerThread ? std::this_thread::get_id() : std::thread::id();
    std::lock_guard<std::mutex> lock(mu);
    Buf& b = cache[{dev, (uintptr_t)st, tid}];
    if (b.bytes < bytes) {
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        e = hipStreamIsCapturing(st, &cs);
        if (e != hipSuccess) return e;
        if (cs != hipStreamCaptureStatusNone) return hipErrorStreamCaptureUnsupported;
        const size_t nb = std::max(bytes, 2 * b.bytes);
        uint8_t* p = nullptr;
        e = hipMalloc((void**)&p, nb);
        if (e != hipSuccess) return e;
        // queued launches and captured graphs may still read the old buffer
        if (b.p) retired.push_back(b.p);
        b = Buf{p, nb};
    }
    *out = (uint16_t*)b.p;
    return hipSuccess;
}

}  // namespace bf
