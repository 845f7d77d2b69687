// Sanitizer build of the host code: the CPU oracle (oracle/oracle.c) and the
// GGUF reader (bus-fill_amd/csrc/bf_gguf.cpp), compiled with
// -fsanitize=address,undefined by tests/test_sanitize.py and driven here.
//   * The oracle: every format at small and ragged shapes, every entry point.
//   * The reader: each file named on the command line (valid, truncated or
//     corrupted) through every entry point; rejecting a file is fine, a
//     sanitizer report is not.
// bf_gguf_upload's device copy is replaced by a host memcpy into a host buffer
// (this build has no HIP), so its bounds checks run too.
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "busfill.h"
#include "bf_host.h"
#include "oracle.h"

namespace bf {
void set_last_error(const char*) {}
bool copy_to_device(void* dst, const void* src, size_t n, void*) {
    std::memcpy(dst, src, n);
    return true;
}
}  // namespace bf

namespace {

int check(int rc, const char* what) {
    if (rc != 0) {
        std::printf("oracle %s returned %d\n", what, rc);
        std::exit(1);
    }
    return rc;
}

void oracle_cases() {
    const int shapes[][2] = {{1, 256}, {3, 512}, {17, 1024}, {5, 256 * 3}};
    for (int qt = 0; qt < 3; qt++)
        for (const auto& sh : shapes) {
            const int N = sh[0], K = sh[1];
            std::vector<uint8_t> W((size_t)N * K * 9 / 16 + 16), Wq((size_t)N * K / 2);
            std::vector<uint16_t> Ws((size_t)N * K / 32);
            const void* aux = nullptr;
            if (qt == OR_Q4_0_PLANES) {
                or_gen_q4_0_planes(11, N, K, 0.002f, 0.02f, Wq.data(), Ws.data());
                aux = Ws.data();
            } else if (qt == OR_Q4_0) {
                or_gen_q4_0_blocks(11, N, K, 0.002f, 0.02f, W.data());
                or_q4_0_blocks_to_planes(W.data(), N, K, Wq.data(), Ws.data());
                or_q4_0_planes_to_blocks(Wq.data(), Ws.data(), N, K, W.data());
            } else {
                or_gen_q4_k(11, N, K, 0.001f, 0.01f, W.data());
            }
            const void* w = qt == OR_Q4_0_PLANES ? (const void*)Wq.data() : (const void*)W.data();
            std::vector<uint16_t> d16((size_t)N * K);
            std::vector<float> d32((size_t)N * K);
            check(or_dequant_f16(qt, w, aux, N, K, d16.data()), "dequant_f16");
            check(or_dequant_f32(qt, w, aux, N, K, d32.data()), "dequant_f32");
            for (int M : {1, 3}) {
                std::vector<uint16_t> A((size_t)M * K);
                or_gen_act(12, M, K, A.data());
                std::vector<double> C((size_t)M * N), C2((size_t)M * N);
                check(or_gemm_f64(qt, w, aux, A.data(), M, N, K, C.data(), 1), "gemm_f64");
                check(or_gemm_f64(qt, w, aux, A.data(), M, N, K, C2.data(), 2), "gemm_f64 threads");
                check(or_gemm_f16w_f64(qt, w, aux, A.data(), M, N, K, C2.data(), 0), "gemm_f16w_f64");
                std::vector<float> scratch((size_t)N * K), Cf((size_t)M * N);
                double tdq = 0, tmm = 0;
                check(or_cpu_dequant_matmul(qt, w, aux, A.data(), M, N, K, scratch.data(), Cf.data(), 2, &tdq, &tmm),
                      "cpu_dequant_matmul");
            }
            // invalid shapes are refused, not read
            if (or_dequant_f16(qt, w, aux, N, K + 16, d16.data()) == 0 && qt == OR_Q4_K) {
                std::printf("oracle accepted K %% 256 != 0 for Q4_K\n");
                std::exit(1);
            }
        }
    for (int j = 0; j < 8; j++) {
        uint8_t sc[8], m[8], packed[12], s1, m1;
        for (int i = 0; i < 8; i++) {
            sc[i] = (uint8_t)((7 * i + j) & 63);
            m[i] = (uint8_t)((13 * i + 3 * j) & 63);
        }
        or_q4k_pack_scales(sc, m, packed);
        or_q4k_get_scale_min(j, packed, &s1, &m1);
        if (s1 != sc[j] || m1 != m[j]) {
            std::printf("scale pack/unpack mismatch\n");
            std::exit(1);
        }
    }
    for (uint32_t h = 0; h < 65536; h += 7) (void)or_f32_to_f16(or_f16_to_f32((uint16_t)h));
}

int gguf_file(const char* path) {
    bf_gguf* g = nullptr;
    if (bf_gguf_open(path, &g) != BF_OK) return 0;          // rejected: fine
    const int64_t n = bf_gguf_tensor_count(g);
    int walked = 0;
    for (int64_t i = 0; i < n; i++) {
        bf_gguf_tensor t;
        if (bf_gguf_tensor_at(g, i, &t) != BF_OK) continue;
        bf_gguf_tensor t2;
        (void)bf_gguf_find(g, t.name, &t2);
        if (t.nbytes && t.nbytes < (64u << 20)) {
            std::vector<uint8_t> host(t.nbytes);
            (void)bf_gguf_upload(g, &t, host.data(), nullptr);
            volatile uint8_t sink = 0;
            for (uint64_t b = 0; b < t.nbytes; b += 61) sink = sink ^ ((const uint8_t*)t.data)[b];
        }
        walked++;
    }
    bf_gguf_tensor none;
    (void)bf_gguf_tensor_at(g, n, &none);
    (void)bf_gguf_find(g, "no.such.tensor", &none);
    for (const char* key : {"general.architecture", "general.alignment", "llama.block_count", "tokens", "ids",
                            "i8neg", "missing.key"}) {
        uint64_t v = 0, len = 0;
        const char* s = nullptr;
        (void)bf_gguf_get_u64(g, key, &v);
        if (bf_gguf_get_str(g, key, &s, &len) == BF_OK) {
            volatile char c = 0;
            for (uint64_t i = 0; i < len; i++) c = c ^ s[i];
        }
    }
    bf_gguf_close(g);
    return walked;
}

}  // namespace

int main(int argc, char** argv) {
    oracle_cases();
    int opened = 0;
    for (int i = 1; i < argc; i++) opened += gguf_file(argv[i]) > 0;
    std::printf("sanitized run ok: oracle cases, %d files, %d with tensors walked\n", argc - 1, opened);
    return 0;
}
