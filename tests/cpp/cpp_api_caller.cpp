// cpp_api_caller.cpp -- a C++ caller of include/megakernel.h, written the way
// the reference's own C++ harnesses drive its header (test/check.cu:204-205,
// test/mybench.cu:222-237): caller-owned buffers, fp8mega::layout for the
// workspace, fill_weights_lane for the weights, one launch_full on a stream,
// then the status words.  Raw (unscaled) e4m3 path.
//
// Usage: cpp_api_caller DIR
//   DIR/dims.txt  "E K H I T SEED1 SEED2"
//   DIR/x.bin     uint8  [T][H]   fp8 e4m3 activations
//   DIR/idx.bin   int64  [T][K]   expert ids
//   DIR/wts.bin   float  [T][K]   top-k weights
// Writes DIR/y.bin (float [T][H]) and prints "ok items=... slots=...".
#include <cstdio>
#include <cstdlib>
#include <string>
#include <vector>

#include <hip/hip_runtime.h>

#include "megakernel.h"

#define CHECK_HIP(x)                                                                 \
    do {                                                                             \
        hipError_t e_ = (x);                                                         \
        if (e_ != hipSuccess) {                                                      \
            std::fprintf(stderr, "%s: %s\n", #x, hipGetErrorString(e_));             \
            return 2;                                                                \
        }                                                                            \
    } while (0)

static bool read_file(const std::string& path, void* dst, size_t bytes) {
    FILE* f = std::fopen(path.c_str(), "rb");
    if (!f) return false;
    const size_t n = std::fread(dst, 1, bytes, f);
    std::fclose(f);
    return n == bytes;
}

int main(int argc, char** argv) {
    if (argc != 2) {
        std::fprintf(stderr, "usage: %s DIR\n", argv[0]);
        return 2;
    }
    const std::string dir = argv[1];
    int E, K, H, I, T;
    unsigned s1, s2;
    FILE* f = std::fopen((dir + "/dims.txt").c_str(), "r");
    if (!f || std::fscanf(f, "%d %d %d %d %d %u %u", &E, &K, &H, &I, &T, &s1, &s2) != 7) {
        std::fprintf(stderr, "bad dims.txt\n");
        return 2;
    }
    std::fclose(f);
    std::vector<uint8_t> x((size_t)T * H);
    std::vector<int64_t> idx((size_t)T * K);
    std::vector<float> wts((size_t)T * K);
    if (!read_file(dir + "/x.bin", x.data(), x.size()) ||
        !read_file(dir + "/idx.bin", idx.data(), idx.size() * 8) ||
        !read_file(dir + "/wts.bin", wts.data(), wts.size() * 4)) {
        std::fprintf(stderr, "missing inputs\n");
        return 2;
    }
    hipStream_t s;
    CHECK_HIP(hipStreamCreate(&s));
    // weights: the reference's deterministic generator over all experts'
    // logical rows (expert e's W1 rows are e*2I .. e*2I + 2I - 1)
    uint8_t *w1, *w2;
    CHECK_HIP(hipMalloc(&w1, (size_t)E * 2 * I * H));
    CHECK_HIP(hipMalloc(&w2, (size_t)E * H * I));
    fp8mega::fill_weights_lane(w1, E * 2 * I, H, s1, s);
    fp8mega::fill_weights_lane(w2, E * H, I, s2, s);
    if (fp8mega::last_error() != fp8mega::kOk) return 3;
    // x and the top-k weights live in one caller buffer ("self"), as in the
    // reference's symmetric buffer
    const int64_t x_off = 0, w_off = ((int64_t)T * H + 255) / 256 * 256;
    uint8_t* self;
    int64_t* d_idx;
    float *y;
    uint16_t* yb;
    CHECK_HIP(hipMalloc(&self, w_off + (size_t)T * K * 4));
    CHECK_HIP(hipMalloc(&d_idx, idx.size() * 8));
    CHECK_HIP(hipMalloc(&y, (size_t)T * H * 4));
    CHECK_HIP(hipMalloc(&yb, (size_t)T * H * 2));
    CHECK_HIP(hipMemcpy(self + x_off, x.data(), x.size(), hipMemcpyHostToDevice));
    CHECK_HIP(hipMemcpy(self + w_off, wts.data(), wts.size() * 4, hipMemcpyHostToDevice));
    CHECK_HIP(hipMemcpy(d_idx, idx.data(), idx.size() * 8, hipMemcpyHostToDevice));
    const fp8mega::MegaLayout L = fp8mega::layout(T, K, E, H, I, 0);
    if (L.total <= 0) return 4;
    void* ws;
    CHECK_HIP(hipMalloc(&ws, L.total));

    fp8mega::MegaLaunchArgs a{};
    a.tokens = T;
    a.max_tokens = T;
    a.rwk = static_cast<rwk_data*>(ws);
    a.workspace_bytes = L.total;
    a.self = self;
    a.x_off = x_off;
    a.weights_off = w_off;
    a.topk_idx = d_idx;
    a.w1 = w1;
    a.w2 = w2;
    a.y = y;
    a.y_bf16 = yb;
    a.num_experts = E;
    a.topk = K;
    a.hidden = H;
    a.intermediate = I;
    fp8mega::launch_full(a, s);
    if (fp8mega::last_error() != fp8mega::kOk) {
        std::fprintf(stderr, "launch_full: status %d\n", fp8mega::last_error());
        return 5;
    }
    int32_t st[5];
    const int rc = fp8mega::read_status(a, st, 5, s);
    if (rc != fp8mega::kOk) {
        std::fprintf(stderr, "read_status: %d (error bits %d)\n", rc, st[0]);
        return 6;
    }
    std::vector<float> out((size_t)T * H);
    CHECK_HIP(hipMemcpy(out.data(), y, out.size() * 4, hipMemcpyDeviceToHost));
    FILE* o = std::fopen((dir + "/y.bin").c_str(), "wb");
    if (!o || std::fwrite(out.data(), 4, out.size(), o) != out.size()) return 7;
    std::fclose(o);
    std::printf("ok items=%d slots=%d\n", st[1], st[2]);
    for (void* p : {(void*)w1, (void*)w2, (void*)self, (void*)d_idx, (void*)y, (void*)yb, ws})
        CHECK_HIP(hipFree(p));
    CHECK_HIP(hipStreamDestroy(s));
    return 0;
}
