// Test driver for the reference-shaped C++ shim (include/qk_shim.h), run by tests/test_gpu_shim.py.
//   shim_check <w.bin> <type> <k> <n> <x.bin> <T> <y.bin> [glu_up.bin]
// uploads the GGUF bytes in w.bin, runs qkshim::matmul (or qkshim::gemv with glu when a second
// weight file is given) on x (fp32 [T][k]) and writes y (fp32) to y.bin.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <vector>

#include "qk_shim.h"

static std::vector<char> slurp(const char* path) {
    FILE* f = fopen(path, "rb");
    if (!f) {
        fprintf(stderr, "cannot open %s\n", path);
        exit(2);
    }
    std::vector<char> b;
    char buf[1 << 16];
    size_t got;
    while ((got = fread(buf, 1, sizeof buf, f)) > 0) b.insert(b.end(), buf, buf + got);
    fclose(f);
    return b;
}

int main(int argc, char** argv) {
    if (argc < 8) {
        fprintf(stderr, "usage: shim_check w.bin type k n x.bin T y.bin [up.bin]\n");
        return 2;
    }
    const uint32_t type = (uint32_t)atoi(argv[2]);
    const int k = atoi(argv[3]), n = atoi(argv[4]), T = atoi(argv[6]);
    const bool glu = argc > 8;
    std::vector<char> w = slurp(argv[1]), x = slurp(argv[5]);
    qkshim::use(nullptr);
    qkshim::Weight W = qkshim::upload(w.data(), type, k, n);
    void *xd = nullptr, *yd = nullptr;
    if (hipMalloc(&xd, x.size()) != hipSuccess || hipMalloc(&yd, (size_t)T * n * 4) != hipSuccess) return 3;
    if (hipMemcpy(xd, x.data(), x.size(), hipMemcpyHostToDevice) != hipSuccess) return 3;
    if (glu) {
        std::vector<char> u = slurp(argv[8]);
        qkshim::Weight U = qkshim::upload(u.data(), type, k, n);
        const qkshim::Weight* ws[2] = {&W, &U};
        qkshim::DevPtr ys[2] = {yd, nullptr};
        qkshim::gemv(ws, ys, 2, true, xd, T);
    } else {
        qkshim::matmul(W, xd, T, yd);
    }
    std::vector<float> y((size_t)T * n);
    if (hipMemcpy(y.data(), yd, y.size() * 4, hipMemcpyDeviceToHost) != hipSuccess) return 3;
    FILE* f = fopen(argv[7], "wb");
    if (!f || fwrite(y.data(), 4, y.size(), f) != y.size()) return 4;
    fclose(f);
    printf("ok\n");
    return 0;
}
