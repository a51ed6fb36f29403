// Test driver for the reference-shaped C++ shim (include/qk_shim.h), run by tests/test_gpu_shim.py.
//
//   shim_check <mode> <w.bin> <type> <k> <n> <x.bin> <T> <y.bin> [up.bin]
//     mode f32:  qkshim::matmul_f32 (or gemv_f32 with glu when up.bin is given), x fp32 [T][k], y fp32
//     mode f16:  qkshim::matmul / gemv with set_xperm(false), x fp16 [T][k]; y fp32, a GLU output fp16
//     mode f16x: the same with set_xperm(true): x (and a GLU output) in the xperm layout when T < 16
//   shim_check gguf <file.gguf> <tensor> <k> <n> <x.bin> <T> <y.bin>
//     load_weights + get_w + matmul_f32 (fp32 x)
//   shim_check embed <file.gguf> <tensor> <k> <n> <tokens.bin> <T> <x.bin> [mask.bin embd.bin]
//     load_weights + get_w + embed: tokens int32 [T], mask uint8 [T], embd fp32 [T][k]; x fp32 [T][k]
// Writes the output to the last path and prints "ok".
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <cstring>
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

static void* to_dev(const std::vector<char>& h) {
    void* d = nullptr;
    if (hipMalloc(&d, h.size() ? h.size() : 16) != hipSuccess) exit(3);
    if (!h.empty() && hipMemcpy(d, h.data(), h.size(), hipMemcpyHostToDevice) != hipSuccess) exit(3);
    return d;
}

static int write_out(const char* path, void* dev, size_t bytes) {
    std::vector<char> y(bytes);
    if (hipMemcpy(y.data(), dev, bytes, hipMemcpyDeviceToHost) != hipSuccess) return 3;
    FILE* f = fopen(path, "wb");
    if (!f || fwrite(y.data(), 1, y.size(), f) != y.size()) return 4;
    fclose(f);
    printf("ok\n");
    return 0;
}

int main(int argc, char** argv) {
    if (argc < 9) {
        fprintf(stderr, "usage: shim_check mode w.bin|file.gguf type|tensor k n x.bin T y.bin [...]\n");
        return 2;
    }
    const char* mode = argv[1];
    const int k = atoi(argv[4]), n = atoi(argv[5]), T = atoi(argv[7]);
    qkshim::use(nullptr);
    if (!strcmp(mode, "gguf") || !strcmp(mode, "embed")) {
        qkshim::load_weights(argv[2]);
        const qkshim::Weight W = qkshim::get_w(argv[3], k, n);
        std::vector<char> in = slurp(argv[6]);
        void* ind = to_dev(in);
        void* out = nullptr;
        if (hipMalloc(&out, (size_t)T * (!strcmp(mode, "gguf") ? n : k) * 4) != hipSuccess) return 3;
        if (!strcmp(mode, "gguf")) {
            qkshim::matmul_f32(W, ind, T, out);
            return write_out(argv[8], out, (size_t)T * n * 4);
        }
        void *maskd = nullptr, *embdd = nullptr;
        if (argc > 10) {
            maskd = to_dev(slurp(argv[9]));
            embdd = to_dev(slurp(argv[10]));
        }
        qkshim::embed(W, ind, maskd, embdd, out, T);
        return write_out(argv[8], out, (size_t)T * k * 4);
    }
    const uint32_t type = (uint32_t)atoi(argv[3]);
    const bool glu = argc > 9, f32 = !strcmp(mode, "f32");
    qkshim::set_xperm(!strcmp(mode, "f16x"));
    std::vector<char> w = slurp(argv[2]), x = slurp(argv[6]);
    qkshim::Weight W = qkshim::upload(w.data(), type, k, n);
    void* xd = to_dev(x);
    const size_t ybytes = (size_t)T * n * (glu && !f32 ? 2 : 4);
    void* yd = nullptr;
    if (hipMalloc(&yd, ybytes) != hipSuccess) return 3;
    if (glu) {
        std::vector<char> u = slurp(argv[9]);
        qkshim::Weight U = qkshim::upload(u.data(), type, k, n);
        const qkshim::Weight* ws[2] = {&W, &U};
        qkshim::DevPtr ys[2] = {yd, nullptr};
        if (f32) qkshim::gemv_f32(ws, ys, 2, true, xd, T);
        else qkshim::gemv(ws, ys, 2, true, xd, T);
    } else {
        if (f32) qkshim::matmul_f32(W, xd, T, yd);
        else qkshim::matmul(W, xd, T, yd);
    }
    return write_out(argv[8], yd, ybytes);
}
