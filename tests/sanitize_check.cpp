// Host-side checks of the C ABI's parsing and argument validation, built with AddressSanitizer and
// UndefinedBehaviorSanitizer (build.py: build_sanitize_check -> tests/_bin/sanitize_check) and run on
// the CPU by tests/test_sanitize.py.  No GPU is used: every call here returns before any device work
// (the GGUF reader is pure host code; the matmul entry points reject their arguments first).
//
//   sanitize_check <file.gguf> ...   prints "<rc> <tensors> <path>" per file after walking every
//                                    tensor and key the reader reports
//   sanitize_check abi               runs the argument-validation cases and prints "abi ok"
#include <cstdio>
#include <cstring>
#include <vector>

#include "qk.h"
#include "qk_gguf.h"

static int walk(const char* path) {
    qk_gguf* f = nullptr;
    const int rc = qk_gguf_open(path, &f);
    int64_t n = -1;
    if (rc == QK_OK) {
        qk_gguf_tensor_count(f, &n);
        for (int64_t i = 0; i < n; i++) {
            const char* name = nullptr;
            uint32_t type = 0;
            int32_t nd = 0;
            int64_t dims[4];
            uint64_t off = 0, nb = 0;
            if (qk_gguf_tensor_info(f, i, &name, &type, &nd, dims, &off, &nb) != QK_OK) return 90;
            int64_t idx = -1;
            if (qk_gguf_find(f, name, &idx) != QK_OK) return 91;
            volatile size_t len = strlen(name);  // the name is a valid C string
            (void)len;
            qk_weight w;
            (void)qk_gguf_weight(f, name, &w);  // not uploaded: QK_E_RANGE
        }
        double v = 0;
        const char* s = nullptr;
        (void)qk_gguf_kv_num(f, "general.alignment", &v);
        (void)qk_gguf_kv_str(f, "general.architecture", &s);
        (void)qk_gguf_tensor_info(f, n, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr);  // out of range
        qk_gguf_close(f);
    }
    printf("%d %lld %s\n", rc, (long long)n, path);
    return 0;
}

#define EXPECT(call, want)                                                          \
    do {                                                                            \
        const int got_ = (call);                                                    \
        if (got_ != (want)) {                                                       \
            fprintf(stderr, "%s:%d: %s = %d, want %d\n", __FILE__, __LINE__, #call, got_, want); \
            return 1;                                                               \
        }                                                                           \
    } while (0)

static int abi() {
    uint64_t rb = 0;
    EXPECT(qk_row_bytes(QK_T_Q4_K, 5120, &rb), QK_OK);
    EXPECT((int)rb, 2880);
    EXPECT(qk_row_bytes(QK_T_Q6_K, 300, &rb), QK_E_SHAPE);
    EXPECT(qk_row_bytes(99, 256, &rb), QK_E_TYPE);
    EXPECT(qk_row_bytes(QK_T_Q8_0, -256, &rb), QK_E_SHAPE);
    EXPECT(qk_row_bytes(QK_T_Q8_0, 256, nullptr), QK_E_NULL);
    alignas(16) static uint8_t fake[64];
    qk_weight w;
    EXPECT(qk_weight_view(fake, QK_T_Q4_K, 512, 32, QK_LAYOUT_T16, &w), QK_OK);
    EXPECT(qk_weight_view(fake + 4, QK_T_Q4_K, 512, 32, QK_LAYOUT_T16, &w), QK_E_ALIGN);
    EXPECT(qk_weight_view(fake, QK_T_Q4_K, 512, 30, QK_LAYOUT_T16, &w), QK_E_SHAPE);
    EXPECT(qk_weight_view(fake, QK_T_F32, 512, 32, QK_LAYOUT_T16, &w), QK_E_LAYOUT);
    EXPECT(qk_weight_view(nullptr, QK_T_Q4_K, 512, 32, QK_LAYOUT_T16, &w), QK_E_NULL);
    EXPECT(qk_weight_view(fake, QK_T_Q4_K, 512, 32, 7, &w), QK_E_LAYOUT);
    EXPECT(qk_weight_view(fake, QK_T_Q4_K, 512, 32, QK_LAYOUT_T16, &w), QK_OK);
    alignas(16) static float x[16 * 1024], y[16 * 1024];
    const qk_weight* ws[2] = {&w, &w};
    float* ys[2] = {y, y};
    void* vys[2] = {y, y};
    EXPECT(qk_matmul(&w, nullptr, 1, y, nullptr), QK_E_NULL);
    EXPECT(qk_matmul(&w, x, 0, y, nullptr), QK_E_SHAPE);
    EXPECT(qk_matmul(&w, x + 1, 1, y, nullptr), QK_E_ALIGN);
    EXPECT(qk_matmul_act(&w, x, 9, 1, y, nullptr), QK_E_RANGE);
    EXPECT(qk_matmul_act(&w, x, QK_ACT_F16_XPERM, 1, y, nullptr), QK_E_SHAPE);  // k = 512: not a multiple of 1024
    EXPECT(qk_matmul_noalloc(&w, x, 1, nullptr, nullptr), QK_E_NULL);
    EXPECT(qk_gemv_group(ws, ys, 0, 0, x, 1, nullptr), QK_E_GROUP);
    EXPECT(qk_gemv_group(ws, ys, 5, 0, x, 1, nullptr), QK_E_GROUP);
    EXPECT(qk_gemv_group(ws, ys, 1, 1, x, 1, nullptr), QK_E_GROUP);
    EXPECT(qk_gemv_group(ws, ys, 1, 0, x, 16, nullptr), QK_E_SHAPE);
    EXPECT(qk_gemv_group_act(ws, vys, 1, 0, x, QK_ACT_F16, QK_ACT_F16, 1, nullptr), QK_E_RANGE);
    EXPECT(qk_gemv_group_act(ws, vys, 2, 1, x, QK_ACT_F16, QK_ACT_F16_XPERM, 1, nullptr), QK_E_SHAPE);
    qk_gemv_plan_info info;
    EXPECT(qk_gemv_plan(ws, 1, 0, 1, nullptr), QK_E_NULL);
    EXPECT(qk_gemv_plan(ws, 1, 0, 0, &info), QK_E_SHAPE);
    EXPECT(qk_embed(&w, nullptr, nullptr, nullptr, 1, y, nullptr), QK_E_NULL);
    EXPECT(qk_embed(&w, (const int32_t*)x, (const uint8_t*)x, nullptr, 1, y, nullptr), QK_E_NULL);
    EXPECT(qk_set_tuning("nope", 1), QK_E_RANGE);
    EXPECT(qk_set_tuning(nullptr, 1), QK_E_NULL);
    EXPECT(qk_set_tuning("gemv_wpg", 3), QK_E_RANGE);
    qk_gguf* f = nullptr;
    EXPECT(qk_gguf_open(nullptr, &f), QK_E_NULL);
    EXPECT(qk_gguf_open("/nonexistent/file.gguf", &f), QK_E_IO);
    printf("abi ok\n");
    return 0;
}

int main(int argc, char** argv) {
    if (argc > 1 && !strcmp(argv[1], "abi")) return abi();
    for (int i = 1; i < argc; i++) {
        const int rc = walk(argv[i]);
        if (rc) return rc;
    }
    return 0;
}
