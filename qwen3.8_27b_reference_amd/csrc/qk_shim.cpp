// Reference-shaped C++ entry points (include/qk_shim.h) over the C ABI: translate the POD weight,
// call qk_*, and turn any failure into the reference's print-and-_Exit(1) (qwen_cuda/cu.h:21-27).
#include "../../include/qk_shim.h"

#include <cstdio>
#include <cstdlib>
#include <unistd.h>

#include "../../include/qk_gguf.h"

namespace qkshim {
namespace {

thread_local qk_stream_t t_stream = nullptr;
bool g_xperm = false;         // qwen_cuda/qwen.cpp:82
qk_gguf* g_file = nullptr;    // the uploaded weight file (qwen_cuda/qwen.cpp:65 G_dbase, G_file)

void check(int rc, const char* where) {
    if (rc == QK_OK) return;
    fprintf(stderr, "qk: %s failed: %s (%d)\n", where, qk_status_string(rc), rc);
    _Exit(1);
}

qk_weight view(const Weight& w) {
    qk_weight v;
    v.data = w.data;
    v.type = w.type;
    v.k = w.k;
    v.n = w.n;
    v.rb = w.rb;
    v.layout = w.layout;
    return v;
}

Weight from_view(const qk_weight& v) {
    Weight w;
    w.data = const_cast<void*>(v.data);
    w.type = v.type;
    w.k = v.k;
    w.n = v.n;
    w.rb = v.rb;
    w.layout = v.layout;
    return w;
}

void group(const Weight* const* ws, const DevPtr* ys, int cnt, bool glu, DevPtr x, int T, uint32_t xfmt,
           uint32_t yfmt, const char* where) {
    if (cnt < 1 || cnt > 4) check(QK_E_GROUP, where);
    qk_weight v[4];
    const qk_weight* vp[4];
    void* y[4];
    for (int i = 0; i < cnt; i++) {
        v[i] = view(*ws[i]);
        vp[i] = &v[i];
        y[i] = glu ? ys[0] : ys[i];
    }
    check(qk_gemv_group_act(vp, y, cnt, glu ? 1 : 0, x, xfmt, glu ? yfmt : QK_ACT_F32, T, t_stream), where);
}

}  // namespace

void use(qk_stream_t stream) {
    check(qk_init_stream(stream), "use");
    t_stream = stream;
}

void set_xperm(bool on) { g_xperm = on; }

void load_weights(const char* gguf_path) {
    if (g_file) {
        fprintf(stderr, "qk: load_weights: a weight file is already loaded\n");
        _Exit(1);
    }
    qk_gguf* f = nullptr;
    check(qk_gguf_open(gguf_path, &f), "load_weights (open)");
    check(qk_gguf_upload(f, t_stream), "load_weights (upload)");
    g_file = f;
}

Weight get_w(const std::string& name, int k, int n) {
    if (!g_file) {
        fprintf(stderr, "qk: get_w(%s): no weight file loaded\n", name.c_str());
        _Exit(1);
    }
    int64_t idx = 0;
    if (qk_gguf_find(g_file, name.c_str(), &idx) != QK_OK) {
        fprintf(stderr, "qk: get_w: no tensor %s\n", name.c_str());
        _Exit(1);
    }
    const char* nm = nullptr;
    uint32_t type = 0;
    int32_t nd = 0;
    int64_t dims[4] = {0, 0, 0, 0};
    uint64_t off = 0, nbytes = 0;
    check(qk_gguf_tensor_info(g_file, idx, &nm, &type, &nd, dims, &off, &nbytes), "get_w");
    if (nd != 2 || dims[0] != k || dims[1] != n) {
        fprintf(stderr, "qk: get_w: %s has the wrong shape, expected [%d, %d]\n", name.c_str(), k, n);
        _Exit(1);
    }
    qk_weight v;
    check(qk_gguf_weight(g_file, name.c_str(), &v), "get_w");  // rejects types without kernels
    return from_view(v);
}

Weight upload(const void* host_gguf_bytes, uint32_t type, int k, int n) {
    qk_weight v;
    check(qk_upload(host_gguf_bytes, type, k, n, QK_LAYOUT_T16, t_stream, &v), "upload");
    return from_view(v);
}

void gemv(const Weight* const* ws, const DevPtr* ys, int cnt, bool glu, DevPtr x, int T) {
    const bool xp = T < 16 && g_xperm;  // qwen_cuda/qwen.cpp:234
    const uint32_t f = xp ? QK_ACT_F16_XPERM : QK_ACT_F16;
    group(ws, ys, cnt, glu, x, T, f, f, "gemv");
}

void matmul(const Weight& w, DevPtr x, int T, DevPtr y) {
    // qwen_cuda/qwen.cpp:240-247: fp16 x, in the xperm layout for T < 16 when the step runs it (the
    // reference then takes its GEMV); qk_matmul_act keeps T <= 4 on the GEMV and reads the weights
    // once on the GEMM from five tokens
    const qk_weight v = view(w);
    const uint32_t f = T < 16 && g_xperm ? QK_ACT_F16_XPERM : QK_ACT_F16;
    check(qk_matmul_act(&v, x, f, T, (float*)y, t_stream), "matmul");
}

void embed(const Weight& table, DevPtr tokens, DevPtr mask, DevPtr embd, DevPtr x, int T) {
    const qk_weight v = view(table);
    check(qk_embed(&v, (const int32_t*)tokens, (const uint8_t*)mask, (const float*)embd, T, (float*)x, t_stream),
          "embed");
}

void gemv_f32(const Weight* const* ws, const DevPtr* ys, int cnt, bool glu, DevPtr x, int T) {
    group(ws, ys, cnt, glu, x, T, QK_ACT_F32, QK_ACT_F32, "gemv_f32");
}

void matmul_f32(const Weight& w, DevPtr x, int T, DevPtr y) {
    const qk_weight v = view(w);
    check(qk_matmul(&v, (const float*)x, T, (float*)y, t_stream), "matmul_f32");
}

}  // namespace qkshim
