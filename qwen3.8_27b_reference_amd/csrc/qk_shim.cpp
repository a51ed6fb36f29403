// Reference-shaped C++ entry points (include/qk_shim.h) over the C ABI: translate the POD weight,
// call qk_*, and turn any failure into the reference's print-and-_Exit(1) (qwen_cuda/cu.h:21-27).
#include "../../include/qk_shim.h"

#include <cstdio>
#include <cstdlib>
#include <unistd.h>

namespace qkshim {
namespace {

thread_local qk_stream_t t_stream = nullptr;

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

}  // namespace

void use(qk_stream_t stream) {
    check(qk_init_stream(stream), "use");
    t_stream = stream;
}

Weight upload(const void* host_gguf_bytes, uint32_t type, int k, int n) {
    qk_weight v;
    check(qk_upload(host_gguf_bytes, type, k, n, QK_LAYOUT_T16, t_stream, &v), "upload");
    Weight w;
    w.data = const_cast<void*>(v.data);
    w.type = v.type;
    w.k = v.k;
    w.n = v.n;
    w.rb = v.rb;
    w.layout = v.layout;
    return w;
}

void gemv(const Weight* const* ws, const DevPtr* ys, int cnt, bool glu, DevPtr x, int T) {
    if (cnt < 1 || cnt > 4) check(QK_E_GROUP, "gemv");
    qk_weight v[4];
    const qk_weight* vp[4];
    float* y[4];
    for (int i = 0; i < cnt; i++) {
        v[i] = view(*ws[i]);
        vp[i] = &v[i];
        y[i] = (float*)(glu ? ys[0] : ys[i]);
    }
    check(qk_gemv_group(vp, y, cnt, glu ? 1 : 0, (const float*)x, T, t_stream), "gemv");
}

void matmul(const Weight& w, DevPtr x, int T, DevPtr y) {
    const qk_weight v = view(w);
    check(qk_matmul(&v, (const float*)x, T, (float*)y, t_stream), "matmul");
}

}  // namespace qkshim
