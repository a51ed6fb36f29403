// C ABI (include/qk.h): argument validation, per-stream split-K workspaces and launch planning.
//
// Mirrors the reference's CUDA host glue (qwen_cuda/qwen.cpp:150-247): get_w's shape/type checks,
// gemv()'s grouping of matrices that share x, matmul()'s T<16 -> GEMV / GEMM dispatch and the
// upload + repack of qwen.cpp:756-761 / 185-193 — but every failure is a returned status instead of
// _Exit(1), so the checks are testable without a GPU.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <set>
#include <utility>

#include "../../include/qk.h"
#include "../../include/qk_synth.h"
#include "qk_internal.h"

namespace {

using qk::GemvParams;

constexpr size_t WS_PART_BYTES = 64ull << 20;  // split-K partials per stream
constexpr int WS_COUNTERS = 1 << 16;           // 16-row tiles per launch (arrival counters)
constexpr size_t WS_IMG_BYTES = 8ull << 20;    // activation image of x (k up to ~440k at m = 4)
constexpr size_t WS_GEMM_BYTES = 64ull << 20;  // fp16 activation image of a GEMM token chunk
constexpr size_t WS_XSLOTS = 4ull << 20;       // int8 GEMV combine slots (32 MiB), zero = empty
constexpr size_t WS_KPART_BYTES = 128ull << 20;  // GEMM split-K partials
// The reference runs m < 16 on its GEMV (qwen_cuda/qwen.cpp:240-247), with fp16 x, in the xperm
// layout when its forward sets G_xperm; xperm x is accepted for m < GEMM_MIN_M only, as there.
// From GEMM_ROUTE_M tokens qk_matmul(_act), a group's runs of one type and a gate/up pair take the
// GEMM instead, any activation format: the int8 GEMV carries eight tokens per launch (two weight
// passes from nine) and its eight-token form is compute-bound, while the GEMM in work-groups of one
// 32-token block reads the weights once.  Measured on MI355X (us per call, fp16 xperm x, GEMV
// against GEMM): at five tokens K=17408 N=5120 Q4_K 29.4 / 22.6, Q6_K 38.0 / 36.4, Q5_K 32.4 / 32.8;
// K=5120 N=17408 Q4_K 24.2 / 20.3; the output projection 487 / 257; the gate/up pair 46.4 / 32.4;
// at four tokens the GEMV wins (the pair 25.9 / 32.0).
constexpr int GEMM_MIN_M = 16;
constexpr int GEMM_ROUTE_M = 5;
std::atomic<int> g_gemm_min_m{0};  // tuning override of GEMM_ROUTE_M (2..16; 0 = the default)
int gemm_route_m() {
    const int v = g_gemm_min_m.load(std::memory_order_relaxed);
    return v ? v : GEMM_ROUTE_M;
}

using qk::Workspace;

std::mutex g_mu;
std::map<std::pair<int, hipStream_t>, Workspace> g_ws;
std::map<int, int> g_cu_count;
std::set<const void*> g_owned;  // allocations made by qk_upload

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

bool type_supported(uint32_t type) {
    return type == QK_T_F32 || type == QK_T_Q8_0 || type == QK_T_Q4_K || type == QK_T_Q5_K || type == QK_T_Q6_K;
}

int cu_count(int dev) {
    auto it = g_cu_count.find(dev);
    if (it != g_cu_count.end()) return it->second;
    hipDeviceProp_t prop;
    int n = 256;
    if (hipGetDeviceProperties(&prop, dev) == hipSuccess && prop.multiProcessorCount > 0) n = prop.multiProcessorCount;
    g_cu_count[dev] = n;
    return n;
}

// Returns the stream's workspace, creating it on first use (the only allocation of the matmul path).
int get_workspace(hipStream_t s, Workspace** out, int* ncu) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return QK_E_HIP;
    std::lock_guard<std::mutex> lock(g_mu);
    *ncu = cu_count(dev);
    auto key = std::make_pair(dev, s);
    auto it = g_ws.find(key);
    if (it == g_ws.end()) {
        Workspace w;
        void* p[6] = {};
        const size_t bytes[6] = {WS_PART_BYTES, WS_COUNTERS * sizeof(int), WS_IMG_BYTES, WS_GEMM_BYTES,
                                 WS_XSLOTS * sizeof(uint64_t), WS_KPART_BYTES};
        for (int i = 0; i < 6; i++) {
            if (hipMalloc(&p[i], bytes[i]) != hipSuccess) {
                for (int j = 0; j < i; j++) (void)hipFree(p[j]);
                return QK_E_HIP;
            }
        }
        w.part = (float*)p[0];
        w.part_bytes = WS_PART_BYTES;
        w.counters = (int*)p[1];
        w.ncounters = WS_COUNTERS;
        w.img = (uint8_t*)p[2];
        w.img_bytes = WS_IMG_BYTES;
        w.gimg = (uint8_t*)p[3];
        w.gimg_bytes = WS_GEMM_BYTES;
        w.xslot = (uint64_t*)p[4];
        w.nxslot = WS_XSLOTS;
        w.kpart = (float*)p[5];
        w.kpart_bytes = WS_KPART_BYTES;
        // counters start at zero and combine slots empty (zero), once; every launch leaves them so again
        if (hipMemset(w.counters, 0, WS_COUNTERS * sizeof(int)) != hipSuccess ||
            hipMemset(w.xslot, 0, WS_XSLOTS * sizeof(uint64_t)) != hipSuccess ||
            hipDeviceSynchronize() != hipSuccess) {
            for (int j = 0; j < 6; j++) (void)hipFree(p[j]);
            return QK_E_HIP;
        }
        it = g_ws.emplace(key, w).first;
    }
    *out = &it->second;
    return QK_OK;
}

int device_cus() { return qk::current_cus(); }

int check_weight(const qk_weight* w) {
    if (!w || !w->data) return QK_E_NULL;
    if (!type_supported(w->type)) return QK_E_TYPE;
    if (w->k <= 0 || w->k % 256 || w->n <= 0) return QK_E_SHAPE;
    uint64_t rb = 0;
    if (qk_row_bytes(w->type, w->k, &rb) != QK_OK || rb != w->rb) return QK_E_SHAPE;
    if (w->layout != QK_LAYOUT_GGUF && w->layout != QK_LAYOUT_T16) return QK_E_LAYOUT;
    if (w->type == QK_T_F32 && w->layout != QK_LAYOUT_GGUF) return QK_E_LAYOUT;  // used as stored
    if (w->layout == QK_LAYOUT_T16 && w->n % 16) return QK_E_SHAPE;
    if (!aligned16(w->data)) return QK_E_ALIGN;
    return QK_OK;
}

// Activations at the boundary: format (ACT_* = QK_ACT_*) and bytes per element.
struct Act {
    const void* p;
    int fmt;
    size_t esz() const { return fmt == QK_ACT_F32 ? 4 : 2; }
    Act at(size_t elems) const { return Act{p ? (const uint8_t*)p + elems * esz() : nullptr, fmt}; }
};
// Outputs: fp32 [m][n] (yfmt applies to a GLU pair's output only).
inline size_t out_esz(int yfmt) { return yfmt == QK_ACT_F32 ? 4 : 2; }
inline void* out_at(void* y, int yfmt, size_t elems) { return y ? (uint8_t*)y + elems * out_esz(yfmt) : nullptr; }

// Plans and launches one GEMV over `cnt` weights of one type for tokens [0, m) (m <= 8) in the
// workspace wsp (info != nullptr: plan only).  Five to eight tokens whose eight-slot plan does not
// fit the LDS run as four tokens and then the rest; two to four whose plan does not fit, token by
// token; a shape that has no plan even for one token is a shape error.
int run_gemv(const qk_weight* const* ws, void* const* ys, int cnt, bool glu, Act x, int yfmt, int m, int k,
             hipStream_t s, const Workspace* wsp, qk::GemvPlan* info) {
    GemvParams p;
    memset(&p, 0, sizeof(p));
    p.cnt = cnt;
    p.glu = glu ? 1 : 0;
    p.tile0[0] = 0;
    for (int i = 0; i < cnt; i++) {
        p.w[i] = (const uint8_t*)ws[i]->data;
        p.y[i] = ys[glu ? 0 : i];
        p.n[i] = ws[i]->n;
        p.tile0[i + 1] = p.tile0[i] + ws[i]->n / 16;
    }
    const int ntiles = glu ? p.tile0[1] : p.tile0[cnt];
    const int na = glu ? 2 : 1;
    if (ntiles > wsp->ncounters) return QK_E_RANGE;
    p.x = x.p;
    p.xfmt = x.fmt;
    p.yfmt = glu ? yfmt : QK_ACT_F32;
    p.ldx = k;
    p.k = k;
    p.nsb = k / 256;
    p.m = m;
    p.units = ntiles * p.nsb;
    p.waves = qk::gemv_plan_waves((int)ws[0]->type, na, m, p.units);
    if (p.waves < 1) return QK_E_RANGE;
    if (qk::gemv_part_floats(p.waves, na, m) * sizeof(float) > wsp->part_bytes) return QK_E_RANGE;
    if (qk::gemv_image_bytes((int)ws[0]->type, m, p.nsb) > wsp->img_bytes) return QK_E_RANGE;
    p.part = wsp->part;
    p.part_cap = wsp->part_bytes / sizeof(float);
    p.counters = wsp->counters;
    p.xslot = wsp->xslot;
    p.xslot_cap = wsp->nxslot;
    p.ximg = wsp->img;
    const int rc = qk::launch_gemv((int)ws[0]->type, p, s, info);
    if (rc == 1 && m > 4) {  // no eight-token plan: four tokens, then the rest
        void* yt[qk::GEMV_MAX_CNT];
        for (int i = 0; i < (glu ? 1 : cnt); i++) yt[i] = out_at(ys[i], glu ? yfmt : QK_ACT_F32, (size_t)4 * ws[i]->n);
        const int r = run_gemv(ws, ys, cnt, glu, x, yfmt, 4, k, s, wsp, info);
        if (r != QK_OK || info) return r;
        return run_gemv(ws, yt, cnt, glu, x.at((size_t)4 * k), yfmt, m - 4, k, s, wsp, info);
    }
    if (rc == 1 && m > 1) {  // no plan for m tokens at once: one launch per token
        for (int t = 0; t < m; t++) {
            void* yt[qk::GEMV_MAX_CNT];
            for (int i = 0; i < (glu ? 1 : cnt); i++)
                yt[i] = out_at(ys[i], glu ? yfmt : QK_ACT_F32, (size_t)t * ws[i]->n);
            const int r = run_gemv(ws, yt, cnt, glu, x.at((size_t)t * k), yfmt, 1, k, s, wsp, info);
            if (r != QK_OK || info) return r;
        }
        return QK_OK;
    }
    return rc == 0 ? QK_OK : rc == 1 ? QK_E_SHAPE : QK_E_HIP;
}

// A run of one quantized type on the GEMM: all its matrices in one launch, fp32 outputs.
int run_gemm_group(const qk_weight* const* ws, void* const* ys, int cnt, Act x, int m, hipStream_t s,
                   const Workspace* wsp) {
    const int k = ws[0]->k;
    if (x.fmt == QK_ACT_F32 && (size_t)m * k * 2 > wsp->gimg_bytes) return QK_E_RANGE;
    const uint8_t* w[qk::GEMV_MAX_CNT];
    int n[qk::GEMV_MAX_CNT];
    float* y[qk::GEMV_MAX_CNT];
    for (int i = 0; i < cnt; i++) {
        w[i] = (const uint8_t*)ws[i]->data;
        n[i] = ws[i]->n;
        y[i] = (float*)ys[i];
    }
    return qk::launch_gemm_group((int)ws[0]->type, w, n, y, cnt, k, x.p, x.fmt, m, wsp->gimg, wsp->kpart,
                                 wsp->kpart_bytes / sizeof(float), s) != 0
               ? QK_E_HIP
               : QK_OK;
}

// A gate/up pair on the GEMM: both matrices in one launch, y = silu(g) u in yfmt.
int run_gemm_glu(const qk_weight* const* ws, void* y, Act x, int yfmt, int m, hipStream_t s, const Workspace* wsp) {
    const int k = ws[0]->k;
    if (x.fmt == QK_ACT_F32 && (size_t)m * k * 2 > wsp->gimg_bytes) return QK_E_RANGE;
    return qk::launch_gemm_glu((int)ws[0]->type, (const uint8_t*)ws[0]->data, (const uint8_t*)ws[1]->data, k,
                               ws[0]->n, x.p, x.fmt, m, wsp->gimg, y, yfmt, wsp->kpart,
                               wsp->kpart_bytes / sizeof(float), s) != 0
               ? QK_E_HIP
               : QK_OK;
}

// Splits the tokens into launches of at most GEMV_MAX_M and the group into runs of one type
// (info != nullptr: the plan of the first launch only).  From GEMM_ROUTE_M tokens (the gemm_min_m
// knob) a gate/up pair and the quantized runs of a group take the GEMM instead, all m tokens and a
// run's matrices in one launch (K=5120 N=17408 Q4_K pair at 13 tokens: 99.0 us on the GEMV, two
// weight passes, against 33.6 us).
int gemv_group(const qk_weight* const* ws, void* const* ys, int cnt, bool glu, Act x, int yfmt, int m,
               hipStream_t s, const Workspace* wsp, qk::GemvPlan* info = nullptr) {
    const int k = ws[0]->k;
    auto gemm_plan = [&](int mt) {
        memset(info, 0, sizeof(*info));
        info->kernel = qk::GEMV_KERNEL_GEMM;
        info->token_slots = mt;
        return QK_OK;
    };
    if (glu && m >= gemm_route_m() && ws[0]->type != QK_T_F32 &&
        (size_t)2 * m * ws[0]->n <= wsp->kpart_bytes / sizeof(float))
        return info ? gemm_plan(m) : run_gemm_glu(ws, ys[0], x, yfmt, m, s, wsp);
    const bool gemm_runs = !glu && m >= gemm_route_m();
    for (int t0 = 0; t0 < m; t0 += gemm_runs ? m : qk::GEMV_MAX_M) {
        const int mt = gemm_runs ? m : std::min(qk::GEMV_MAX_M, m - t0);
        const Act xt = x.at((size_t)t0 * k);
        if (glu) {
            void* yt[1] = {out_at(ys[0], yfmt, (size_t)t0 * ws[0]->n)};
            int rc = run_gemv(ws, yt, 2, true, xt, yfmt, mt, k, s, wsp, info);
            if (rc != QK_OK || info) return rc;
            continue;
        }
        // consecutive matrices of equal type share one launch; F32 matrices run one by one
        for (int i = 0; i < cnt;) {
            if (ws[i]->type == QK_T_F32) {
                if (info) {
                    memset(info, 0, sizeof(*info));
                    info->kernel = qk::GEMV_KERNEL_F32;
                    info->token_slots = mt;
                    return QK_OK;
                }
                if (qk::launch_f32((const float*)ws[i]->data, k, ws[i]->n, xt.p, xt.fmt, mt,
                                   (float*)out_at(ys[i], QK_ACT_F32, (size_t)t0 * ws[i]->n), s))
                    return QK_E_HIP;
                i++;
                continue;
            }
            int j = i + 1;
            while (j < cnt && ws[j]->type == ws[i]->type) j++;  // (never F32: handled above)
            const qk_weight* sub[qk::GEMV_MAX_CNT];
            void* yt[qk::GEMV_MAX_CNT];
            for (int q = i; q < j; q++) {
                sub[q - i] = ws[q];
                yt[q - i] = out_at(ys[q], QK_ACT_F32, (size_t)t0 * ws[q]->n);
            }
            int rc;
            if (gemm_runs)  // the run's matrices and all m tokens in one GEMM launch (one weight pass)
                rc = info ? gemm_plan(mt) : run_gemm_group(sub, yt, j - i, xt, mt, s, wsp);
            else
                rc = run_gemv(sub, yt, j - i, false, xt, QK_ACT_F32, mt, k, s, wsp, info);
            if (rc != QK_OK || info) return rc;
            i = j;
        }
    }
    return QK_OK;
}

// The GEMM route (m >= GEMM_ROUTE_M by default): token chunks whose fp16 image fits the workspace, one
// launch each (the fp16 image only holds fp32 x rounded by the GEMM's conversion pass).
int run_gemm(const qk_weight* w, Act x, int m, float* y, hipStream_t s, const Workspace* wsp) {
    const int k = w->k;
    int chunk = (int)(wsp->gimg_bytes / ((size_t)k * 2)) / qk::GEMM_BM * qk::GEMM_BM;
    if (chunk < qk::GEMM_BM) return QK_E_RANGE;
    for (int t0 = 0; t0 < m; t0 += chunk) {
        const int mt = std::min(chunk, m - t0);
        const Act xt = x.at((size_t)t0 * k);
        if (qk::launch_gemm((int)w->type, (const uint8_t*)w->data, k, w->n, xt.p, xt.fmt, mt, wsp->gimg,
                            y + (size_t)t0 * w->n, wsp->kpart, wsp->kpart_bytes / sizeof(float), s) != 0)
            return QK_E_HIP;
    }
    return QK_OK;
}

bool fmt_ok(uint32_t f) { return f == QK_ACT_F32 || f == QK_ACT_F16 || f == QK_ACT_F16_XPERM; }

// Argument checks of qk_gemv_group_act (without the outputs when plan_only).  The xperm layouts are
// defined on runs of 1024 elements: x in xperm needs k % 1024 == 0 (as the reference's GEMV does,
// qwen_cuda/qwen.cpp:221-224), a GLU output in xperm n % 1024 == 0.
int check_group(const qk_weight* const* ws, void* const* ys, int cnt, int glu, const void* x, uint32_t xfmt,
                uint32_t yfmt, int m, bool plan_only) {
    if (!ws || (!plan_only && (!ys || !x))) return QK_E_NULL;
    if (cnt < 1 || cnt > qk::GEMV_MAX_CNT) return QK_E_GROUP;
    if (glu && cnt != 2) return QK_E_GROUP;
    if (m < 1 || m >= 16) return QK_E_SHAPE;
    if (!fmt_ok(xfmt) || !fmt_ok(yfmt) || (!glu && yfmt != QK_ACT_F32)) return QK_E_RANGE;
    for (int i = 0; i < cnt; i++) {
        int rc = check_weight(ws[i]);
        if (rc != QK_OK) return rc;
        if (ws[i]->layout != QK_LAYOUT_T16 && ws[i]->type != QK_T_F32) return QK_E_LAYOUT;
        if (ws[i]->k != ws[0]->k) return QK_E_GROUP;
        if (!plan_only && (!glu || i == 0)) {
            if (!ys[i]) return QK_E_NULL;
            if (!aligned16(ys[i])) return QK_E_ALIGN;
        }
    }
    if (glu && (ws[1]->n != ws[0]->n || ws[1]->type != ws[0]->type)) return QK_E_GROUP;
    if (glu && ws[0]->type == QK_T_F32) return QK_E_TYPE;  // the gate/up pair is quantized
    if (xfmt == QK_ACT_F16_XPERM && ws[0]->k % 1024) return QK_E_SHAPE;
    if (yfmt == QK_ACT_F16_XPERM && ws[0]->n % 1024) return QK_E_SHAPE;
    if (!plan_only && !aligned16(x)) return QK_E_ALIGN;
    return QK_OK;
}

// qk_matmul_act on the workspace wsp.
int matmul_on(const qk_weight* w, Act x, int m, float* y, hipStream_t s, const Workspace* wsp) {
    if (w->type == QK_T_F32)
        return qk::launch_f32((const float*)w->data, w->k, w->n, x.p, x.fmt, m, y, s) ? QK_E_HIP : QK_OK;
    if (m >= gemm_route_m()) return run_gemm(w, x, m, y, s, wsp);
    const qk_weight* ws[1] = {w};
    void* ys[1] = {y};
    return gemv_group(ws, ys, 1, false, x, QK_ACT_F32, m, s, wsp);
}

int check_matmul(const qk_weight* w, const void* x, uint32_t xfmt, int m, const float* y) {
    if (!x || !y) return QK_E_NULL;
    int rc = check_weight(w);
    if (rc != QK_OK) return rc;
    if (w->layout != QK_LAYOUT_T16 && w->type != QK_T_F32) return QK_E_LAYOUT;
    if (m < 1) return QK_E_SHAPE;
    if (!fmt_ok(xfmt)) return QK_E_RANGE;
    // xperm is the decode GEMV's layout (qwen_cuda/qwen.cpp:234: only for T < 16)
    if (xfmt == QK_ACT_F16_XPERM && (m >= GEMM_MIN_M || w->k % 1024)) return QK_E_SHAPE;
    if (!aligned16(x) || !aligned16(y)) return QK_E_ALIGN;
    return QK_OK;
}

}  // namespace

namespace qk {
int current_device() {
    int dev = 0;
    return hipGetDevice(&dev) == hipSuccess && dev >= 0 ? dev : 0;
}
int current_cus() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 256;
    std::lock_guard<std::mutex> lock(g_mu);
    return cu_count(dev);
}
}  // namespace qk

extern "C" {

const char* qk_status_string(int status) {
    switch (status) {
        case QK_OK: return "ok";
        case QK_E_NULL: return "null pointer argument";
        case QK_E_TYPE: return "unsupported tensor type";
        case QK_E_SHAPE: return "unsupported shape";
        case QK_E_LAYOUT: return "unsupported layout";
        case QK_E_ALIGN: return "device pointer not 16-byte aligned";
        case QK_E_HIP: return "HIP runtime error";
        case QK_E_GROUP: return "inconsistent gemv group";
        case QK_E_RANGE: return "value out of range";
        case QK_E_FORMAT: return "not a GGUF v3 file or truncated";
        case QK_E_NOTFOUND: return "no such tensor or key";
        case QK_E_IO: return "file cannot be read";
    }
    return "unknown status";
}

int qk_row_bytes(uint32_t type, int64_t k, uint64_t* rb) {
    if (!rb) return QK_E_NULL;
    if (k <= 0) return QK_E_SHAPE;
    switch (type) {
        case QK_T_F32: *rb = (uint64_t)k * 4; return QK_OK;
        case QK_T_Q8_0:
            if (k % 32) return QK_E_SHAPE;
            *rb = (uint64_t)(k / 32) * 34;
            return QK_OK;
        case QK_T_Q4_K:
        case QK_T_Q5_K:
        case QK_T_Q6_K:
            if (k % 256) return QK_E_SHAPE;
            *rb = (uint64_t)(k / 256) * (type == QK_T_Q4_K ? 144 : type == QK_T_Q5_K ? 176 : 210);
            return QK_OK;
    }
    return QK_E_TYPE;
}

int qk_weight_view(const void* data, uint32_t type, int32_t k, int32_t n, uint32_t layout, qk_weight* w) {
    if (!w) return QK_E_NULL;
    qk_weight v;
    v.data = data;
    v.type = type;
    v.k = k;
    v.n = n;
    v.layout = layout;
    v.rb = 0;
    if (!data) return QK_E_NULL;
    if (!type_supported(type)) return QK_E_TYPE;
    if (k <= 0 || n <= 0) return QK_E_SHAPE;
    int rc = qk_row_bytes(type, k, &v.rb);
    if (rc != QK_OK) return rc;
    rc = check_weight(&v);
    if (rc != QK_OK) return rc;
    *w = v;
    return QK_OK;
}

int qk_init_stream(qk_stream_t stream) {
    Workspace* w = nullptr;
    int ncu = 0;
    int rc = get_workspace((hipStream_t)stream, &w, &ncu);
    if (rc != QK_OK) return rc;
    // the allocation-free entry point's static workspace on this device, set up here once
    Workspace st;
    if (qk::noalloc_workspace((hipStream_t)stream, &st) != 0 || hipStreamSynchronize((hipStream_t)stream) != hipSuccess)
        return QK_E_HIP;
    return QK_OK;
}

int qk_repack(const qk_weight* src, void* dst, uint32_t dst_layout, qk_stream_t stream, qk_weight* out) {
    if (!src || !dst || !out) return QK_E_NULL;
    int rc = check_weight(src);
    if (rc != QK_OK) return rc;
    if (dst_layout != QK_LAYOUT_GGUF && dst_layout != QK_LAYOUT_T16) return QK_E_LAYOUT;
    if (src->type == QK_T_F32 && dst_layout != QK_LAYOUT_GGUF) return QK_E_LAYOUT;
    if (src->n % 16) return QK_E_SHAPE;
    if (!aligned16(dst)) return QK_E_ALIGN;
    qk_weight v = *src;
    v.data = dst;
    v.layout = dst_layout;
    if (dst_layout == src->layout) {
        if (hipMemcpyAsync(dst, src->data, (size_t)src->n * src->rb, hipMemcpyDeviceToDevice, (hipStream_t)stream) !=
            hipSuccess)
            return QK_E_HIP;
    } else {
        const int dir = dst_layout == QK_LAYOUT_T16 ? 0 : 1;
        if (qk::launch_repack((const uint8_t*)src->data, (uint8_t*)dst, (int)src->type, src->k, src->n, src->rb, dir,
                              (hipStream_t)stream) != 0)
            return QK_E_HIP;
    }
    *out = v;
    return QK_OK;
}

int qk_upload(const void* host, uint32_t type, int32_t k, int32_t n, uint32_t layout, qk_stream_t stream,
              qk_weight* out) {
    if (!host || !out) return QK_E_NULL;
    if (!type_supported(type)) return QK_E_TYPE;
    if (layout != QK_LAYOUT_GGUF && layout != QK_LAYOUT_T16) return QK_E_LAYOUT;
    if (type == QK_T_F32 && layout != QK_LAYOUT_GGUF) return QK_E_LAYOUT;
    if (k <= 0 || k % 256 || n <= 0 || (layout == QK_LAYOUT_T16 && n % 16)) return QK_E_SHAPE;
    uint64_t rb = 0;
    int rc = qk_row_bytes(type, k, &rb);
    if (rc != QK_OK) return rc;
    const size_t bytes = (size_t)n * rb;
    hipStream_t s = (hipStream_t)stream;
    void* dst = nullptr;
    if (hipMalloc(&dst, bytes) != hipSuccess) return QK_E_HIP;
    qk_weight w;
    w.data = dst;
    w.type = type;
    w.k = k;
    w.n = n;
    w.rb = rb;
    w.layout = layout;
    if (layout == QK_LAYOUT_GGUF) {
        if (hipMemcpyAsync(dst, host, bytes, hipMemcpyHostToDevice, s) != hipSuccess) {
            (void)hipFree(dst);
            return QK_E_HIP;
        }
    } else {
        void* tmp = nullptr;
        if (hipMalloc(&tmp, bytes) != hipSuccess) {
            (void)hipFree(dst);
            return QK_E_HIP;
        }
        bool ok = hipMemcpyAsync(tmp, host, bytes, hipMemcpyHostToDevice, s) == hipSuccess &&
                  qk::launch_repack((const uint8_t*)tmp, (uint8_t*)dst, (int)type, k, n, rb, 0, s) == 0 &&
                  hipStreamSynchronize(s) == hipSuccess;
        (void)hipFree(tmp);
        if (!ok) {
            (void)hipFree(dst);
            return QK_E_HIP;
        }
    }
    if (hipStreamSynchronize(s) != hipSuccess) {
        (void)hipFree(dst);
        return QK_E_HIP;
    }
    {
        std::lock_guard<std::mutex> lock(g_mu);
        g_owned.insert(dst);
    }
    *out = w;
    return QK_OK;
}

int qk_free(qk_weight* w) {
    if (!w || !w->data) return QK_E_NULL;
    {
        std::lock_guard<std::mutex> lock(g_mu);
        auto it = g_owned.find(w->data);
        if (it == g_owned.end()) return QK_E_RANGE;  // not allocated by qk_upload
        g_owned.erase(it);
    }
    if (hipFree((void*)w->data) != hipSuccess) return QK_E_HIP;
    memset(w, 0, sizeof(*w));
    return QK_OK;
}

int qk_dequant_rows(const qk_weight* w, const int32_t* rows, int32_t nrows, float* out, qk_stream_t stream) {
    if (!rows || !out) return QK_E_NULL;
    int rc = check_weight(w);
    if (rc != QK_OK) return rc;
    if (nrows <= 0) return QK_E_SHAPE;
    return qk::launch_dequant((const uint8_t*)w->data, (int)w->type, (int)w->layout, w->k, w->n, w->rb, rows, nrows,
                              out, (hipStream_t)stream) == 0
               ? QK_OK
               : QK_E_HIP;
}

int qk_embed(const qk_weight* table, const int32_t* tokens, const uint8_t* mask, const float* embd, int32_t m, float* x,
             qk_stream_t stream) {
    if (!tokens || !x || (mask && !embd)) return QK_E_NULL;
    int rc = check_weight(table);
    if (rc != QK_OK) return rc;
    if (m < 1) return QK_E_SHAPE;
    if (!aligned16(x) || (embd && !aligned16(embd))) return QK_E_ALIGN;
    return qk::launch_embed((const uint8_t*)table->data, (int)table->type, (int)table->layout, table->k, table->n,
                            table->rb, tokens, mask, embd, m, x, (hipStream_t)stream) == 0
               ? QK_OK
               : QK_E_HIP;
}

int qk_gemv_group_act(const qk_weight* const* ws, void* const* ys, int32_t cnt, int32_t glu, const void* x,
                      uint32_t xfmt, uint32_t glu_yfmt, int32_t m, qk_stream_t stream) {
    int rc = check_group(ws, ys, cnt, glu, x, xfmt, glu_yfmt, m, false);
    if (rc != QK_OK) return rc;
    Workspace* wsp = nullptr;
    int ncu = 0;
    rc = get_workspace((hipStream_t)stream, &wsp, &ncu);
    if (rc != QK_OK) return rc;
    return gemv_group(ws, ys, cnt, glu != 0, Act{x, (int)xfmt}, (int)glu_yfmt, m, (hipStream_t)stream, wsp);
}

int qk_gemv_group(const qk_weight* const* ws, float* const* ys, int32_t cnt, int32_t glu, const float* x, int32_t m,
                  qk_stream_t stream) {
    return qk_gemv_group_act(ws, (void* const*)ys, cnt, glu, x, QK_ACT_F32, QK_ACT_F32, m, stream);
}

int qk_gemv_plan(const qk_weight* const* ws, int32_t cnt, int32_t glu, int32_t m, qk_gemv_plan_info* out) {
    if (!out) return QK_E_NULL;
    int rc = check_group(ws, nullptr, cnt, glu, nullptr, QK_ACT_F32, QK_ACT_F32, m, true);
    if (rc != QK_OK) return rc;
    (void)device_cus();
    // the planner reads only the workspace's capacities: describe the per-stream one
    Workspace caps;
    caps.part_bytes = WS_PART_BYTES;
    caps.ncounters = WS_COUNTERS;
    caps.img_bytes = WS_IMG_BYTES;
    caps.gimg_bytes = WS_GEMM_BYTES;
    caps.nxslot = WS_XSLOTS;
    caps.kpart_bytes = WS_KPART_BYTES;
    qk::GemvPlan info;
    memset(&info, 0, sizeof(info));
    void* dummy[qk::GEMV_MAX_CNT] = {};
    rc = gemv_group(ws, dummy, cnt, glu != 0, Act{nullptr, QK_ACT_F32}, QK_ACT_F32, m, nullptr, &caps, &info);
    if (rc != QK_OK) return rc;
    out->kernel = info.kernel;
    out->work_groups = info.work_groups;
    out->waves_per_group = info.waves_per_group;
    out->ring_depth = info.ring_depth;
    out->slices = info.slices;
    out->token_slots = info.token_slots;
    out->lds_bytes = info.lds_bytes;
    return QK_OK;
}

int qk_matmul_act(const qk_weight* w, const void* x, uint32_t xfmt, int32_t m, float* y, qk_stream_t stream) {
    int rc = check_matmul(w, x, xfmt, m, y);
    if (rc != QK_OK) return rc;
    const Act xa{x, (int)xfmt};
    if (w->type == QK_T_F32) return matmul_on(w, xa, m, y, (hipStream_t)stream, nullptr);
    Workspace* wsp = nullptr;
    int ncu = 0;
    rc = get_workspace((hipStream_t)stream, &wsp, &ncu);
    if (rc != QK_OK) return rc;
    return matmul_on(w, xa, m, y, (hipStream_t)stream, wsp);
}

int qk_matmul(const qk_weight* w, const float* x, int32_t m, float* y, qk_stream_t stream) {
    return qk_matmul_act(w, x, QK_ACT_F32, m, y, stream);
}

int qk_matmul_noalloc(const qk_weight* w, const float* x, int32_t m, float* y, qk_stream_t stream) {
    int rc = check_matmul(w, x, QK_ACT_F32, m, y);
    if (rc != QK_OK) return rc;
    Workspace ws;
    if (qk::noalloc_workspace((hipStream_t)stream, &ws) != 0) return QK_E_HIP;
    return matmul_on(w, Act{x, QK_ACT_F32}, m, y, (hipStream_t)stream, &ws);
}

int qk_set_tuning(const char* name, int32_t value) {
    if (!name) return QK_E_NULL;
    if (!strcmp(name, "gemv_waves")) {
        if (value < 0) return QK_E_RANGE;
        qk::gemv_set_waves(value);
        return QK_OK;
    }
    if (!strcmp(name, "gemm_pairs")) return qk::gemm_set_pairs(value) ? QK_OK : QK_E_RANGE;
    if (!strcmp(name, "gemm_ksplit")) return qk::gemm_set_ksplit(value) ? QK_OK : QK_E_RANGE;
    if (!strcmp(name, "gemm_map")) {
        if (value != 0 && value != 1) return QK_E_RANGE;
        qk::gemm_set_map(value);
        return QK_OK;
    }
    if (!strcmp(name, "gemv_wpg")) {
        if (value < 0 || value > 16 || (value > 0 && value < 4)) return QK_E_RANGE;
        qk::gemv_set_wpg(value);
        return QK_OK;
    }
    if (!strcmp(name, "gemv_img_kib")) {
        if (value < 0 || value > 160) return QK_E_RANGE;
        qk::gemv_set_img_kib(value);
        return QK_OK;
    }
    if (!strcmp(name, "gemv_dshift")) {
        if (value < 0 || value > 31) return QK_E_RANGE;
        qk::gemv_set_dshift(value);
        return QK_OK;
    }
    if (!strcmp(name, "gemm_min_m")) {
        if (value != 0 && (value < 2 || value > GEMM_MIN_M)) return QK_E_RANGE;
        g_gemm_min_m = value;
        return QK_OK;
    }
    if (!strcmp(name, "gemv_min_waves")) {
        if (value < 0 || value > 16) return QK_E_RANGE;
        qk::gemv_set_min_waves(value);
        return QK_OK;
    }
    if (!strcmp(name, "gemv_token_slots")) {
        if (value != 4 && value != 8) return QK_E_RANGE;
        qk::gemv_set_max_slots(value);
        return QK_OK;
    }
    if (!strcmp(name, "gemv_fused")) {
        if (value != 0 && value != 1) return QK_E_RANGE;
        qk::gemv_set_fused(value == 1);
        return QK_OK;
    }
    return QK_E_RANGE;
}

int qk_synth_fill(uint32_t type, uint64_t seed, uint64_t block0, uint64_t nblocks, void* dst, qk_stream_t stream) {
    if (!dst) return QK_E_NULL;
    if (!type_supported(type) || type == QK_T_F32) return QK_E_TYPE;
    if (nblocks == 0) return QK_E_SHAPE;
    return qk::launch_synth((uint8_t*)dst, (int)type, seed, block0, nblocks, (hipStream_t)stream) == 0 ? QK_OK
                                                                                                         : QK_E_HIP;
}

}  // extern "C"
