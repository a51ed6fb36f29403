// TEST INFRASTRUCTURE — checker only, never product code.
//
// Binding translation unit that exports the reference's own CPU quantized-matmul path
// (header-only, anonymous namespaces) with C linkage so tests can load it with ctypes.
// Compiled by oracle/Makefile (target `ref`) straight from the headers where they lie in
// /root/reference/qwen_cpu; the output goes to oracle/_ref/ only.  No reference source is
// copied: the headers are #included from the reference tree through -I.
//
// Bound reference items:
//   Quants::row_bytes            qwen_cpu/quants.h:21-31
//   Quants::get_scale_min_k4     qwen_cpu/quants.h:33-41
//   Quants::Ref::{q8_0,q4_k,q5_k,q6_k}   qwen_cpu/quants.h:45-121 (scalar reference dequant)
//   Quants::dequant_row          qwen_cpu/quants.h:193-203 (AVX-512 dequant dispatch)
//   Ops::matmul                  qwen_cpu/ops.h:54-76 (4-row tasks, fp32 FMA micro-kernel)
//   Pool::init / Ops::init_buffers  qwen_cpu/pool.h:149-152, qwen_cpu/ops.h:28-30
// plus a timing loop over Ops::matmul for the benchmark's CPU baseline (qkref_time_seq).
#include <chrono>
#include <cstring>
#include "quants.h"
#include "ops.h"

extern "C" {

static int g_threads = 0;

int qkref_init(int threads) {
    if (g_threads) return g_threads;
    if (threads < 1) threads = 1;
    if (threads > Ops::MAX_THREADS) threads = Ops::MAX_THREADS;
    Pool::init(threads);
    Ops::init_buffers(threads);
    g_threads = threads;
    return g_threads;
}

unsigned long long qkref_row_bytes(unsigned type, long long k) { return Quants::row_bytes(type, k); }

void qkref_scale_min_k4(int j, const unsigned char* q, unsigned char* sc, unsigned char* m) {
    Quants::get_scale_min_k4(j, q, sc, m);
}

int qkref_dequant_scalar(unsigned type, const void* src, float* y, long long k) {
    switch (type) {
        case Gguf::T_Q8_0: Quants::Ref::q8_0(src, y, k); return 0;
        case Gguf::T_Q4_K: Quants::Ref::q4_k(src, y, k); return 0;
        case Gguf::T_Q5_K: Quants::Ref::q5_k(src, y, k); return 0;
        case Gguf::T_Q6_K: Quants::Ref::q6_k(src, y, k); return 0;
    }
    return -1;
}

int qkref_dequant_avx(unsigned type, const void* src, float* y, long long k) {
    if (type != Gguf::T_F32 && type != Gguf::T_Q8_0 && type != Gguf::T_Q4_K && type != Gguf::T_Q5_K &&
        type != Gguf::T_Q6_K)
        return -1;
    Quants::dequant_row(type, src, y, k);
    return 0;
}

// Requires qkref_init first; k <= Ops::K_MAX, n % 4 == 0 (ops.h:15-16, 55).
int qkref_matmul(const unsigned char* data, unsigned type, int k, int n, const float* x, int T, float* y) {
    if (!g_threads || k > Ops::K_MAX || n % Ops::ROWS) return -1;
    Ops::Weight w;
    w.data = data;
    w.type = type;
    w.k = k;
    w.n = n;
    w.rb = Quants::row_bytes(type, k);
    Ops::matmul(w, x, T, y);
    return 0;
}

// The CPU baseline's timing loop, in C so that per-call overhead of the caller does not enter small
// matmuls: runs matmul i of `count` (weights data[i] of types[i], k ks[i], n ns[i], input xs[i] [T][k],
// output ys[i]) in order, `reps` times over, and returns the elapsed wall time in nanoseconds (-1 on a
// rejected shape).
long long qkref_time_seq(int count, const unsigned char* const* data, const unsigned* types, const int* ks,
                         const int* ns, const float* const* xs, int T, float* const* ys, int reps) {
    if (!g_threads) return -1;
    for (int i = 0; i < count; i++)
        if (ks[i] > Ops::K_MAX || ns[i] % Ops::ROWS) return -1;
    const auto t0 = std::chrono::steady_clock::now();
    for (int r = 0; r < reps; r++)
        for (int i = 0; i < count; i++) {
            Ops::Weight w;
            w.data = data[i];
            w.type = types[i];
            w.k = ks[i];
            w.n = ns[i];
            w.rb = Quants::row_bytes(types[i], ks[i]);
            Ops::matmul(w, xs[i], T, ys[i]);
        }
    return (long long)std::chrono::duration_cast<std::chrono::nanoseconds>(std::chrono::steady_clock::now() - t0)
        .count();
}

}  // extern "C"
