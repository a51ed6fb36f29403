// F32 weights (the projections a Q4_K_M file keeps unquantized, e.g. the DeltaNet alpha/beta of
// docs/model.md:328): y[t][r] = sum_k W[r][k] x[t][k], replacing the reference's F32 instantiation
// of its GEMV/GEMM (qwen_cuda/kernels.cu:74-78, 397) and the CPU path's F32 rows used as stored
// (qwen_cpu/ops.h:60-67, quants.h:193-203).  W stays row-major as in the file (no dequant, no
// repack): one wave per row reads it with 16-byte loads once per block of up to four tokens, x
// (a few KB per token, fp32 or fp16) comes from L2, fp32 FMA accumulation and a cross-lane sum.  These matrices
// are small (5120 x 48 in the model), so the kernel is latency-, not bandwidth-, bound.
#include "qk_device.h"
#include "qk_internal.h"

namespace qk {
namespace {

__device__ inline float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
    return v;
}

__global__ __launch_bounds__(256) void k_matmul_f32(const float* __restrict__ w, int k, int n,
                                                    const void* __restrict__ x, int xfmt, int m,
                                                    float* __restrict__ y) {
    const int lane = threadIdx.x & 63, row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= n) return;  // no barrier follows
    const float* wr = w + (size_t)row * k;
    for (int t0 = 0; t0 < m; t0 += 4) {
        float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        for (int i = 4 * lane; i < k; i += 256) {  // k % 256 == 0
            const f4 wv = *(const f4*)(wr + i);
#pragma unroll
            for (int t = 0; t < 4; t++) {
                if (t0 + t < m) {
                    const f4 xv = load_act4(x, xfmt, k, t0 + t, i);
                    acc[t] = fmaf(wv.x, xv.x, fmaf(wv.y, xv.y, fmaf(wv.z, xv.z, fmaf(wv.w, xv.w, acc[t]))));
                }
            }
        }
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const float v = wave_sum(acc[t]);
            if (lane == 0 && t0 + t < m) y[(size_t)(t0 + t) * n + row] = v;
        }
    }
}

}  // namespace

int launch_f32(const float* w, int k, int n, const void* x, int xfmt, int m, float* y, hipStream_t s) {
    hipLaunchKernelGGL(k_matmul_f32, dim3((n + 3) / 4), dim3(256), 0, s, w, k, n, x, xfmt, m, y);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace qk
