/* qk_shim.h — the reference's C++ matmul entry points, re-expressed over the C ABI (qk.h).
 *
 * A maintainer replaces the anonymous-namespace Weight / get_w / gemv / matmul of
 * qwen_cuda/qwen.cpp:43-49, 152-173, 220-247 with these (same names, argument meaning and
 * fail-stop behaviour: any error prints one line to stderr and ends the process with _Exit(1),
 * as qwen_cuda/cu.h:21-27 does).  Device pointers are HIP device addresses.  Differences, by
 * design: activations x are fp32 (the reference feeds fp16, qwen_cuda/kernels.cu:27-28), and the
 * GLU output of gemv is fp32 silu(gate)*up (the reference writes fp16, kernels.cu:419-426).
 */
#pragma once

#include <stdint.h>

#include "qk.h"

namespace qkshim {

using DevPtr = void*;  // the reference's CUdeviceptr

/* qwen_cuda/qwen.cpp:43-49 Weight{data, type, k, n, rb}, plus the byte layout in HBM. */
struct Weight {
    DevPtr data = nullptr;
    uint32_t type = 0;
    int k = 0;  // input dim (row length)
    int n = 0;  // output dim (rows)
    uint64_t rb = 0;
    uint32_t layout = QK_LAYOUT_T16;
};

/* qwen_cuda/cu.h:67-70 use(sid): later launches of this thread go to `stream`. */
void use(qk_stream_t stream);

/* qwen_cuda/qwen.cpp:152-173 get_w + 756-761 upload + 185-193 repack, for one tensor: copies the
 * GGUF bytes of an n x k Q4_K/Q6_K tensor to HBM in the T16 layout.  Shape/type errors are fatal. */
Weight upload(const void* host_gguf_bytes, uint32_t type, int k, int n);

/* qwen_cuda/qwen.cpp:220-238: cnt (<= 4) matrices sharing x (fp32 [T][k], T < 16), one launch;
 * glu: ws[0]/ws[1] are gate/up and ys[0] receives silu(gate x) * (up x). */
void gemv(const Weight* const* ws, const DevPtr* ys, int cnt, bool glu, DevPtr x, int T);

/* qwen_cuda/qwen.cpp:240-247: y[T][n] = x[T][k] W^T; T < 16 runs the GEMV, else the GEMM. */
void matmul(const Weight& w, DevPtr x, int T, DevPtr y);

}  // namespace qkshim
