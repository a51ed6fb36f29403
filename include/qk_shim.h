/* qk_shim.h — the reference's C++ matmul entry points, re-expressed over the C ABI (qk.h).
 *
 * A maintainer replaces the anonymous-namespace Weight / get_w / gemv / matmul / k_embed launch of
 * qwen_cuda/qwen.cpp:43-49, 152-173, 220-247, 265 and its whole-file upload (:737-761) with these
 * (same names, argument meaning and fail-stop behaviour: any error prints one line to stderr and ends
 * the process with _Exit(1), as qwen_cuda/cu.h:21-27 does).  Device pointers are HIP device
 * addresses.  As in the reference, gemv / matmul take fp16 activations, in the xperm layout when the
 * step runs it (set_xperm, the reference's G_xperm, qwen_cuda/qwen.cpp:82, 234, 264), and a GLU pair
 * writes fp16 silu(gate) up at the xperm position of its row; gemv_f32 / matmul_f32 take fp32
 * activations and write fp32 (the CPU path's formats).
 */
#pragma once

#include <stdint.h>

#include <string>

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

/* qwen_cuda/qwen.cpp:82 G_xperm: whether the activations of this step's GEMVs (T < 16) are in the
 * xperm layout (the reference's forward sets it to T < 16, forward_batch to true). */
void set_xperm(bool on);

/* qwen_cuda/qwen.cpp:737-761: opens the GGUF file, copies it whole into one device allocation and
 * repacks the quantized matrices in place (T16 here, :185-193 there); the host copy is released. */
void load_weights(const char* gguf_path);

/* qwen_cuda/qwen.cpp:152-173 get_w: a non-owning view of tensor `name` in the one device copy,
 * checked to be 2-D [k, n] with kernels for its type. */
Weight get_w(const std::string& name, int k, int n);

/* One tensor's GGUF bytes to HBM in the T16 layout, an allocation of its own (tests, tools). */
Weight upload(const void* host_gguf_bytes, uint32_t type, int k, int n);

/* qwen_cuda/qwen.cpp:220-238: cnt (<= 4) matrices sharing x (fp16 [T][k], xperm if T < 16 and
 * set_xperm(true)), T < 16, one launch; glu: ws[0]/ws[1] are gate/up and ys[0] receives fp16
 * silu(gate x) * (up x) (at the xperm position of its row under the same condition); otherwise
 * ys[i] are fp32 [T][n_i].  T <= 4 on the GEMV, T >= 5 on the GEMM (one weight pass). */
void gemv(const Weight* const* ws, const DevPtr* ys, int cnt, bool glu, DevPtr x, int T);

/* qwen_cuda/qwen.cpp:240-247: y[T][n] (fp32) = x[T][k] (fp16, xperm if T < 16 and set_xperm(true))
 * W^T; T <= 4 on the GEMV, T >= 5 on the GEMM (the reference runs its GEMV below 16 tokens). */
void matmul(const Weight& w, DevPtr x, int T, DevPtr y);

/* qwen_cuda/qwen.cpp:265 (k_embed_<type>): x[t] (fp32 [T][k]) = embd[t] where mask[t] != 0, else
 * row tokens[t] of the table; mask / embd may be null (then every row is a table row). */
void embed(const Weight& table, DevPtr tokens, DevPtr mask, DevPtr embd, DevPtr x, int T);

/* gemv / matmul with fp32 activations and fp32 outputs (the GLU output too). */
void gemv_f32(const Weight* const* ws, const DevPtr* ys, int cnt, bool glu, DevPtr x, int T);
void matmul_f32(const Weight& w, DevPtr x, int T, DevPtr y);

}  // namespace qkshim
