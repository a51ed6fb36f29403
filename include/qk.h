/* qk.h — C ABI of the MI355X (gfx950) GGUF Q4_K / Q6_K quantized matmul with fused dequant.
 *
 * Plain pointers and sizes only.  Every entry point returns QK_OK (0) or a negative QK_E_* code
 * and never exits the process; the reference-shaped C++ shim (qk_shim.h) turns codes into the
 * reference's print-and-exit behaviour.  Device pointers are HIP device addresses; `stream` is a
 * hipStream_t (NULL = the default stream).  All launches are asynchronous on `stream`, allocate
 * nothing on the call path once the library is initialised for that stream, and are safe to
 * capture into a HIP graph after a first eager call (or qk_init_stream) on the same stream.
 *
 * Reference interfaces replaced (file:line in jtc1246/qwen3.8_27b_reference):
 *   the CUDA backend's anonymous-namespace matmul glue, qwen_cuda/qwen.cpp:43-49, 150-247, 756-761,
 *   its kernels qwen_cuda/kernels.cu:195-438, 945-961, and the CPU Ops::matmul, qwen_cpu/ops.h:54-76.
 */
#ifndef QK_H
#define QK_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGUF tensor type codes (qwen_cpu/gguf.h:22, qwen_cuda/kernels.cu:12). */
enum {
    QK_T_F32 = 0,
    QK_T_Q8_0 = 8,
    QK_T_Q4_K = 12,
    QK_T_Q5_K = 13,
    QK_T_Q6_K = 14
};

/* Byte layout of a weight in HBM.  Both hold exactly the GGUF bytes of the tensor (a repack is a
 * byte permutation inside the tensor's own range), so algorithmic bytes = GGUF bytes.
 *   QK_LAYOUT_GGUF: rows of K/256 super-blocks exactly as in the file (qwen_cuda/qwen.cpp:86-99).
 *   QK_LAYOUT_T16:  16-row tiles; inside a tile one group per super-block column holding the 16
 *                   rows' blocks split into planes ordered so that each 64-lane load instruction
 *                   of the GEMV/GEMM reads one contiguous 1 KiB run.  Needs n % 16 == 0.  Plays the
 *                   role of the reference's Q8_0/Q6_K row repack (qwen_cuda/kernels.cu:30-35,
 *                   945-961; qwen_cuda/qwen.cpp:176-193). */
enum {
    QK_LAYOUT_GGUF = 0,
    QK_LAYOUT_T16 = 1
};

enum {
    QK_OK = 0,
    QK_E_NULL = -1,   /* a required pointer is NULL */
    QK_E_TYPE = -2,   /* tensor type not supported by this entry point */
    QK_E_SHAPE = -3,  /* k, n, m or a row count outside what the kernels accept */
    QK_E_LAYOUT = -4, /* layout not supported for this type / entry point */
    QK_E_ALIGN = -5,  /* a device pointer is not 16-byte aligned */
    QK_E_HIP = -6,    /* a HIP runtime call or launch failed */
    QK_E_GROUP = -7,  /* inconsistent gemv group (count, k, glu pairing) */
    QK_E_RANGE = -8,  /* value out of range (e.g. x magnitude limit, workspace) */
    QK_E_FORMAT = -9, /* not a GGUF v3 file, or truncated (qk_gguf.h) */
    QK_E_NOTFOUND = -10, /* no tensor / key of that name (qk_gguf.h) */
    QK_E_IO = -11     /* the file cannot be opened or read (qk_gguf.h) */
};

typedef void* qk_stream_t; /* hipStream_t */

/* Activation formats of x (and of a GLU pair's output) at the *_act entry points.
 *   QK_ACT_F32:       fp32 [m][k] (the CPU path's, qwen_cpu/ops.h:54-76; the default entry points).
 *   QK_ACT_F16:       fp16 [m][k], as the reference's GPU matmuls read x (qwen_cuda/kernels.cu:307-361,
 *                     412-438).
 *   QK_ACT_F16_XPERM: fp16 with every 1024-element run of a row in the reference's decode layout
 *                     (qwen_cuda/kernels.cu:27-28 xperm: element 256 s + 32 j + 8 c + e of a run at
 *                     256 c + 8 (8 s + j) + e), which its producers write for T < 16
 *                     (k_add_norm kernels.cu:441-465, k_dn_post :611-617, qwen_cuda/qwen.cpp:234).
 * fp16 activations are widened exactly; results equal the fp32 entry points fed the widened values. */
enum {
    QK_ACT_F32 = 0,
    QK_ACT_F16 = 1,
    QK_ACT_F16_XPERM = 2
};

/* Non-owning view of one 2-D weight, y = W x with W of n rows by k columns
 * (qwen_cuda/qwen.cpp:43-49 `Weight{data,type,k,n,rb}` plus the layout tag). */
typedef struct qk_weight {
    const void* data; /* device address of the tensor's first byte */
    uint32_t type;    /* QK_T_* */
    int32_t k;        /* input dim (row length in elements), multiple of 256 */
    int32_t n;        /* output dim (rows) */
    uint64_t rb;      /* GGUF bytes per row (qwen_cpu/quants.h:21-31) */
    uint32_t layout;  /* QK_LAYOUT_* */
} qk_weight;

/* Human-readable text for a status code. */
const char* qk_status_string(int status);

/* Bytes per row of `k` elements of `type` (qwen_cpu/quants.h:21-31; the reference _Exit(1)s on an
 * unknown type, this returns QK_E_TYPE). */
int qk_row_bytes(uint32_t type, int64_t k, uint64_t* rb);

/* Build a validated view (qwen_cuda/qwen.cpp:152-173 get_w): k % 256 == 0, n > 0, the type has
 * kernels (F32, Q8_0, Q4_K, Q5_K, Q6_K), T16 needs n % 16 == 0, data 16-byte aligned.  F32 weights
 * are used as stored: QK_LAYOUT_GGUF only (QK_E_LAYOUT otherwise), no GLU pair. */
int qk_weight_view(const void* data, uint32_t type, int32_t k, int32_t n, uint32_t layout, qk_weight* w);

/* One-time per-stream setup: allocates the stream's workspace (partials, self-resetting counters,
 * activation images) and looks up qk_matmul_noalloc's static workspace on the current device.  Called
 * implicitly by the first matmul on a stream; call it explicitly before capturing a graph on a
 * stream that has not run a matmul yet.  Synchronous. */
int qk_init_stream(qk_stream_t stream);

/* Weight upload (qwen_cuda/qwen.cpp:756-761 whole-file cuMemcpyHtoD, then :185-193 repack):
 * allocates n*rb device bytes, copies `host` (GGUF bytes of the tensor) and, for QK_LAYOUT_T16,
 * repacks on the GPU.  Synchronous with respect to `stream` on return.  Release with qk_free. */
int qk_upload(const void* host, uint32_t type, int32_t k, int32_t n, uint32_t layout, qk_stream_t stream,
              qk_weight* out);

/* Frees a weight allocated by qk_upload and clears the view. */
int qk_free(qk_weight* w);

/* Out-of-place layout change on the GPU (exact byte permutation, tensor-sized): src -> dst
 * (dst: n*rb device bytes, not overlapping src).  GGUF <-> T16 in either direction. */
int qk_repack(const qk_weight* src, void* dst, uint32_t dst_layout, qk_stream_t stream, qk_weight* out);

/* Dequantize rows `rows[0..nrows)` (device int32 array) to fp32 out[nrows][k], bit-exact with
 * qwen_cpu/quants.h dequant_row (the reference's k_dq_* selftest vehicle, qwen_cuda/kernels.cu:363-373,
 * qwen_cuda/qwen.cpp:1317-1328).  Any layout.  A row index outside [0, n) yields a NaN row. */
int qk_dequant_rows(const qk_weight* w, const int32_t* rows, int32_t nrows, float* out, qk_stream_t stream);

/* Token embedding (the reference's k_embed_<type>, qwen_cuda/kernels.cu:375-389, launched per step at
 * qwen_cuda/qwen.cpp:265): x[t][0..k) = embd[t][0..k) where mask != NULL and mask[t] != 0 (an
 * embedding computed elsewhere, e.g. an image token), else row tokens[t] of the table dequantized
 * bit-exactly as qwen_cpu/quants.h dequant_row, from either layout; t < m.  tokens (int32 [m]), mask
 * (uint8 [m]) and embd / x (fp32 [m][k], 16-byte aligned) are device pointers.  A token id outside
 * [0, n) yields a NaN row (the reference reads out of bounds). */
int qk_embed(const qk_weight* table, const int32_t* tokens, const uint8_t* mask, const float* embd, int32_t m, float* x,
             qk_stream_t stream);

/* y[m][n] = sum_k W[n][k] * x[m][k]; x fp32 [m][k], y fp32 [m][n], both 16-byte aligned.
 * m <= 4 runs the fused-dequant MFMA GEMV, m >= 5 the LDS-dequant MFMA GEMM (qwen_cuda/qwen.cpp:240-247
 * matmul, which runs its GEMV below 16 tokens on fp16 x; CPU Ops::matmul qwen_cpu/ops.h:54-76): from
 * five tokens the GEMV's eight-token form is compute-bound (and needs a second weight pass from nine)
 * while the GEMM, one 32-token block per work-group, reads the weights once at the memory system's
 * pace (the gemm_min_m knob moves the boundary).  The GEMV path
 * (int8 MFMA kernel) carries each token's x per 256-element super-block as three int8 parts with
 * fp32 scales, every element within max|x| / 16387064 of its value, for any finite fp32 x (a
 * super-block below 2^-100 is converted from x * 2^100 and scaled back); a NaN or inf in x makes
 * the outputs it feeds NaN.  The GEMM path rounds x to fp16.  Returns QK_E_SHAPE when no kernel has
 * a plan for the shape. */
int qk_matmul(const qk_weight* w, const float* x, int32_t m, float* y, qk_stream_t stream);

/* qk_matmul without any allocation: the same kernels and results, with the workspace taken from a
 * static device array of 72.25 MiB per GPU (its address looked up by qk_init_stream or by the first
 * call on a device; zero-initialised static storage is already the state its combine slots and
 * counters need, so no set-up work is enqueued and the first call on a device may come under graph
 * capture) instead of the per-stream buffers qk_matmul allocates on first use.  It never calls
 * hipMalloc / hipFree.  Shapes whose workspace does not fit the array return QK_E_RANGE: a GEMV
 * with more than 65536 16-row tiles, or whose Q4_K / Q6_K x image (general kernel) exceeds 4 MiB
 * (k > ~225k at four tokens); a GEMM with k > 65536 (its fp16 copy of x holds 128-token chunks).  The
 * GEMM runs larger m in more chunks and splits K only as far as 16 MiB of partials allow.
 * Every call on one GPU shares the array: calls that overlap on one GPU (other streams, other host
 * threads) race and must be serialised by the caller.
 * No counterpart in the reference: for callers that cannot allocate (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc). */
int qk_matmul_noalloc(const qk_weight* w, const float* x, int32_t m, float* y, qk_stream_t stream);

/* qk_matmul with x in format xfmt (QK_ACT_*): the reference's matmul(w, x, T, y) with fp16 x
 * (qwen_cuda/qwen.cpp:240-247).  QK_ACT_F16_XPERM needs m < 16 (as in the reference) and k % 1024 == 0.
 * The routing is qk_matmul's for every format: m <= 4 on the GEMV, m >= 5 on the GEMM, which reads
 * fp16 x, plain or xperm, where it lies (no rounding, no copy).  y is fp32 [m][n]. */
int qk_matmul_act(const qk_weight* w, const void* x, uint32_t xfmt, int32_t m, float* y, qk_stream_t stream);

/* Grouped GEMV for m < 16 (qwen_cuda/qwen.cpp:220-238 gemv, MmGroup kernels.cu:403-438): `cnt`
 * (1..4) weights sharing x and k, one output ys[i][m][n_i] each.  glu != 0: cnt must be 2,
 * ws[0]/ws[1] are gate/up with equal n and ys[0][m][n] = silu(gate x) * (up x) in fp32.  A quantized
 * gate/up pair, and each run of one quantized type in a group, of five or more tokens run on the GEMM
 * (a run's matrices in one launch, one weight pass; fp16 operands, the GEMM's bar); fewer tokens on
 * the GEMV, F32 matrices on their own kernel. */
int qk_gemv_group(const qk_weight* const* ws, float* const* ys, int32_t cnt, int32_t glu, const float* x, int32_t m,
                  qk_stream_t stream);

/* qk_gemv_group with x in format xfmt and, for a GLU pair, its output in glu_yfmt (QK_ACT_*): the
 * reference's gemv(ws, ys, cnt, glu, x, T) (qwen_cuda/qwen.cpp:220-238), whose GLU writes fp16
 * silu(g) u at the xperm position of its row when the step runs the xperm layout (kernels.cu:419-426).
 * Non-GLU outputs stay fp32 [m][n].  An fp16 GLU output is rounded to nearest even.  xperm x needs
 * k % 1024 == 0, an xperm GLU output n % 1024 == 0; glu_yfmt must be QK_ACT_F32 without glu. */
int qk_gemv_group_act(const qk_weight* const* ws, void* const* ys, int32_t cnt, int32_t glu, const void* x,
                      uint32_t xfmt, uint32_t glu_yfmt, int32_t m, qk_stream_t stream);

/* What qk_gemv_group (or qk_matmul) would launch for these weights and token count: the
 * first launch's kernel and shape.  Launches nothing and touches no device memory.  A planning query
 * with no counterpart in the reference (its GEMV has one fixed launch shape, qwen_cuda/qwen.cpp:
 * 227-237); for tests and tuning. */
enum {
    QK_GEMV_INT8 = 1,    /* int8 MFMA kernel, x converted inside (m <= 8 per launch, all quantized types) */
    QK_GEMV_GENERAL = 2, /* Q4_K / Q6_K fp16-pair kernel with an x prepass */
    QK_GEMV_F32 = 3,     /* F32 weights */
    QK_GEMV_GEMM = 4     /* the GEMM takes the call (five tokens or more, the gemm_min_m knob): a
                          * gate/up pair or a group's run of one type, its matrices in one launch */
};
typedef struct qk_gemv_plan_info {
    int32_t kernel;          /* QK_GEMV_* */
    int32_t work_groups;
    int32_t waves_per_group;
    int32_t ring_depth;      /* units (weight groups) in flight per wave */
    int32_t slices;          /* K-slices of the int8 kernel's unit order */
    int32_t token_slots;     /* tokens the launch's kernel instance carries (1, 2 or 4) */
    int32_t lds_bytes;       /* LDS per work-group */
} qk_gemv_plan_info;
int qk_gemv_plan(const qk_weight* const* ws, int32_t cnt, int32_t glu, int32_t m, qk_gemv_plan_info* out);

/* Tuning override for measurement sweeps: "gemv_waves" (waves of the general persistent GEMV grid;
 * a nonzero value also routes Q4_K / Q6_K calls of every m through that kernel; 0 restores the
 * built-in plan), "gemv_fused" (1 = m <= 8 per launch through the int8 kernel where its plan applies,
 * the default; 0 = Q4_K / Q6_K through the general kernel, an exact fp16 pair per element of x
 * whose domain is |x| < 65504 with Q4_K 32-element sub-block sums below that too, for comparisons
 * only; Q8_0 / Q5_K always take the int8 kernel),
 * "gemv_wpg" (at most this many waves, 4..16, per int8-kernel work-group; 0 = as many as the LDS
 * holds), "gemv_img_kib" (int8 kernel: the K-slices double until a range's activation image fits this
 * many KiB, 1..160; 0 restores 32), "gemv_dshift" (int8 kernel: about nu >> value of a work-group's nu
 * units are handed out by a counter, the rest statically; 0..31, default 1), "gemv_min_waves" (int8
 * kernel at m >= 2: the fewest waves per work-group its plan may leave before Q4_K / Q6_K calls go to
 * the general kernel; 0..16, default 0), "gemv_token_slots" (int8 kernel: the most tokens one launch
 * carries, 8 (default: one weight pass per eight tokens) or 4 (m = 5..8 as four tokens and the rest)),
 * "gemm_min_m" (the smallest m qk_matmul and qk_matmul_act route to the GEMM, and qk_gemv_group(_act)
 * a gate/up pair or a group; 2..16, 0 restores the default 5), "gemm_ksplit" (GEMM K-parts, 1..16,
 * partials added in part order by a second kernel; 0 restores the plan), "gemm_pairs" (16-row tile pairs per GEMM work-group: 2, 3, 4, 5, 8 or 9;
 * 0 restores the built-in plan) or "gemm_map" (1 = each XCD serves one token block where 2, 4 or 8
 * token blocks divide the XCDs, the default; 0 = the (K-part, pair group) units dealt densely over the
 * XCDs, each with its token blocks on one XCD, which every call with one token block or another count
 * of them takes).  Returns QK_E_RANGE for an unknown name or value. */
int qk_set_tuning(const char* name, int32_t value);

#ifdef __cplusplus
}
#endif

#endif /* QK_H */
