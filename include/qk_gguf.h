/* qk_gguf.h — GGUF v3 file → HBM: the on-disk format feeding the matmul path.
 *
 * Replaces the reference's Gguf::open (qwen_cpu/gguf.h:106-175: whole file read into host memory,
 * header / key-value / tensor-info parse, tensor data at the aligned data start) and its CUDA
 * upload (qwen_cuda/qwen.cpp:737-761: the whole file copied into one device allocation, then the
 * quantized rows repacked in place, repack_weights at :185-193).  Errors return QK_E_* codes (the
 * reference prints and exits).  Here every quantized 2-D tensor whose shape the T16 layout takes
 * (k % 256 == 0, n % 16 == 0) is repacked in place to QK_LAYOUT_T16; the others stay as stored.
 * Host memory is released after the upload, the device copy by qk_gguf_close. */
#ifndef QK_GGUF_H
#define QK_GGUF_H

#include <stdint.h>
#include "qk.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct qk_gguf qk_gguf; /* opaque */

/* Reads and parses a GGUF v3 file (magic "GGUF", version 3): numeric and string scalar key-values
 * are kept, arrays skipped; tensor data starts at the header end rounded up to general.alignment
 * (32 when absent).  QK_E_IO: the file cannot be read; QK_E_FORMAT: not GGUF v3, truncated, or a
 * tensor past the end of the file. */
int qk_gguf_open(const char* path, qk_gguf** out);
void qk_gguf_close(qk_gguf* f);

int qk_gguf_tensor_count(const qk_gguf* f, int64_t* count);
/* Tensor i: name (valid until close), GGML type code, dims (dims[0] innermost, at most 4), byte
 * offset of its data from the file start, and its byte size. */
int qk_gguf_tensor_info(const qk_gguf* f, int64_t i, const char** name, uint32_t* type, int32_t* ndims,
                        int64_t dims[4], uint64_t* file_offset, uint64_t* nbytes);
int qk_gguf_find(const qk_gguf* f, const char* name, int64_t* index); /* QK_E_NOTFOUND if absent */
int qk_gguf_kv_num(const qk_gguf* f, const char* key, double* value);    /* numeric scalars */
int qk_gguf_kv_str(const qk_gguf* f, const char* key, const char** value); /* string scalars */

/* Copies the whole file into one device allocation on `stream`, repacks the T16-eligible quantized
 * tensors in place and frees the host copy; synchronous on return. */
int qk_gguf_upload(qk_gguf* f, qk_stream_t stream);
/* View of an uploaded 2-D tensor [n][k] (k = dims[0], n = dims[1]) in its HBM layout. */
int qk_gguf_weight(const qk_gguf* f, const char* name, qk_weight* w);

#ifdef __cplusplus
}
#endif

#endif /* QK_GGUF_H */
