// Measurement aid for bench.py, built as its own library (libqkprobe.so), not part of the C ABI of
// include/: a plain streaming read of a device buffer, the practical ceiling for a kernel that reads
// the same bytes once.  It has no counterpart in the reference.
//
// Work-group b reads the contiguous 16-byte words [b * per, (b + 1) * per) of the buffer with
// non-temporal 16-byte loads, U loads per thread in flight, and folds them into an xor that is
// stored only if it equals a constant no synthetic input produces (so the loads cannot be dropped
// and the kernel writes nothing in practice).
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace {

typedef uint32_t u4 __attribute__((ext_vector_type(4)));

template <int U>
__global__ __launch_bounds__(256) void k_read(const u4* __restrict__ p, size_t n, size_t per, uint32_t* sink) {
    const size_t b0 = (size_t)blockIdx.x * per, b1 = b0 + per < n ? b0 + per : n;
    u4 acc = {0u, 0u, 0u, 0u};
    for (size_t i = b0 + threadIdx.x; i < b1; i += 256 * U) {
        u4 v[U];
#pragma unroll
        for (int j = 0; j < U; j++) {
            const size_t k = i + 256 * (size_t)j;
            v[j] = k < b1 ? __builtin_nontemporal_load(p + k) : u4{0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int j = 0; j < U; j++) acc ^= v[j];
    }
    const uint32_t s = acc.x ^ acc.y ^ acc.z ^ acc.w;
    if (s == 0x9E3779B9u) sink[blockIdx.x] = s;
}

}  // namespace

extern "C" {

// Reads `bytes` (a multiple of 16) at `p` with `wgs` work-groups of 256 threads, `unroll` (4 or 8)
// loads per thread in flight; `sink` needs 4 * wgs device bytes.  Returns 0, or -1 on bad
// arguments or a launch error.
int qkp_read(const void* p, size_t bytes, int wgs, int unroll, void* sink, void* stream) {
    if (!p || !sink || bytes % 16 || wgs < 1 || (unroll != 4 && unroll != 8)) return -1;
    const size_t n = bytes / 16, per = (n + wgs - 1) / wgs;
    const hipStream_t s = (hipStream_t)stream;
    if (unroll == 4)
        hipLaunchKernelGGL(k_read<4>, dim3(wgs), dim3(256), 0, s, (const u4*)p, n, per, (uint32_t*)sink);
    else
        hipLaunchKernelGGL(k_read<8>, dim3(wgs), dim3(256), 0, s, (const u4*)p, n, per, (uint32_t*)sink);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // extern "C"
