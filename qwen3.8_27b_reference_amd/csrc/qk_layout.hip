// Weight-placement kernels: GGUF <-> T16 repack, bit-exact row dequant, synthetic block fill.
//
//   repack    plays the role of k_repack (qwen_cuda/kernels.cu:945-961) driven by repack_weights
//             (qwen_cuda/qwen.cpp:185-193), with the T16 group layout of qk_device.h.
//   dequant   is the selftest vehicle k_dq_* (qwen_cuda/kernels.cu:363-373, qwen_cuda/qwen.cpp:1317):
//             fp32 results identical to qwen_cpu/quants.h Ref::q4_k / Ref::q6_k (:53-71, :96-121).
#include "qk_device.h"
#include "qk_internal.h"

namespace qk {
namespace {

// One work-group per (tile, super-block) group; threads stride over the group's bytes.
// dir 0: GGUF -> T16 (gather), dir 1: T16 -> GGUF (scatter back).
__global__ __launch_bounds__(256) void k_repack(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst,
                                                int type, int nsb, uint64_t rb, int dir) {
    const int bs = type == T_Q4_K ? Q4K_BYTES : Q6K_BYTES;
    const int gbytes = 16 * bs;
    const uint64_t tile = blockIdx.y, sb = blockIdx.x;
    const uint64_t gofs = (tile * nsb + sb) * (uint64_t)gbytes;
    for (int o = threadIdx.x; o < gbytes; o += blockDim.x) {
        int r, p;
        t16_src(type, o, r, p);
        const uint64_t gg = (tile * 16 + r) * rb + sb * bs + p;
        if (dir == 0) dst[gofs + o] = src[gg];
        else dst[gg] = src[gofs + o];
    }
}

__device__ inline uint8_t wbyte(const uint8_t* w, int layout, int type, int nsb, uint64_t rb, int row, int sb, int p) {
    const int bs = type == T_Q4_K ? Q4K_BYTES : Q6K_BYTES;
    if (layout == LAYOUT_GGUF) return w[(uint64_t)row * rb + (uint64_t)sb * bs + p];
    const uint64_t g = ((uint64_t)(row >> 4) * nsb + sb) * (uint64_t)(16 * bs);
    return w[g + t16_dst(type, row & 15, p)];
}

__device__ inline uint32_t wu16(const uint8_t* w, int layout, int type, int nsb, uint64_t rb, int row, int sb, int p) {
    return (uint32_t)wbyte(w, layout, type, nsb, rb, row, sb, p) |
           ((uint32_t)wbyte(w, layout, type, nsb, rb, row, sb, p + 1) << 8);
}

// One work-group per requested row; each thread produces whole elements with the reference's exact
// fp32 expression: Q4_K (d*sc)*q - dmin*m, Q6_K (d*sc)*(q-32).  Both are single-rounding exact
// forms (products exact in fp32), so FMA contraction cannot change the bits.
__global__ __launch_bounds__(256) void k_dequant(const uint8_t* __restrict__ w, int type, int layout, int k,
                                                 uint64_t rb, const int32_t* __restrict__ rows, float* __restrict__ out) {
    const int row = rows[blockIdx.x];
    const int nsb = k / 256;
    float* dst = out + (uint64_t)blockIdx.x * k;
    for (int e = threadIdx.x; e < k; e += blockDim.x) {
        const int sb = e >> 8, ee = e & 255;
        float v;
        if (type == T_Q4_K) {
            const float d = h2f_bits(wu16(w, layout, type, nsb, rb, row, sb, 0));
            const float dmin = h2f_bits(wu16(w, layout, type, nsb, rb, row, sb, 2));
            uint8_t sc12[12];
            for (int i = 0; i < 12; i++) sc12[i] = wbyte(w, layout, type, nsb, rb, row, sb, 4 + i);
            const int g = ee >> 6, h = (ee >> 5) & 1, l = ee & 31;
            int sc, m;
            scale_min_k4(2 * g + h, sc12, sc, m);
            const int q = (wbyte(w, layout, type, nsb, rb, row, sb, 16 + 32 * g + l) >> (4 * h)) & 0xF;
            const float d1 = d * (float)sc, m1 = dmin * (float)m;
            v = d1 * (float)q - m1;
        } else {
            const float d = h2f_bits(wu16(w, layout, type, nsb, rb, row, sb, 208));
            const int n = ee >> 7, s = (ee >> 5) & 3, l = ee & 31;
            const int lo = (wbyte(w, layout, type, nsb, rb, row, sb, 64 * n + 32 * (s & 1) + l) >> (s >= 2 ? 4 : 0)) & 0xF;
            const int hi = (wbyte(w, layout, type, nsb, rb, row, sb, 128 + 32 * n + l) >> (2 * s)) & 3;
            const int sc = (int8_t)wbyte(w, layout, type, nsb, rb, row, sb, 192 + (ee >> 4));
            v = (d * (float)sc) * (float)((lo | (hi << 4)) - 32);
        }
        dst[e] = v;
    }
}

// ---------------------------------------------------------------- synthetic blocks
__device__ inline uint64_t mix64(uint64_t z) {  // splitmix64 finaliser, qwen_cpu/qwen.cpp:314-319
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ULL;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebULL;
    return z ^ (z >> 31);
}
__device__ inline uint64_t sm_at(uint64_t seed, uint64_t i) { return mix64(seed + (i + 1) * 0x9e3779b97f4a7c15ULL); }
__device__ inline uint16_t f16_bits(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }

// One thread per output byte of the GGUF block stream; byte i of the fill (counted from block0) is
// handled by the launch whose window [off, off + nb) contains it.
__global__ __launch_bounds__(256) void k_synth(uint8_t* __restrict__ dst, int type, uint64_t seed, uint64_t block0,
                                               uint64_t off, uint64_t nb) {
    const uint64_t t = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= nb) return;
    const uint64_t i = off + t;
    const int bs = type == T_Q4_K ? Q4K_BYTES : Q6K_BYTES;
    const uint64_t blk = block0 + i / bs;
    const int p = (int)(i % bs);
    uint8_t v;
    if (type == T_Q4_K) {
        const uint64_t base = blk * 142;
        if (p < 4) {
            const uint64_t r = sm_at(seed, base + (p >> 1));
            const uint16_t h = f16_bits((float)(r >> 40) * (1.0f / 16777216.0f) * 0.01f);
            v = (uint8_t)(h >> (8 * (p & 1)));
        } else {
            v = (uint8_t)(sm_at(seed, base + 2 + (p - 4)) >> 56);
        }
    } else {
        const uint64_t base = blk * 209;
        if (p < 192) {
            v = (uint8_t)(sm_at(seed, base + p) >> 56);
        } else if (p < 208) {
            v = (uint8_t)(int8_t)((int)(sm_at(seed, base + p) % 64) - 32);
        } else {
            const uint64_t r = sm_at(seed, base + 208);
            const uint16_t h = f16_bits((float)(r >> 40) * (1.0f / 16777216.0f) * 0.005f);
            v = (uint8_t)(h >> (8 * (p & 1)));
        }
    }
    dst[i] = v;
}

}  // namespace

int launch_repack(const uint8_t* src, uint8_t* dst, int type, int k, int n, uint64_t rb, int dir, hipStream_t s) {
    dim3 grid(k / 256, n / 16);
    hipLaunchKernelGGL(k_repack, grid, dim3(256), 0, s, src, dst, type, k / 256, rb, dir);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_dequant(const uint8_t* w, int type, int layout, int k, uint64_t rb, const int32_t* rows, int nrows,
                   float* out, hipStream_t s) {
    hipLaunchKernelGGL(k_dequant, dim3(nrows), dim3(256), 0, s, w, type, layout, k, rb, rows, out);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_synth(uint8_t* dst, int type, uint64_t seed, uint64_t block0, uint64_t nblocks, hipStream_t s) {
    const uint64_t nbytes = nblocks * (type == T_Q4_K ? Q4K_BYTES : Q6K_BYTES);
    const uint64_t chunk = 1ull << 30;  // bytes per launch: 4M work-groups of 256 threads
    for (uint64_t off = 0; off < nbytes; off += chunk) {
        const uint64_t nb = nbytes - off < chunk ? nbytes - off : chunk;
        hipLaunchKernelGGL(k_synth, dim3((unsigned)((nb + 255) / 256)), dim3(256), 0, s, dst, type, seed, block0,
                           off, nb);
        if (hipGetLastError() != hipSuccess) return -1;
    }
    return 0;
}

}  // namespace qk
