// Weight-placement kernels: GGUF <-> T16 repack, bit-exact row dequant, synthetic block fill.
//
//   repack    plays the role of k_repack (qwen_cuda/kernels.cu:945-961) driven by repack_weights
//             (qwen_cuda/qwen.cpp:185-193), with the T16 group layout of qk_device.h.
//   dequant   is the selftest vehicle k_dq_* (qwen_cuda/kernels.cu:363-373, qwen_cuda/qwen.cpp:1317):
//             fp32 results identical to qwen_cpu/quants.h Ref::q8_0 / q4_k / q5_k / q6_k (:45-121).
//   embed     is k_embed_* (qwen_cuda/kernels.cu:375-389): token rows through the same expressions
//             (a run's block gathered into LDS, four elements per lane), or a caller's embedding row
//             under a mask.
#include "qk_device.h"
#include "qk_internal.h"

namespace qk {
namespace {

// One work-group per (tile, super-block) group; threads stride over the group's bytes.
// dir 0: GGUF -> T16 (gather), dir 1: T16 -> GGUF (scatter back).
__global__ __launch_bounds__(256) void k_repack(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst,
                                                int type, int nsb, uint64_t rb, int dir) {
    const int bs = sb_bytes(type);
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
    const int bs = sb_bytes(type);
    if (layout == LAYOUT_GGUF) return w[(uint64_t)row * rb + (uint64_t)sb * bs + p];
    const uint64_t g = ((uint64_t)(row >> 4) * nsb + sb) * (uint64_t)(16 * bs);
    return w[g + t16_dst(type, row & 15, p)];
}

__device__ inline uint32_t wu16(const uint8_t* w, int layout, int type, int nsb, uint64_t rb, int row, int sb, int p) {
    return (uint32_t)wbyte(w, layout, type, nsb, rb, row, sb, p) |
           ((uint32_t)wbyte(w, layout, type, nsb, rb, row, sb, p + 1) << 8);
}

// Element e of row `row`, with the reference's exact fp32 expression: Q8_0 q*d, Q4_K / Q5_K
// (d*sc)*q - dmin*m, Q6_K (d*sc)*(q-32).  All are single-rounding forms (products exact in fp32), so
// FMA contraction cannot change the bits.
__device__ inline float dq_elem(const uint8_t* __restrict__ w, int type, int layout, int nsb, uint64_t rb, int row,
                                int e) {
    const int sb = e >> 8, ee = e & 255;
    if (type == T_F32)  // rows as stored (qwen_cpu/quants.h:193-203); GGUF layout only
        return *(const float*)(w + (uint64_t)row * rb + 4 * (uint64_t)e);
    if (type == T_Q8_0) {  // qwen_cpu/quants.h:45-51
        const int j = ee >> 5;
        const float d = h2f_bits(wu16(w, layout, type, nsb, rb, row, sb, 34 * j));
        return (float)(int8_t)wbyte(w, layout, type, nsb, rb, row, sb, 34 * j + 2 + (ee & 31)) * d;
    }
    if (type == T_Q4_K || type == T_Q5_K) {  // qwen_cpu/quants.h:53-94
        const float d = h2f_bits(wu16(w, layout, type, nsb, rb, row, sb, 0));
        const float dmin = h2f_bits(wu16(w, layout, type, nsb, rb, row, sb, 2));
        uint8_t sc12[12];
        for (int i = 0; i < 12; i++) sc12[i] = wbyte(w, layout, type, nsb, rb, row, sb, 4 + i);
        const int g = ee >> 6, h = (ee >> 5) & 1, l = ee & 31;
        int sc, m;
        scale_min_k4(2 * g + h, sc12, sc, m);
        const int qs0 = type == T_Q5_K ? 48 : 16;
        int q = (wbyte(w, layout, type, nsb, rb, row, sb, qs0 + 32 * g + l) >> (4 * h)) & 0xF;
        if (type == T_Q5_K) q |= ((wbyte(w, layout, type, nsb, rb, row, sb, 16 + l) >> (2 * g + h)) & 1) << 4;
        const float d1 = d * (float)sc, m1 = dmin * (float)m;
        return d1 * (float)q - m1;
    }
    // Q6_K, qwen_cpu/quants.h:96-121
    const float d = h2f_bits(wu16(w, layout, type, nsb, rb, row, sb, 208));
    const int n = ee >> 7, s = (ee >> 5) & 3, l = ee & 31;
    const int lo = (wbyte(w, layout, type, nsb, rb, row, sb, 64 * n + 32 * (s & 1) + l) >> (s >= 2 ? 4 : 0)) & 0xF;
    const int hi = (wbyte(w, layout, type, nsb, rb, row, sb, 128 + 32 * n + l) >> (2 * s)) & 3;
    const int sc = (int8_t)wbyte(w, layout, type, nsb, rb, row, sb, 192 + (ee >> 4));
    return (d * (float)sc) * (float)((lo | (hi << 4)) - 32);
}

// One work-group per requested row, bit-exact with qwen_cpu/quants.h dequant_row.  A row index
// outside [0, n) writes a NaN row instead of reading outside the tensor.
__global__ __launch_bounds__(256) void k_dequant(const uint8_t* __restrict__ w, int type, int layout, int k, int n,
                                                 uint64_t rb, const int32_t* __restrict__ rows, float* __restrict__ out) {
    const int row = rows[blockIdx.x];
    const int nsb = k / 256;
    float* dst = out + (uint64_t)blockIdx.x * k;
    const bool ok = (unsigned)row < (unsigned)n;
    for (int e = threadIdx.x; e < k; e += blockDim.x) dst[e] = ok ? dq_elem(w, type, layout, nsb, rb, row, e) : __builtin_nanf("");
}

// Token embedding (the reference's k_embed_* , qwen_cuda/kernels.cu:375-389, 396, launched at
// qwen_cuda/qwen.cpp:265): x[t] = embd[t] where mask[t] is set (an embedding computed elsewhere, e.g.
// an image token), else row tokens[t] of the table, bit-exact; a token id outside [0, n) writes a NaN
// row instead of reading outside the table.  One wave per (256-column run sb, token t): the lanes
// gather the row's block of that run into LDS in GGUF byte order (every byte load independent of the
// others, so the run costs one memory round trip however the layout scatters it), then lane l
// decodes elements 4l .. 4l + 3 of the run, which share their scale (and for Q8_0 their block), with
// the expressions of dq_elem, and stores them as one 16-byte write.
__device__ inline f4 dq4_block(const uint8_t* blk, int type, int ee) {  // blk: LDS, GGUF block order
    f4 o;
    if (type == T_Q8_0) {  // qwen_cpu/quants.h:45-51
        const int j = ee >> 5;
        const float d = h2f_bits((uint32_t)blk[34 * j] | ((uint32_t)blk[34 * j + 1] << 8));
#pragma unroll
        for (int i = 0; i < 4; i++) o[i] = (float)(int8_t)blk[34 * j + 2 + (ee & 31) + i] * d;
    } else if (type == T_Q4_K || type == T_Q5_K) {  // qwen_cpu/quants.h:53-94
        const float d = h2f_bits((uint32_t)blk[0] | ((uint32_t)blk[1] << 8));
        const float dmin = h2f_bits((uint32_t)blk[2] | ((uint32_t)blk[3] << 8));
        const int g = ee >> 6, h = (ee >> 5) & 1, l = ee & 31;
        int sc, m;
        scale_min_k4(2 * g + h, blk + 4, sc, m);
        const int qs0 = type == T_Q5_K ? 48 : 16;
        const float d1 = d * (float)sc, m1 = dmin * (float)m;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            int q = (blk[qs0 + 32 * g + l + i] >> (4 * h)) & 0xF;
            if (type == T_Q5_K) q |= ((blk[16 + l + i] >> (2 * g + h)) & 1) << 4;
            o[i] = d1 * (float)q - m1;
        }
    } else {  // Q6_K, qwen_cpu/quants.h:96-121
        const float d = h2f_bits((uint32_t)blk[208] | ((uint32_t)blk[209] << 8));
        const int n = ee >> 7, s = (ee >> 5) & 3, l = ee & 31;
        const int sc = (int8_t)blk[192 + (ee >> 4)];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int lo = (blk[64 * n + 32 * (s & 1) + l + i] >> (s >= 2 ? 4 : 0)) & 0xF;
            const int hi = (blk[128 + 32 * n + l + i] >> (2 * s)) & 3;
            o[i] = (d * (float)sc) * (float)((lo | (hi << 4)) - 32);
        }
    }
    return o;
}

__global__ __launch_bounds__(64) void k_embed(const uint8_t* __restrict__ w, int type, int layout, int k, int n,
                                              uint64_t rb, const int32_t* __restrict__ tokens,
                                              const uint8_t* __restrict__ mask, const float* __restrict__ embd,
                                              float* __restrict__ x) {
    __shared__ __align__(16) uint8_t blk[Q8_COL_BYTES];
    const int sb = blockIdx.x, t = blockIdx.y, lane = threadIdx.x, nsb = k / 256;
    const size_t e0 = (size_t)t * k + 256 * (size_t)sb + 4 * lane;  // this lane's four outputs
    if (mask && mask[t]) {
        *(f4*)(x + e0) = *(const f4*)(embd + e0);
        return;
    }
    const int row = tokens[t];
    if ((unsigned)row >= (unsigned)n) {
        const float q = __builtin_nanf("");
        *(f4*)(x + e0) = f4{q, q, q, q};
        return;
    }
    if (type == T_F32) {  // rows as stored (qwen_cpu/quants.h:193-203); GGUF layout only
        *(f4*)(x + e0) = *(const f4*)(w + (uint64_t)row * rb + 4 * (256 * (uint64_t)sb + 4 * lane));
        return;
    }
    const int bs = sb_bytes(type);
    const uint8_t* base = layout == LAYOUT_GGUF ? w + (uint64_t)row * rb + (uint64_t)sb * bs
                                                : w + ((uint64_t)(row >> 4) * nsb + sb) * (uint64_t)(16 * bs);
    uint8_t v[8];
#pragma unroll
    for (int i = 0; i < 8; i++) {  // bytes 4 lane + i and 256 + 4 lane + i - 4 of the block
        const int p = i < 4 ? 4 * lane + i : 256 + 4 * lane + i - 4;
        v[i] = p < bs ? base[layout == LAYOUT_GGUF ? p : t16_dst(type, row & 15, p)] : 0;
    }
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const int p = i < 4 ? 4 * lane + i : 256 + 4 * lane + i - 4;
        if (p < bs) blk[p] = v[i];
    }
    __syncthreads();
    *(f4*)(x + e0) = dq4_block(blk, type, 4 * lane);
}

// ---------------------------------------------------------------- synthetic blocks
__device__ inline uint64_t mix64(uint64_t z) {  // splitmix64 finaliser, qwen_cpu/qwen.cpp:314-319
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ULL;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebULL;
    return z ^ (z >> 31);
}
__device__ inline uint64_t sm_at(uint64_t seed, uint64_t i) { return mix64(seed + (i + 1) * 0x9e3779b97f4a7c15ULL); }
// fp16 bits of 0 <= f < 65504, rounded to nearest even in integer arithmetic: the device's float ->
// half conversion was measured to round a few fp16-subnormal results (about 1 in 2000 of the
// generator's d values) to the other neighbour.  Normal results have unit 2^(e-10), subnormal ones
// 2^-24; a carry out of the mantissa moves to the next binade by itself.
__device__ inline uint16_t f16_bits(float f) {
    const uint32_t x = __builtin_bit_cast(uint32_t, f);
    const int e = (int)(x >> 23) - 127;
    if (e < -25) return 0;
    const uint32_t mant = (x & 0x7FFFFFu) | 0x800000u;
    const int shift = e >= -14 ? 13 : -e - 1;  // 13 .. 24
    uint32_t q = mant >> shift;
    const uint32_t rem = mant & ((1u << shift) - 1), half = 1u << (shift - 1);
    if (rem > half || (rem == half && (q & 1))) q++;
    return e >= -14 ? (uint16_t)(((uint32_t)(e + 15) << 10) + q - 1024) : (uint16_t)q;
}

// One thread per output byte of the GGUF block stream; byte i of the fill (counted from block0) is
// handled by the launch whose window [off, off + nb) contains it.
__global__ __launch_bounds__(256) void k_synth(uint8_t* __restrict__ dst, int type, uint64_t seed, uint64_t block0,
                                               uint64_t off, uint64_t nb) {
    const uint64_t t = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= nb) return;
    const uint64_t i = off + t;
    const int bs = sb_bytes(type);
    const uint64_t blk = block0 + i / bs;
    const int p = (int)(i % bs);
    uint8_t v;
    if (type == T_Q8_0) {  // per 34-byte block j of the run: d = fp16_rne(u24 * 0.01f), then qs[32]
        const int j = p / 34, pb = p - 34 * j;
        const uint64_t base = (blk * 8 + j) * 33;
        if (pb < 2) {
            const uint16_t h = f16_bits((float)(sm_at(seed, base) >> 40) * (1.0f / 16777216.0f) * 0.01f);
            v = (uint8_t)(h >> (8 * pb));
        } else {
            v = (uint8_t)(sm_at(seed, base + 1 + (pb - 2)) >> 56);
        }
    } else if (type == T_Q5_K) {  // d, dmin = fp16_rne(u24 * 0.01f), then scales, qh, qs bytes
        const uint64_t base = blk * 174;
        if (p < 4) {
            const uint64_t r = sm_at(seed, base + (p >> 1));
            const uint16_t h = f16_bits((float)(r >> 40) * (1.0f / 16777216.0f) * 0.01f);
            v = (uint8_t)(h >> (8 * (p & 1)));
        } else {
            v = (uint8_t)(sm_at(seed, base + 2 + (p - 4)) >> 56);
        }
    } else if (type == T_Q4_K) {
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

int launch_dequant(const uint8_t* w, int type, int layout, int k, int n, uint64_t rb, const int32_t* rows, int nrows,
                   float* out, hipStream_t s) {
    hipLaunchKernelGGL(k_dequant, dim3(nrows), dim3(256), 0, s, w, type, layout, k, n, rb, rows, out);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_embed(const uint8_t* w, int type, int layout, int k, int n, uint64_t rb, const int32_t* tokens,
                 const uint8_t* mask, const float* embd, int m, float* x, hipStream_t s) {
    constexpr int MAXY = 65535;  // tokens per launch (the grid's second dimension)
    for (int t0 = 0; t0 < m; t0 += MAXY) {
        const int mt = m - t0 < MAXY ? m - t0 : MAXY;
        hipLaunchKernelGGL(k_embed, dim3(k / 256, mt), dim3(64), 0, s, w, type, layout, k, n, rb, tokens + t0,
                           mask ? mask + t0 : nullptr, embd ? embd + (size_t)t0 * k : nullptr, x + (size_t)t0 * k);
        if (hipGetLastError() != hipSuccess) return -1;
    }
    return 0;
}

int launch_synth(uint8_t* dst, int type, uint64_t seed, uint64_t block0, uint64_t nblocks, hipStream_t s) {
    const uint64_t nbytes = nblocks * sb_bytes(type);
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
