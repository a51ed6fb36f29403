// Device-side building blocks shared by the layout, GEMV and GEMM kernels (gfx950 / CDNA4 only).
//
// Block formats follow GGUF (qwen_cpu/quants.h:13-17, docs/model.md:263-318):
//   Q8_0  34 B: u16 d, i8 qs[32]                                      (32 weights; 8 per 256 columns)
//   Q4_K 144 B: u16 d, u16 dmin, u8 scales[12], u8 qs[128]          (8 sub-blocks x 32)
//   Q5_K 176 B: u16 d, u16 dmin, u8 scales[12], u8 qh[32], u8 qs[128] (8 sub-blocks x 32)
//   Q6_K 210 B: u8 ql[128], u8 qh[64], i8 scales[16], u16 d           (16 sub-blocks x 16)
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

namespace qk {

// Compile-time loop: f(std::integral_constant<int, i>) for i = 0 .. N-1.
template <int I, int N, typename F>
__device__ inline void static_for_impl(F&& f) {
    if constexpr (I < N) {
        f(std::integral_constant<int, I>{});
        static_for_impl<I + 1, N>(f);
    }
}
template <int N, typename F>
__device__ inline void static_for(F&& f) {
    static_for_impl<0, N>(f);
}

constexpr int T_F32 = 0, T_Q8_0 = 8, T_Q4_K = 12, T_Q5_K = 13, T_Q6_K = 14;
constexpr int LAYOUT_GGUF = 0, LAYOUT_T16 = 1;
constexpr int Q4K_BYTES = 144, Q5K_BYTES = 176, Q6K_BYTES = 210;
constexpr int Q8_COL_BYTES = 272;          // Q8_0: the eight 34-byte blocks of one 256-column run
constexpr int Q4K_GROUP = 16 * Q4K_BYTES;  // one T16 group: 16 rows x one super-block = 2304 B
constexpr int Q5K_GROUP = 16 * Q5K_BYTES;  // 2816 B
constexpr int Q6K_GROUP = 16 * Q6K_BYTES;  // 3360 B
constexpr int Q8_GROUP = 16 * Q8_COL_BYTES;  // 4352 B

// Bytes of one row's 256-column run (a "super-block column"; for Q8_0 eight blocks) and of one T16
// group of 16 such runs.
__host__ __device__ constexpr int sb_bytes(int type) {
    return type == T_Q4_K ? Q4K_BYTES : type == T_Q5_K ? Q5K_BYTES : type == T_Q6_K ? Q6K_BYTES : Q8_COL_BYTES;
}
__host__ __device__ constexpr int group_bytes(int type) { return 16 * sb_bytes(type); }

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));
typedef uint32_t u2 __attribute__((ext_vector_type(2)));

// ------------------------------------------------------------------------------------------------
// T16 layout.  A weight with n % 16 == 0 is cut into n/16 tiles of 16 rows; tile t occupies the
// same byte range as GGUF rows 16t..16t+15 and holds one group per super-block column sb, at
// ((t * nsb) + sb) * group_bytes.  Inside a group (l = lane 0..63, r = l & 15, g = l >> 4):
//
// Q4_K group (2304 B):
//   [0, 2048)     qs plane: byte 1024*i + 16*l + b  = qs_r[32*g + 16*i + b]   (i in {0,1})
//   [2048, 2112)  d/dmin:   byte 2048 + 4*r + p     = block_r byte p (p < 4)
//   [2112, 2304)  scales:   byte 2112 + 12*r + p    = scales_r[p]
// Q5_K group (2816 B): the Q4_K group (qs plane, d/dmin, scales at the same offsets), then
//   [2304, 2816)  qh plane: byte 2304 + 256*i + 16*r + b = qh_r[16*i + b]   (i in {0,1})
// Q8_0 group (4352 B), element e of the run = block e/32, qs byte e%32:
//   [0, 4096)     qs plane: byte 1024*t + 16*l + b  = element 64*t + 16*g + b of row r
//   [4096, 4352)  d:        byte 4096 + 16*r + 8*(j&1) + 2*(j>>1) + p = byte p of block j's d
// Q6_K group (3360 B):
//   [0, 2048)     ql plane: byte 1024*n + 16*l + b  = ql_r[64*n + 32*(g>>1) + 16*(g&1) + b]
//   [2048, 3072)  qh plane: byte 2048 + 512*n + 16*(r + 16*h) + b = qh_r[32*n + 16*h + b]
//   [3072, 3328)  scales:   byte 3072 + 128*n + 32*G + 4*u + i   = scales_{4G+i}[8*n + u]
//   [3328, 3360)  d:        byte 3328 + 2*r + p     = d_r byte p
// so every 64-lane 16-byte load of the GEMV/GEMM reads one contiguous run, and the per-lane
// scale/d reads of the MFMA accumulator layout (rows 4G..4G+3 of a lane) are single loads.
//
// t16_src(type, o, r, p): group byte o comes from byte p of row r's GGUF block.  Used by the
// repack (gather) and unrepack (scatter) kernels and by the dequant kernel's T16 reads.
__host__ __device__ inline void t16_src(int type, int o, int& r, int& p) {
    if (type == T_Q5_K && o >= 2304) {  // qh plane; the rest is the Q4_K group with qs 32 bytes later
        const int q = o - 2304, i = q >> 8;
        r = (q >> 4) & 15;
        p = 16 + 16 * i + (q & 15);
        return;
    }
    if (type == T_Q8_0) {
        if (o < 4096) {
            const int t = o >> 10, l = (o >> 4) & 63, b = o & 15, e = 64 * t + 16 * (l >> 4) + b;
            r = l & 15;
            p = 34 * (e >> 5) + 2 + (e & 31);
        } else {
            const int q = o - 4096, j = 2 * ((q >> 1) & 3) + ((q >> 3) & 1);
            r = q >> 4;
            p = 34 * j + (q & 1);
        }
        return;
    }
    if (type == T_Q4_K || type == T_Q5_K) {
        const int qs0 = type == T_Q5_K ? 48 : 16;  // first qs byte of the GGUF block
        if (o < 2048) {
            const int i = o >> 10, l = (o >> 4) & 63, b = o & 15;
            r = l & 15;
            p = qs0 + 32 * (l >> 4) + 16 * i + b;
        } else if (o < 2112) {
            r = (o - 2048) >> 2;
            p = (o - 2048) & 3;
        } else {
            const int q = o - 2112;
            r = q / 12;
            p = 4 + q % 12;
        }
    } else {  // Q6_K
        if (o < 2048) {
            const int n = o >> 10, l = (o >> 4) & 63, b = o & 15, g = l >> 4;
            r = l & 15;
            p = 64 * n + 32 * (g >> 1) + 16 * (g & 1) + b;
        } else if (o < 3072) {
            const int q = o - 2048, n = q >> 9, rr = (q >> 4) & 31, b = q & 15;
            r = rr & 15;
            p = 128 + 32 * n + 16 * (rr >> 4) + b;
        } else if (o < 3328) {
            const int q = o - 3072, n = q >> 7, G = (q >> 5) & 3, u = (q >> 2) & 7, i = q & 3;
            r = 4 * G + i;
            p = 192 + 8 * n + u;
        } else {
            const int q = o - 3328;
            r = q >> 1;
            p = 208 + (q & 1);
        }
    }
}

// Inverse of t16_src: offset inside the group of (row r, GGUF block byte p).
__host__ __device__ inline int t16_dst(int type, int r, int p) {
    if (type == T_Q8_0) {
        const int j = p / 34, pb = p - 34 * j;
        if (pb < 2) return 4096 + 16 * r + 8 * (j & 1) + 2 * (j >> 1) + pb;
        const int e = 32 * j + pb - 2, t = e >> 6, g = (e >> 4) & 3, b = e & 15;
        return 1024 * t + 16 * (16 * g + r) + b;
    }
    if (type == T_Q4_K || type == T_Q5_K) {
        if (p < 4) return 2048 + 4 * r + p;
        if (p < 16) return 2112 + 12 * r + (p - 4);
        if (type == T_Q5_K && p < 48) {
            const int q = p - 16;
            return 2304 + 256 * (q >> 4) + 16 * r + (q & 15);
        }
        const int q = p - (type == T_Q5_K ? 48 : 16), g = q >> 5, i = (q >> 4) & 1, b = q & 15;
        return 1024 * i + 16 * (16 * g + r) + b;
    }
    if (p < 128) {
        const int n = p >> 6, pp = p & 63, g = 2 * (pp >> 5) + ((pp >> 4) & 1), b = pp & 15;
        return 1024 * n + 16 * (16 * g + r) + b;
    }
    if (p < 192) {
        const int q = p - 128, n = q >> 5, h = (q >> 4) & 1, b = q & 15;
        return 2048 + 512 * n + 16 * (r + 16 * h) + b;
    }
    if (p < 208) {
        const int j = p - 192, n = j >> 3, u = j & 7;
        return 3072 + 128 * n + 32 * (r >> 2) + 4 * u + (r & 3);
    }
    return 3328 + 2 * r + (p - 208);
}

// ------------------------------------------------------------------------------------------------
// Scalar helpers.
__device__ inline float h2f_bits(uint32_t h16) {  // exact fp16 -> fp32 (subnormals included)
    return (float)__builtin_bit_cast(_Float16, (uint16_t)h16);
}

// 6-bit scale/min of sub-block j from the 12 packed bytes (qwen_cpu/quants.h:33-41).
__device__ inline void scale_min_k4(int j, const uint8_t* q, int& sc, int& m) {
    if (j < 4) {
        sc = q[j] & 63;
        m = q[j + 4] & 63;
    } else {
        sc = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
        m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
    }
}

// ------------------------------------------------------------------------------------------------
// Packed-fp16 helpers for building MFMA operands.
//
// perm_lo/hi: bytes b0..b3 of v (each < 256 after masking) -> two fp16 lanes 1024 + b, exactly:
// 0x64 in the high byte is the fp16 exponent of 1024, whose mantissa unit is 1.
__device__ inline uint32_t perm_lo(uint32_t v) { return __builtin_amdgcn_perm(0x64646464u, v, 0x04010400u); }
__device__ inline uint32_t perm_hi(uint32_t v) { return __builtin_amdgcn_perm(0x64646464u, v, 0x04030402u); }

__device__ inline h2 as_h2(uint32_t v) { return __builtin_bit_cast(h2, v); }
__device__ inline uint32_t as_u32(h2 v) { return __builtin_bit_cast(uint32_t, v); }

__device__ inline uint32_t pk_fma(uint32_t a, h2 b, h2 c) {  // one rounding per lane
    return as_u32(__builtin_elementwise_fma(as_h2(a), b, c));
}

__device__ inline h8 make_h8(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
    return __builtin_bit_cast(h8, u4{a, b, c, d});
}

// D(16x16 f32) += A(16x32 f16) * B(32x16 f16).  Lane l holds A[l&15][8*(l>>4) .. +7],
// B[8*(l>>4) .. +7][l&15] and D[4*(l>>4) + i][l&15], i = 0..3.
__device__ inline f4 mfma(const h8& a, const h8& b, const f4& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// Split fp32 x into fp16 hi + lo with x == hi + lo to ~2^-22 relative (hi = rne(x),
// lo = rne(x - hi); x - hi is exact in fp32).  Valid for |x| < 65504.
__device__ inline void split_h(float x, _Float16& hi, _Float16& lo) {
    hi = (_Float16)x;
    lo = (_Float16)(x - (float)hi);
}

// Cross-lane moves inside rows of 16 lanes on the VALU (DPP), no LDS round trip:
//   xor1 / xor2: quad_perm [1,0,3,2] / [2,3,0,1]; mirror8: lane i <-> 7-i of each 8 (row_half_mirror);
//   mirror16: lane i <-> 15-i of each 16 (row_mirror); down8: lane i <- i+8 within the row (row_shl:8,
//   lanes 8..15 read 0).
__device__ inline float dpp_xor1(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));
}
__device__ inline float dpp_xor2(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false));
}
__device__ inline float dpp_mirror8(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x141, 0xF, 0xF, false));
}
__device__ inline float dpp_mirror16(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x140, 0xF, 0xF, false));
}
__device__ inline float dpp_down8(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x108, 0xF, 0xF, true));
}
// Sums over aligned groups of 2 / 4 / 8 / 16 lanes (every lane of the group gets the sum).
__device__ inline float sum2(float v) { return v + dpp_xor1(v); }
__device__ inline float sum4(float v) { v = sum2(v); return v + dpp_xor2(v); }
__device__ inline float sum8(float v) { v = sum4(v); return v + dpp_mirror8(v); }
__device__ inline float sum16(float v) { v = sum8(v); return v + dpp_mirror16(v); }

__device__ inline u4 ld16(const void* p) { return *(const u4*)p; }
__device__ inline u2 ld8(const void* p) { return *(const u2*)p; }
__device__ inline uint32_t ld4(const void* p) { return *(const uint32_t*)p; }

// ------------------------------------------------------------------------------------------------
// Activation formats at the boundary.  ACT_F32: fp32 [m][k] (the CPU path's, qwen_cpu/ops.h:54-76).
// ACT_F16: fp16 [m][k], the reference GPU path's (qwen_cuda/kernels.cu:307-361 GEMM input).
// ACT_F16_XPERM: fp16 with each 1024-element run of a row permuted as the reference's decode GEMV
// reads it (qwen_cuda/kernels.cu:27-28): element 256 s + 32 j + 8 c + e (s, c < 4, j, e < 8) of a run
// sits at 256 c + 8 (8 s + j) + e.  The same permutation places the gate/up pair's fp16 output when
// the reference writes it for the down projection (kernels.cu:419-426).
enum { ACT_F32 = 0, ACT_F16 = 1, ACT_F16_XPERM = 2 };
__host__ __device__ inline int xperm_pos(int i) {
    return (i & ~1023) | (((i >> 3) & 3) << 8) | (((i >> 8) & 3) << 6) | (((i >> 5) & 7) << 3) | (i & 7);
}
// Four consecutive activations of token t, elements e .. e + 3 (e % 4 == 0) of a row of ld elements,
// as fp32 (fp16 widens exactly; xperm keeps any 4-aligned run of 4 contiguous).
__device__ inline f4 load_act4(const void* x, int fmt, size_t ld, int t, int e) {
    if (fmt == ACT_F32) return *(const f4*)((const float*)x + (size_t)t * ld + e);
    const int pos = fmt == ACT_F16_XPERM ? xperm_pos(e) : e;
    const u2 h = *(const u2*)((const _Float16*)x + (size_t)t * ld + pos);
    return f4{h2f_bits(h.x & 0xFFFFu), h2f_bits(h.x >> 16), h2f_bits(h.y & 0xFFFFu), h2f_bits(h.y >> 16)};
}
// Stores one output: fp32, or fp16 (round to nearest even) at the plain or xperm position.
__device__ inline void store_act(void* y, int fmt, size_t ld, int t, int row, float v) {
    if (fmt == ACT_F32) {
        ((float*)y)[(size_t)t * ld + row] = v;
        return;
    }
    ((_Float16*)y)[(size_t)t * ld + (fmt == ACT_F16_XPERM ? xperm_pos(row) : row)] = (_Float16)v;
}

}  // namespace qk
