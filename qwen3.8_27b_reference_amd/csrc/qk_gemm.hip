// Prefill GEMM (m >= 5 through qk_matmul and grouped launches) for Q8_0 / Q4_K / Q5_K / Q6_K weights: super-blocks dequantized to fp16
// feeding CDNA4 MFMA (v_mfma_f32_32x32x16_f16), fp32 accumulate.
//
// Replaces the reference's k_gemm_q4k / k_gemm_q6k (qwen_cuda/kernels.cu:307-361, 394, 397-401:
// 64x64x64 tiles, 2x2 warps of mma.m16n8k16, dequant via dq8h into shared memory) with a design
// for 256-CU CDNA4:
//
//  * The 32x32x16 MFMA: on MI355X it runs at about twice the rate of 16x16x32 (measured
//    ~2.07 vs ~1.19 PFLOP/s fp16).  Its 32 A rows are a pair of T16 tiles.
//  * A work-group owns P tile pairs x 128 tokens; P is chosen per shape so that the work-groups
//    fill whole rounds of CUs (N=17408, M=512: 544 pairs = 60 x 9 + 4, 61 x 4 token blocks =
//    244 work-groups on 256 CUs).
//  * Eight waves, two per SIMD.  Compute waves 0..3 each own P/4 pairs for all 128 tokens; DMA
//    waves 4..7 issue the weight LDS-DMAs (their issue stalls then never hold up an MFMA) and
//    multiply the P%4 remaining pairs, one 32-token block each.  The compute waves issue the
//    activation LDS-DMAs just before their barrier, where they would wait anyway.  A compute wave
//    keeps 4 x P/4 accumulator tiles in 256 registers, the occupancy of two waves per SIMD.
//  * K advances 64 elements (a quarter super-block) per step; LDS holds up to four stages.  The
//    compute waves pipeline over K/16 chunks: while chunk c's MFMAs run, they read chunk c+1's
//    activations from LDS and dequantize chunk c+1's A fragments in registers (the reference's
//    tolerance path, kernels.cu:127-181: scales rounded to fp16, one packed FMA per pair of
//    weights), so the dequantized weights never travel through LDS.  One barrier per step.
//  * x is read as fp16 [m][k] where it lies when the caller passes fp16, as the reference's GEMM
//    takes it (no prepass), also in the xperm layout its decode path feeds for m < 16; fp32 x is
//    first rounded to fp16 by k_gemm_cvt_x.  Each LDS-DMA of activations moves eight tokens'
//    16-byte k-pieces (whole 128-byte lines in the plain layout) into B-operand order.
//  * y is fp32 [m][n] row-major like the reference's GEMM output (y[tok*n + row]).
#include <atomic>

#include "qk_device.h"
#include "qk_internal.h"

namespace qk {
namespace {

#define LDS_AS __attribute__((address_space(3)))

typedef float f16v __attribute__((ext_vector_type(16)));

constexpr int THREADS = 512;  // 4 compute waves + 4 DMA waves (one of each per SIMD)
constexpr int GEMM_MATS = 4;   // matrices of one grouped launch (the reference's gemv groups hold <= 4)
constexpr int MAX_STAGES = 4;

template <int N>
__device__ inline void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

template <int N>
__device__ inline void wait_vm_le(int n) {  // wait until at most n (<= N) operations are in flight
    if constexpr (N > 0) {
        if (n >= N) {
            wait_vm<N>();
            return;
        }
        wait_vm_le<N - 1>(n);
    } else {
        wait_vm<0>();
    }
}

__device__ inline uint32_t lds_addr(const void* p) { return (uint32_t)(uintptr_t)(LDS_AS const void*)p; }

// 16 bytes per lane from global memory into LDS (M0 + 16 * lane), from inline assembly: the
// compiler then holds no pending LDS-DMA, which it would wait out (vmcnt(0)) before LDS accesses it
// cannot prove disjoint from the destination.  Every read of DMA'd bytes follows wait_vm* and a
// barrier.  s_nop: M0 written by the SALU needs one wait state before an LDS-DMA reads it.
__device__ inline void dma16(const void* g, uint8_t* lds) {
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "{m0}"(lds_addr(lds)) : "memory");
}

// Work-group barrier that waits only for this wave's LDS operations: the release fence of
// __syncthreads() would also wait for every LDS-DMA in flight, i.e. for the prefetched stages.
__device__ inline void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// D(32x32 f32) += A(32x16 f16) * B(16x32 f16).  Lane l holds A[l & 31][8*(l >> 5) .. +7],
// B[8*(l >> 5) .. +7][l & 31] and D[8*(v/4) + 4*(l >> 5) + v%4][l & 31] in register v (checked
// on the device against a host product).
__device__ inline f16v mfma32(const h8& a, const h8& b, const f16v& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// ------------------------------------------------------------------------------------------------
// Activations.  The GEMM reads x as fp16 [m][k], row-major, as the reference's GEMM takes it
// (qwen_cuda/qwen.cpp:246): fp16 x straight from the caller, fp32 x after k_gemm_cvt_x has rounded
// it to nearest even into the workspace.  A step's 64 k of one token are one aligned 128-byte line,
// and one LDS-DMA (64 lanes x 16 bytes) moves eight tokens' lines of a 32-token block: DMA j of the
// block takes tokens 8j .. 8j + 7, lane i the 16 bytes of token 8j + (i & 7) that hold its k-piece
// p = 2 (i >> 4) + (((i >> 3) & 1) ^ (j & 1)) (eight halves, k = 8p .. 8p + 7 of the step).  The
// B operand of chunk c (k 16c .. 16c + 15) for lane l (token t = l & 31, half h = l >> 5) is then at
// 1024 (t >> 3) + 128 (h ^ ((t >> 3) & 1)) + 16 (t & 7) + 256 c of the block's 4 KiB: the chunk is an
// immediate offset, and the 16 lanes of each 256-byte LDS cycle read 16 different 16-byte bank groups.
__global__ __launch_bounds__(256) void k_gemm_cvt_x(const float* __restrict__ x, size_t n8, u4* __restrict__ xh) {
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n8; i += (size_t)gridDim.x * 256) {
        const f4 a = *(const f4*)(x + 8 * i), b = *(const f4*)(x + 8 * i + 4);
        const h2 p0 = {(_Float16)a.x, (_Float16)a.y}, p1 = {(_Float16)a.z, (_Float16)a.w};
        const h2 p2 = {(_Float16)b.x, (_Float16)b.y}, p3 = {(_Float16)b.z, (_Float16)b.w};
        xh[i] = u4{as_u32(p0), as_u32(p1), as_u32(p2), as_u32(p3)};
    }
}

// Byte offset of lane l's B operand (chunk 0) inside a 32-token block's 4 KiB of one stage.
__device__ inline int xb_lane_off(int lane) {
    const int t = lane & 31, h = lane >> 5, j = t >> 3;
    return 1024 * j + 128 * (h ^ (j & 1)) + 16 * (t & 7);
}


// ------------------------------------------------------------------------------------------------
// Raw bytes of one step (quarter q of super-block sb) of one tile, staged in LDS by LDS-DMA as
// 256-byte pieces.
//   Q4_K: piece 0/1 = the two 256-byte qs runs of the quarter (T16 bytes 1024i + 256q ..); the
//         scale piece = d/dmin (offset 0) and scales (offset 64) (T16 bytes 2048..2303), once per
//         super-block.
//   Q6_K: pieces 0..3 = ql half-plane n = q/2 (T16 1024n ..), 4..5 = qh plane n (2048 + 512n ..),
//         piece 6 = scales of half n (offset 0, T16 3072 + 128n) and d (offset 128, T16 3328).
//   Q5_K: the Q4_K pieces; three scale pieces per super-block (T16 bytes 2048..2815: d/dmin and
//         scales, then the two 256-byte halves of the qh plane).
//   Q8_0: pieces 0..3 = the quarter's 1 KiB of quants (T16 1024q + 256c: chunk c); the scale piece
//         = the d plane (T16 4096..4351), once per super-block.
constexpr int Q6_PIECES = 7;

// Per type: raw pieces per tile and step, scale pieces per tile (loaded at quarter 0), the T16
// offset of the first scale piece and the group-byte stride of one quarter step.
template <int TYPE>
struct GT {
    static constexpr int RP = TYPE == T_Q6_K ? Q6_PIECES : TYPE == T_Q8_0 ? 4 : 2;
    static constexpr int SP = TYPE == T_Q6_K ? 0 : TYPE == T_Q5_K ? 3 : 1;
    static constexpr int SOFF = TYPE == T_Q8_0 ? 4096 : 2048;
    static constexpr int QSTEP = TYPE == T_Q6_K ? 0 : TYPE == T_Q8_0 ? 1024 : 256;
};

// Q6_K piece j, lane li: source offset in the group = off + (q >> 1) * nstr.
__device__ inline void q6_piece_base(int j, int li, uint32_t& off, uint32_t& nstr) {
    if (j < 4) {
        off = 256 * j + 16 * li;
        nstr = 1024;
    } else if (j < 6) {
        off = 2048 + 256 * (j - 4) + 16 * li;
        nstr = 512;
    } else if (li < 8) {
        off = 3072 + 16 * li;
        nstr = 128;
    } else {
        off = 3328 + 16 * (li & 1);  // lanes 10..15 repeat d
        nstr = 0;
    }
}

// Per super-block, per lane (row r): the eight 6-bit scales and mins as bytes (6-bit unpack as in
// qwen_cpu/quants.h:33-41, bytewise on whole dwords) and (d, -dmin).  q4_dm gives sub-block j's
// (half(d*sc_j), half(-dmin*m_j)): fp16 products of exact fp16 factors round once, as the
// reference's half(d * sc) does (kernels.cu:127-181).
struct Q4Scales {
    uint32_t S[2], M[2];  // byte j & 3 of word j >> 2: sc_j / m_j
    uint32_t dmn;         // h2 (d, -dmin)
};

__device__ inline Q4Scales q4_scales(const uint8_t* S, int r) {  // S: the tile's scale piece
    const uint32_t dd = ld4(S + 4 * r);
    const uint32_t s0 = ld4(S + 64 + 12 * r), s1 = ld4(S + 68 + 12 * r), s2 = ld4(S + 72 + 12 * r);
    Q4Scales o;
    o.S[0] = s0 & 0x3F3F3F3Fu;
    o.M[0] = s1 & 0x3F3F3F3Fu;
    o.S[1] = (s2 & 0x0F0F0F0Fu) | ((s0 >> 2) & 0x30303030u);
    o.M[1] = ((s2 >> 4) & 0x0F0F0F0Fu) | ((s1 >> 2) & 0x30303030u);
    o.dmn = as_u32(h2{__builtin_bit_cast(_Float16, (uint16_t)(dd & 0xFFFFu)),
                      (_Float16)-__builtin_bit_cast(_Float16, (uint16_t)(dd >> 16))});
    return o;
}

__device__ inline uint32_t q4_dm(const Q4Scales& sc, int j) {
    const int b = j & 3;
    // bytes (sc_j, 0, m_j, 0) under the fp16 exponent of 1024: (1024 + sc, 1024 + m), exact
    const uint32_t sel = (uint32_t)b | 0x0C000C00u | ((uint32_t)(b + 4) << 16);
    const bool hi = j >= 4;  // a select, not an index: j may be a run-time value
    const uint32_t packed = __builtin_amdgcn_perm(hi ? sc.M[1] : sc.M[0], hi ? sc.S[1] : sc.S[0], sel) | 0x64006400u;
    return as_u32((as_h2(packed) + h2{(_Float16)-1024.0f, (_Float16)-1024.0f}) * as_h2(sc.dmn));
}

// A fragments of one tile pair for quarter q: lane l = 32h + 16u + r (row 16u + r of the pair,
// K half h) gets W[row][16c + 8h + 0..7] for the four K/16 chunks c of the quarter.  The raw words
// are read from LDS first (*_src), the fragment of each chunk is built on its own (*_frag) so that
// a wave can build the next pair's chunks between the MFMAs of the current pair.
//   Q4_K: chunks 0,1 = low nibbles of qs_r[32q + 16c + 8h ..] (sub-block 2q), chunks 2,3 = high
//   nibbles of the same bytes (sub-block 2q+1) (qwen_cpu/quants.h:53-71 element order).
struct Q4Src {
    u2 lo, hi;  // qs_r[32q + 8h + 0..7], qs_r[32q + 16 + 8h + 0..7]
};

__device__ inline Q4Src q4_src(const uint8_t* R) {  // R: the tile's piece 0 + 16 r + 8 h
    return Q4Src{ld8(R), ld8(R + 256)};
}

// Bytes 0,1 (lo) or 2,3 (hi) of v, each below 16, as an exact fp16 pair: read as FP8 E4M3 a byte
// b < 16 is b * 2^-9 (subnormal for b < 8), so the scaled conversion by 2^9 gives b exactly
// (checked for all 16 values on the device).  One instruction for the byte-perm + 1024 subtract.
__device__ inline uint32_t nib_pair_lo(uint32_t v) {
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(v, 512.0f, false));
}
__device__ inline uint32_t nib_pair_hi(uint32_t v) {
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(v, 512.0f, true));
}

__device__ inline h8 q4_frag(const Q4Src& S4, uint32_t dm, int c) {  // dm: q4_dm of the chunk's sub-block
    const h2 v = as_h2(dm);
    const h2 vds = {v.x, v.x}, vdm = {v.y, v.y};
    const u2 src = (c & 1) ? S4.hi : S4.lo;
    const uint32_t n0 = (c >> 1) ? (src.x >> 4) & 0x0F0F0F0Fu : src.x & 0x0F0F0F0Fu;
    const uint32_t n1 = (c >> 1) ? (src.y >> 4) & 0x0F0F0F0Fu : src.y & 0x0F0F0F0Fu;
    return make_h8(pk_fma(nib_pair_lo(n0), vds, vdm), pk_fma(nib_pair_hi(n0), vds, vdm),
                   pk_fma(nib_pair_lo(n1), vds, vdm), pk_fma(nib_pair_hi(n1), vds, vdm));
}

//   Q6_K: chunk c holds elements 128n + 32s + l' with s = 2(q&1) + c/2, l' = 16(c&1) + 8h + 0..7:
//   ql_r[64n + 16c + 8h ..] (nibble s >= 2), qh_r[32n + 16(c&1) + 8h ..] (crumb s), scale
//   8n + 4(q&1) + c (qwen_cpu/quants.h:96-121).
struct Q6Src {
    u2 qh[2], ql[4];
    uint32_t sc;  // the four int8 scales of the quarter's chunks
    float d;
};

__device__ inline Q6Src q6_src(const uint8_t* R, int q, int r, int h) {
    Q6Src o;
#pragma unroll
    for (int i = 0; i < 2; i++) o.qh[i] = ld8(R + 1024 + 16 * (r + 16 * i) + 8 * h);
#pragma unroll
    for (int c = 0; c < 4; c++) o.ql[c] = ld8(R + 16 * (16 * c + r) + 8 * h);
    // bytes 1536 + 32 (r >> 2) + 4 (4 (q & 1) + c) + (r & 3), c = 0..3
    const uint8_t* scp = R + 1536 + 32 * (r >> 2) + 16 * (q & 1) + (r & 3);
    o.sc = (uint32_t)scp[0] | ((uint32_t)scp[4] << 8) | ((uint32_t)scp[8] << 16) | ((uint32_t)scp[12] << 24);
    o.d = h2f_bits(*(const uint16_t*)(R + 1664 + 2 * r));
    return o;
}

__device__ inline h8 q6_frag(const Q6Src& S, int q, int c) {
    const int hn = q & 1;
    const h2 m1056 = {(_Float16)-1056.0f, (_Float16)-1056.0f};
    const int sc = (int)(int8_t)(uint8_t)(S.sc >> (8 * c));
    const _Float16 ds = (_Float16)(S.d * (float)sc);
    const h2 vds = {ds, ds};
    const int sh = 2 * (2 * hn + (c >> 1));
    uint32_t v[2];
#pragma unroll
    for (int e = 0; e < 2; e++) {
        const uint32_t L = e ? S.ql[c].y : S.ql[c].x, H = e ? S.qh[c & 1].y : S.qh[c & 1].x;
        const uint32_t lo = hn ? (L >> 4) & 0x0F0F0F0Fu : L & 0x0F0F0F0Fu;
        v[e] = lo | (((H >> sh) & 0x03030303u) << 4);
    }
    // (1024 + q) - 1056 = q - 32 exactly, then one rounding of (q - 32) * half(d * sc)
    return make_h8(as_u32((as_h2(perm_lo(v[0])) + m1056) * vds), as_u32((as_h2(perm_hi(v[0])) + m1056) * vds),
                   as_u32((as_h2(perm_lo(v[1])) + m1056) * vds), as_u32((as_h2(perm_hi(v[1])) + m1056) * vds));
}

//   Q5_K: the Q4_K fragment with bit 2q + (c >> 1) of qh_r[16(c & 1) + 8h + e] as the fifth bit of
//   each quant (qwen_cpu/quants.h:73-94); q < 32 goes through the exact fp16 form 1024 + q.
struct Q5Scales {
    Q4Scales s;
    u2 qh[2];  // qh_r[8h + 0..7], qh_r[16 + 8h + 0..7]
};

__device__ inline h8 q5_frag(const Q4Src& S4, const u2 (&qh)[2], uint32_t dm, int q, int c) {
    const h2 v = as_h2(dm);
    const h2 vds = {v.x, v.x}, vdm = {v.y, v.y}, m1024 = {(_Float16)-1024.0f, (_Float16)-1024.0f};
    const u2 src = (c & 1) ? S4.hi : S4.lo;
    const u2 H = qh[c & 1];
    const int bit = 2 * q + (c >> 1);
    const uint32_t n0 = ((c >> 1) ? (src.x >> 4) & 0x0F0F0F0Fu : src.x & 0x0F0F0F0Fu) | (((H.x >> bit) & 0x01010101u) << 4);
    const uint32_t n1 = ((c >> 1) ? (src.y >> 4) & 0x0F0F0F0Fu : src.y & 0x0F0F0F0Fu) | (((H.y >> bit) & 0x01010101u) << 4);
    auto w = [&](uint32_t p) { return as_u32(__builtin_elementwise_fma(as_h2(p) + m1024, vds, vdm)); };
    return make_h8(w(perm_lo(n0)), w(perm_hi(n0)), w(perm_lo(n1)), w(perm_hi(n1)));
}

//   Q8_0: chunk c of quarter q is block 2q + (c >> 1); lane (h, r) takes quants r, 16c + 8h + 0..7 of
//   the quarter (qwen_cpu/quants.h:45-51).  An int8 b becomes fp16 exactly as (1024 + (b ^ 0x80)) -
//   1152; w = q * half(d) rounds once (the reference's fp16 GEMM path).
struct Q8Src {
    u2 q[4];
};

__device__ inline Q8Src q8_src(const uint8_t* R) {  // R: the tile's piece 0 + 16 r + 8 h
    Q8Src o;
#pragma unroll
    for (int c = 0; c < 4; c++) o.q[c] = ld8(R + 256 * c);
    return o;
}

__device__ inline h8 q8_frag(const Q8Src& S, const u4& dq, int q, int c) {  // dq: d of the row's 8 blocks
    // d of block j sits at byte 8(j & 1) + 2(j >> 1) of the row's 16 bytes: j = 2q + (c >> 1)
    const uint32_t dw = (c >> 1) ? (q < 2 ? dq.z : dq.w) : (q < 2 ? dq.x : dq.y);
    const _Float16 d = __builtin_bit_cast(_Float16, (uint16_t)(dw >> (16 * (q & 1))));
    const h2 vd = {d, d}, m1152 = {(_Float16)-1152.0f, (_Float16)-1152.0f};
    const uint32_t b0 = S.q[c].x ^ 0x80808080u, b1 = S.q[c].y ^ 0x80808080u;
    auto w = [&](uint32_t p) { return as_u32((as_h2(p) + m1152) * vd); };
    return make_h8(w(perm_lo(b0)), w(perm_hi(b0)), w(perm_lo(b1)), w(perm_hi(b1)));
}

template <int TYPE>
struct Gcfg {
    static constexpr int GBYTES = group_bytes(TYPE);
    using Src = std::conditional_t<TYPE == T_Q6_K, Q6Src, std::conditional_t<TYPE == T_Q8_0, Q8Src, Q4Src>>;
    // what a compute lane keeps per tile for a whole super-block
    using Sc = std::conditional_t<TYPE == T_Q4_K, Q4Scales, std::conditional_t<TYPE == T_Q5_K, Q5Scales, u4>>;
    static constexpr bool DM = TYPE == T_Q4_K || TYPE == T_Q5_K;  // per-sub-block (d*sc, -dmin*m)
};

// Raw words of one tile for step q (R: the tile's first piece in the stage) and its per-super-block
// values (S: the stage's scale region; the tile's pieces at 256 * (j * tpad + tile), tpad = tiles of
// the region rounded up to whole jobs of four).
template <int TYPE>
__device__ inline typename Gcfg<TYPE>::Src gemm_src(const uint8_t* R, int q, int r, int h) {
    if constexpr (TYPE == T_Q6_K) return q6_src(R, q, r, h);
    else if constexpr (TYPE == T_Q8_0) return q8_src(R + 16 * r + 8 * h);
    else return q4_src(R + 16 * r + 8 * h);
}
template <int TYPE>
__device__ inline typename Gcfg<TYPE>::Sc gemm_scales(const uint8_t* S, int tile, int tpad, int r, int h) {
    if constexpr (TYPE == T_Q4_K) {
        return q4_scales(S + tile * 256, r);
    } else if constexpr (TYPE == T_Q5_K) {
        Q5Scales o;
        o.s = q4_scales(S + tile * 256, r);
        o.qh[0] = ld8(S + (tpad + tile) * 256 + 16 * r + 8 * h);
        o.qh[1] = ld8(S + (2 * tpad + tile) * 256 + 16 * r + 8 * h);
        return o;
    } else if constexpr (TYPE == T_Q8_0) {
        return ld16(S + tile * 256 + 16 * r);
    } else {
        return u4{0u, 0u, 0u, 0u};
    }
}
template <int TYPE>
__device__ inline uint32_t gemm_dm(const typename Gcfg<TYPE>::Sc& sc, int j) {
    if constexpr (TYPE == T_Q4_K) return q4_dm(sc, j);
    else if constexpr (TYPE == T_Q5_K) return q4_dm(sc.s, j);
    else return 0u;
}
template <int TYPE>
__device__ inline h8 gemm_frag(const typename Gcfg<TYPE>::Src& src, const typename Gcfg<TYPE>::Sc& sc,
                               uint32_t dm, int q, int c) {
    if constexpr (TYPE == T_Q4_K) return q4_frag(src, dm, c);
    else if constexpr (TYPE == T_Q5_K) return q5_frag(src, sc.qh, dm, q, c);
    else if constexpr (TYPE == T_Q8_0) return q8_frag(src, sc, q, c);
    else return q6_frag(src, q, c);
}

// LDS of one work-group: as many stages as 160 KiB hold, at most four (measured: a deeper look-ahead
// only queues more requests); LDS-DMA runs STAGES - 1 steps ahead of the step being multiplied.  A stage holds the step's fp16 activations (X), its raw
// weight bytes (R) and, for Q4_K, the tiles' d/dmin/scale pieces (S), filled only for quarter 0:
// the unpacked scales of a super-block stay in registers for its four steps.  Every part is moved
// as 1 KiB LDS-DMA jobs (64 lanes x 16 B).
//   Q4_K: R = tile t's two qs pieces at 512 t (piece j at + 256 j), S = tile t's piece at 256 t.
//   Q6_K: R = tile t's seven pieces at 1792 t.
template <int TYPE, int P, int NTB>
struct GemmLds {
    static constexpr int XJ = NTB * 4;  // activation jobs: (32-token block, eight tokens)
    static constexpr int RPIECES = GT<TYPE>::RP;
    static constexpr int RJ = (2 * P * RPIECES + 3) / 4;
    static constexpr int TJ = (2 * P + 3) / 4;  // jobs per scale piece: four tiles each
    static constexpr int TPAD = 4 * TJ;         // tiles per scale-piece region
    static constexpr int SJ = GT<TYPE>::SP * TJ;
    static constexpr int X = XJ * 1024, R = RJ * 1024, S = SJ * 1024;
    static constexpr int STAGE = X + R + S;
    static constexpr int STAGES = (160 * 1024 / STAGE) < MAX_STAGES ? 160 * 1024 / STAGE : MAX_STAGES;
    static constexpr int TOTAL = STAGES * STAGE;
    static constexpr int MAXJ = (RJ + SJ + 3) / 4;  // weight jobs of one DMA wave in one step, at most
};

// Work-group -> (pair group px, token block ty, K-part part).  Work-groups are dealt to the 8 XCDs
// round-robin (linear id % 8; the grid's x extent is a multiple of 8, so that is blockIdx.x % 8).
// map 0: the (K-part, pair group) units u = part * npx + px are dealt densely, the j-th id of XCD x
// taking unit 8 (j / mblocks) + x and token block j % mblocks, so a unit's token blocks share its XCD
// (its weights come into that L2 once and serve every token block) and no XCD holds more than one
// unit more than another.  Padding each part's pair groups to a multiple of 8 instead put every
// part's idle ids on the same XCDs, and the live work-groups of the others past their CUs (measured:
// Q6_K K=17408 N=5120 at 13 tokens, 18 pair groups x 14 parts, XCDs 0 and 1 held 42 work-groups for
// 32 CUs, a second round starting at 32 us; Q5_K K=17408 N=5120 M=512, 20 pair groups x 3 parts x 4
// token blocks, 172 against 111 us).
// map 1 (2, 4 or 8 token blocks): an XCD serves one token block, its L2 keeping that block's
// activations while the pair groups stream past: the rep = 8 / mblocks XCDs of token block ty take
// its (K-part, pair group) units densely in turn, the j-th id of the i-th of them unit j * rep + i,
// so again no XCD holds more than one unit more than another (with one K-part, pair group j * rep +
// i).  Each K-part padded to rep XCDs on its own had put Q4_K K=17408 N=5120 at 200 tokens (18 pair
// groups x 2 token blocks x 7 parts, 252 work-groups) into a second round: 35 work-groups on each of
// XCDs 0..3 (92 against 61 us with 6 parts).
constexpr int XCDS = 8;
std::atomic<int> g_map{1};  // tuning: qk_set_tuning("gemm_map")
__device__ inline bool wg_coords(int npx, int mblocks, int ks, int map, int& px, int& ty, int& part) {
    const int xcd = blockIdx.x % XCDS, j = blockIdx.x / XCDS;
    if (map == 1) {
        const int rep = XCDS / mblocks;  // XCDs per token block
        const int u = j * rep + xcd / mblocks;
        ty = xcd % mblocks;
        part = u / npx;
        px = u - part * npx;
        return part < ks;
    }
    const int u = (j / mblocks) * XCDS + xcd;
    ty = j % mblocks;
    part = u / npx;
    px = u - part * npx;
    return part < ks;
}

// NTB: 32-token blocks per work-group (1, 2 or 4: up to 32, 64 or 128 tokens), so that a call with
// few tokens moves and multiplies only the blocks it has.
// Up to GEMM_MATS matrices of one type and k sharing x, one per grid z (a grouped launch, or a gate/up
// pair): matrix z has n[z] rows, weights w[z] and output y[z].
struct GemmMats {
    const uint8_t* w[GEMM_MATS];
    float* y[GEMM_MATS];
    int n[GEMM_MATS];
};

template <int TYPE, int P, int NTB>
// Grid: x as wg_coords maps it, z = matrix.  Ids past matrix z's work exit at once.  Split K (ks parts): part j takes super-blocks [j * nsb_row / ks, (j + 1) * nsb_row / ks)
// and, with parts set, writes its sums to y[z] + j * m * n[z] (partials, added by k_splitk_sum /
// k_glu_sum); otherwise y[z] receives the result itself.
__global__ __launch_bounds__(THREADS) void k_gemm(const GemmMats mats, int nsb_row, const _Float16* __restrict__ xh,
                                                  int xperm, int m, int map, int parts, int ks) {
    using C = Gcfg<TYPE>;
    using L = GemmLds<TYPE, P, NTB>;
    static_assert(NTB == 1 || NTB == 2 || NTB == 4, "token blocks");
    constexpr int STAGES = L::STAGES;
    static_assert(STAGES >= 3 && L::TOTAL <= 160 * 1024, "work-group LDS");
    // Tile pairs: compute wave w owns pairs w*OWN .. w*OWN + OWN-1 for all NTB token blocks; the SH
    // remaining pairs are shared by token block: DMA wave 4 + w takes token block w < NTB of each (in
    // the compute waves when there are no owned pairs).
    constexpr int OWN = P / 4, SH = P % 4;
    constexpr int SHC = OWN > 0 ? 0 : SH, SHP = SH - SHC;  // shared pairs in compute / DMA waves
    constexpr int NPL = OWN + SHC;                          // pairs whose fragments a compute wave builds
    extern __shared__ __align__(16) uint8_t smem[];
    auto sX = [&](int st) { return smem + st * L::STAGE; };
    auto sR = [&](int st) { return smem + st * L::STAGE + L::X; };
    auto sS = [&](int st) { return smem + st * L::STAGE + L::X + L::R; };

    const int tid = threadIdx.x, lane = tid & 63, wid = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wave = wid & 3;  // compute waves 0..3; DMA waves 4..7 take job lanes 0..3
    const int r = lane & 15, u = (lane >> 4) & 1, h = lane >> 5;
    const int z = blockIdx.z;
    const uint8_t* const w = mats.w[z];
    const int n = mats.n[z], ntiles = n / 16;
    const int npx = (ntiles + 2 * P - 1) / (2 * P);
    int px, ty, part;
    if (!wg_coords(npx, (m + 32 * NTB - 1) / (32 * NTB), ks, map, px, ty, part)) return;
    const int tile0 = px * 2 * P, tn = min(2 * P, ntiles - tile0);
    const int tb0 = ty * NTB;
    const int sb0 = (int)(((long long)part * nsb_row) / ks);
    const int nsb = (int)(((long long)(part + 1) * nsb_row) / ks) - sb0;  // this part's super-blocks
    const int kx = nsb_row * 256;  // K: halves between consecutive tokens of x
    const int steps = nsb * 4;
    float* const y = mats.y[z] + (parts ? (size_t)part * m * n : 0);

    // DMA jobs of step t.  Activations: XJ jobs (token block tb, tokens 8j .. 8j + 7), compute wave w
    // issuing job j = w of every token block, just before its barrier where it would wait anyway.  Weights:
    // RJ raw-weight jobs, then (Q4_K, quarter 0) SJ scale jobs; DMA wave 4 + w issues jobs w, w + 4,
    // ...  Pieces past the last tile re-read the last valid one into the region's padding.  Every
    // job's per-lane source is computed once; a step adds an offset uniform over the wave.
    constexpr int XPW = NTB;  // activation jobs per compute wave and step
    constexpr int NRW = (L::RJ + 3) / 4, NSW = L::SJ > 0 ? (L::SJ + 3) / 4 : 1;  // jobs per DMA wave, at most
    auto njobs = [&](int t) { return (L::RJ + ((t & 3) == 0 ? L::SJ : 0) - wave + 3) / 4; };
    auto pair_of = [&](int i) { return i < OWN ? wave * OWN + i : 4 * OWN + (i - OWN); };

    // lane holds token 32*tb + (lane & 31), rows 8j + 4h + 0..3 (j = 0..3) of a pair: j < 2 in its
    // first tile, j >= 2 in its second
    auto store = [&](const f16v& v, int pair, int tb) {
        const int tok = 32 * (tb0 + tb) + (lane & 31);
        if (tok >= m) return;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int row = 8 * j + 4 * h;  // within the pair
            if (2 * pair + (row >> 4) < tn)
                *(f4*)(y + (size_t)tok * n + (size_t)tile0 * 16 + 32 * pair + row) =
                    f4{v[4 * j], v[4 * j + 1], v[4 * j + 2], v[4 * j + 3]};
        }
    };
    if (wid >= 4) {
        // DMA waves.  Stage t % STAGES receives step t; barrier B_s (one per step, shared with the
        // compute waves) publishes step s + 1 and releases stage s, which then receives step
        // s + STAGES.  Before B_s a DMA wave waits for its jobs of step s + 1.
        constexpr int MAXQ = (STAGES - 1) * L::MAXJ;
        static_assert(MAXQ < 64, "vmcnt range");
        auto inflight = [&](int t0, int t1) {  // jobs of steps t0 .. min(t1, steps - 1)
            int nq = 0;
            for (int t = t0; t <= min(t1, steps - 1); t++) nq += njobs(t);
            return nq;
        };
        const int li = lane & 15, nr = (L::RJ - wave + 3) / 4, ns = (L::SJ - wave + 3) / 4;
        const uint8_t* rbase[NRW];
        uint32_t rnstr[NRW];  // Q6_K: per-lane source step per half-plane
        const uint8_t* sbase[NSW];
#pragma unroll
        for (int k = 0; k < NRW; k++) {
            const int g = min(wave + 4 * k, L::RJ - 1);
            const int piece = min(4 * g + (lane >> 4), 2 * P * L::RPIECES - 1);
            const int tt = min(piece / L::RPIECES, tn - 1), j = piece % L::RPIECES;
            const uint8_t* G = w + ((size_t)(tile0 + tt) * nsb_row + sb0) * C::GBYTES;
            if constexpr (TYPE != T_Q6_K) {
                rbase[k] = G + (TYPE == T_Q8_0 ? 256 : 1024) * j + 16 * li;
                rnstr[k] = 0;
            } else {
                uint32_t off;
                q6_piece_base(j, li, off, rnstr[k]);
                rbase[k] = G + off;
            }
        }
#pragma unroll
        for (int k = 0; k < NSW; k++) {
            // scale job g: piece g / TJ of tiles 4 (g % TJ) .. + 3 (tiles past the last re-read it)
            const int g = min(wave + 4 * k, max(L::SJ - 1, 0));
            const int tt = min(min(4 * (g % L::TJ) + (lane >> 4), 2 * P - 1), tn - 1);
            sbase[k] = w + ((size_t)(tile0 + tt) * nsb_row + sb0) * C::GBYTES + GT<TYPE>::SOFF + 256 * (g / L::TJ) + 16 * li;
        }
        auto issue_step = [&](int t) {
            const int sb = t >> 2, q = t & 3, st = t % STAGES;
            const size_t off = (size_t)sb * C::GBYTES + GT<TYPE>::QSTEP * q;
#pragma unroll
            for (int k = 0; k < NRW; k++) {
                if (k < nr) dma16(rbase[k] + off + (q >> 1) * rnstr[k], sR(st) + (wave + 4 * k) * 1024);
            }
            if (L::SJ > 0 && q == 0) {
#pragma unroll
                for (int k = 0; k < NSW; k++) {
                    if (k < ns) dma16(sbase[k] + (size_t)sb * C::GBYTES, sS(st) + (wave + 4 * k) * 1024);
                }
            }
        };
        // Shared pairs: token block w of pairs 4*OWN .. 4*OWN + SHP - 1.  Iteration s runs between
        // B_s-1 and B_s: it reads step s's raw words and activations, issues step s + STAGES - 1 into
        // the stage B_s-1 released (the DMA issue stalls cover the LDS latency), then multiplies.
        f16v accp[SHP > 0 ? SHP : 1];
#pragma unroll
        for (int j = 0; j < (SHP > 0 ? SHP : 1); j++)
#pragma unroll
            for (int e = 0; e < 16; e++) accp[j][e] = 0.0f;
        typename C::Sc scp[SHP > 0 ? SHP : 1];
        auto tile = [&](int j) { return 2 * (4 * OWN + j) + u; };
        const bool shw = NTB == 4 || wave < NTB;  // this DMA wave's token block exists
        for (int t = 0; t < STAGES - 1 && t < steps; t++) issue_step(t);
        wait_vm_le<MAXQ>(inflight(1, STAGES - 2));
        lds_barrier();  // B_-1: step 0 published
        for (int s = 0; s < steps; s++) {
            const int st = s % STAGES, q = s & 3;
            typename C::Src sp[SHP > 0 ? SHP : 1];
            h8 bx[4];
            if constexpr (SHP > 0) {
                if (shw) {
                    if constexpr (GT<TYPE>::SP > 0) {
                        if (q == 0) {
#pragma unroll
                            for (int j = 0; j < SHP; j++) scp[j] = gemm_scales<TYPE>(sS(st), tile(j), L::TPAD, r, h);
                        }
                    }
#pragma unroll
                    for (int j = 0; j < SHP; j++) sp[j] = gemm_src<TYPE>(sR(st) + tile(j) * L::RPIECES * 256, q, r, h);
#pragma unroll
                    for (int c = 0; c < 4; c++)
                        bx[c] = __builtin_bit_cast(h8, *(const u4*)(sX(st) + wave * 4096 + xb_lane_off(lane) + 256 * c));
                }
            }
            if (s + STAGES - 1 < steps) issue_step(s + STAGES - 1);
            if constexpr (SHP > 0) {
                if (shw) {
                    uint32_t dmp[C::DM ? SHP : 1] = {};
#pragma unroll
                    for (int c = 0; c < 4; c++) {
#pragma unroll
                        for (int j = 0; j < SHP; j++) {
                            if constexpr (C::DM) {
                                if (c == 0 || c == 2) dmp[j] = gemm_dm<TYPE>(scp[j], 2 * q + (c >> 1));
                            }
                            const h8 af = gemm_frag<TYPE>(sp[j], scp[j], C::DM ? dmp[j] : 0u, q, c);
                            accp[j] = mfma32(af, bx[c], accp[j]);
                        }
                    }
                }
            }
            wait_vm_le<MAXQ>(inflight(s + 2, s + STAGES - 1));
            lds_barrier();  // B_s
        }
        wait_vm<0>();
        if (shw) {
#pragma unroll
            for (int j = 0; j < SHP; j++) store(accp[j], 4 * OWN + j, wave);
        }
        return;
    }

    f16v acc[OWN > 0 ? OWN : 1][NTB], accs[SHC > 0 ? SHC : 1];
    // the token block of this wave's shared pairs (waves past the last block repeat it unstored)
    const int wtb = NTB == 4 ? wave : min(wave, NTB - 1);
#pragma unroll
    for (int i = 0; i < (OWN > 0 ? OWN : 1); i++)
#pragma unroll
        for (int b = 0; b < NTB; b++)
#pragma unroll
            for (int e = 0; e < 16; e++) acc[i][b][e] = 0.0f;
#pragma unroll
    for (int i = 0; i < (SHC > 0 ? SHC : 1); i++)
#pragma unroll
        for (int e = 0; e < 16; e++) accs[i][e] = 0.0f;

    // activation DMAs: steps 0 .. STAGES - 2 now, step s + STAGES - 1 in region 2 of step s
    // compute wave w issues DMA j = w of every token block: lane i brings token 8w + (i & 7) (tokens
    // past m re-read token m - 1; their columns are never stored), k-piece 2 (i >> 4) + (((i >> 3) & 1)
    // ^ (w & 1)) of each step
    // x in the xperm layout (runs of 1024 elements permuted, xperm_pos): element e = 64 T + 8 p of
    // global step T and k-piece p sits at 1024 (T >> 4) + 256 (p & 3) + 64 ((T >> 2) & 3) + 16 (T & 3)
    // + 8 (p >> 2), a 16-byte run like the plain layout's, so a lane keeps its part (256 (p & 3) +
    // 8 (p >> 2)) and each step adds a part uniform over the wave.
    const uint8_t* xb[XPW];
    {
        const int p = 2 * (lane >> 4) + (((lane >> 3) & 1) ^ (wave & 1));
        const int pe = xperm ? 256 * (p & 3) + 8 * (p >> 2) : 256 * sb0 + 8 * p;
#pragma unroll
        for (int tb = 0; tb < XPW; tb++) {
            const int tok = min(32 * (tb0 + tb) + 8 * wave + (lane & 7), m - 1);
            xb[tb] = (const uint8_t*)(xh + (size_t)tok * kx + pe);
        }
    }
    auto issue_x = [&](int t) {
        const int st = t % STAGES, T = 4 * sb0 + t;
        const size_t off = xperm ? (size_t)2 * (1024 * (T >> 4) + 64 * ((T >> 2) & 3) + 16 * (T & 3)) : (size_t)t * 128;
#pragma unroll
        for (int tb = 0; tb < XPW; tb++) dma16(xb[tb] + off, sX(st) + (tb * 4 + wave) * 1024);
    };
    constexpr int XQ = (STAGES - 2) * XPW;
    for (int t = 0; t < STAGES - 1 && t < steps; t++) issue_x(t);
    wait_vm_le<XQ>(XPW * (min(STAGES - 1, steps) - 1));
    lds_barrier();  // B_-1: step 0 published

    // Compute waves: a software pipeline over K/16 chunks.  While the MFMAs of chunk c run, the wave
    // reads chunk c+1's activations from LDS and builds chunk c+1's weight fragments; registers
    // alternate by chunk parity.  Stage s is read from region 3 of step s - 1 (raw words, scales,
    // activations of chunk 0) to region 2 of step s (chunk 3); barrier B_s closes region 2 of step s.
    typename C::Sc sc4[GT<TYPE>::SP > 0 ? NPL : 1];
    uint32_t dmc[C::DM ? NPL : 1];  // Q4_K / Q5_K: gemm_dm of the sub-block of the chunk being built
    typename C::Src src[NPL];
    h8 a[2][NPL], b[OWN > 0 ? NTB : 1], bs;
    auto tile_idx = [&](int i) { return 2 * pair_of(i) + u; };
    // per-lane LDS bases: every step adds its stage offset once, the rest are immediate offsets
    const uint8_t* const xlane = smem + xb_lane_off(lane);
    const uint8_t* const rown = sR(0) + (2 * wave * OWN + u) * L::RPIECES * 256 + 16 * r + 8 * h;
    const uint8_t* const rsh = sR(0) + (8 * OWN + u) * L::RPIECES * 256 + 16 * r + 8 * h;
    auto load_src = [&](int t) {
        const int st = t % STAGES;
#pragma unroll
        for (int i = 0; i < NPL; i++) {
            if constexpr (TYPE == T_Q4_K || TYPE == T_Q5_K) {
                src[i] = i < OWN ? q4_src(rown + st * L::STAGE + 2 * i * L::RPIECES * 256)
                                 : q4_src(rsh + st * L::STAGE + 2 * (i - OWN) * L::RPIECES * 256);
            } else if constexpr (TYPE == T_Q8_0) {
                src[i] = i < OWN ? q8_src(rown + st * L::STAGE + 2 * i * L::RPIECES * 256)
                                 : q8_src(rsh + st * L::STAGE + 2 * (i - OWN) * L::RPIECES * 256);
            } else {
                src[i] = q6_src(sR(st) + tile_idx(i) * L::RPIECES * 256, t & 3, r, h);
            }
        }
    };
    auto load_scales = [&](int t) {
        if constexpr (GT<TYPE>::SP > 0) {
#pragma unroll
            for (int i = 0; i < NPL; i++) sc4[i] = gemm_scales<TYPE>(sS(t % STAGES), tile_idx(i), L::TPAD, r, h);
        }
    };
    auto load_x = [&](int t, int c, int tb) {  // B operand: token block tb, chunk c of step t
        return __builtin_bit_cast(h8, *(const u4*)(xlane + (t % STAGES) * L::STAGE + tb * 4096 + 256 * c));
    };
    auto frag = [&](int i, int q, int c) {
        return gemm_frag<TYPE>(src[i], sc4[GT<TYPE>::SP > 0 ? i : 0], C::DM ? dmc[i] : 0u, q, c);
    };
    auto set_dm = [&](int j) {  // chunks 0 and 2 start sub-blocks 2q and 2q + 1
        if constexpr (C::DM) {
#pragma unroll
            for (int i = 0; i < NPL; i++) dmc[i] = gemm_dm<TYPE>(sc4[i], j);
        }
    };

    load_src(0);
    load_scales(0);
    if constexpr (OWN > 0) {
#pragma unroll
        for (int tb = 0; tb < NTB; tb++) b[tb] = load_x(0, 0, tb);
    }
    if constexpr (SHC > 0) bs = load_x(0, 0, wtb);
    set_dm(0);
#pragma unroll
    for (int i = 0; i < NPL; i++) a[0][i] = frag(i, 0, 0);

    for (int sb = 0; sb < nsb; sb++) {
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const int s = 4 * sb + q;
            static_for<4>([&](auto Cc) {
                constexpr int c = decltype(Cc)::value, par = c & 1, npar = par ^ 1;
                // the next chunk: c + 1 of this step, or chunk 0 of step s + 1 (past the last step the
                // reads land in a valid stage and their results go unused)
                const int tnx = c < 3 ? s : s + 1;
                constexpr int cnx = c < 3 ? c + 1 : 0;
                if constexpr (c == 3) {
                    load_src(s + 1);
                    if (q == 3) load_scales(s + 1);
                }
                __builtin_amdgcn_sched_barrier(0);
                // chunk c's MFMAs, token block by token block; each B register is reloaded with the
                // next chunk right after its last MFMA, and the next chunk's fragments are built
                // among the MFMAs
                if constexpr (OWN > 0) {
#pragma unroll
                    for (int tb = 0; tb < NTB; tb++) {
#pragma unroll
                        for (int i = 0; i < OWN; i++) acc[i][tb] = mfma32(a[par][i], b[tb], acc[i][tb]);
                        b[tb] = load_x(tnx, cnx, tb);
                    }
                }
                if constexpr (SHC > 0) {
#pragma unroll
                    for (int i = 0; i < SHC; i++) accs[i] = mfma32(a[par][OWN + i], bs, accs[i]);
                    bs = load_x(tnx, cnx, wtb);
                }
                if constexpr (cnx == 0) set_dm(2 * ((q + 1) & 3));
                if constexpr (cnx == 2) set_dm(2 * q + 1);
#pragma unroll
                for (int i = 0; i < NPL; i++) a[npar][i] = frag(i, c < 3 ? q : (q + 1) & 3, cnx);
                // one MFMA per few VALU operations; region 3's fragments wait for the raw words read
                // at its start, so its first MFMAs go without VALU
                constexpr int VA = c == 3 ? 8 : 6;
                if constexpr (OWN > 0) {
                    static_for<NTB>([&](auto T) {
                        static_for<OWN>([&](auto I) {
                            constexpr int k = decltype(T)::value * OWN + decltype(I)::value;
                            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                            __builtin_amdgcn_sched_group_barrier(0x002, c == 3 && k < 3 ? 0 : VA, 0);
                        });
                        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                    });
                }
                if constexpr (SHC > 0) {
                    __builtin_amdgcn_sched_group_barrier(0x008, SHC, 0);
                    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x002, 64, 0);
                }
                // keep the fragments in this region (they would otherwise sink to their first use)
#pragma unroll
                for (int i = 0; i < NPL; i++) asm volatile("" : "+v"(a[npar][i]));
                __builtin_amdgcn_sched_barrier(0);
                if constexpr (c == 2) {
                    if (s + STAGES - 1 < steps) issue_x(s + STAGES - 1);
                    wait_vm_le<XQ>(XPW * max(0, min(STAGES - 2, steps - 2 - s)));  // this wave's step s + 1
                    lds_barrier();  // B_s
                }
            });
        }
    }

    wait_vm<0>();
#pragma unroll
    for (int i = 0; i < OWN; i++)
#pragma unroll
        for (int tb = 0; tb < NTB; tb++) store(acc[i][tb], wave * OWN + i, tb);
    if (NTB == 4 || wave < NTB) {
#pragma unroll
        for (int i = 0; i < SHC; i++) store(accs[i], 4 * OWN + i, wave);
    }
}

// Adds the ks partial results [ks][m][n] of matrix blockIdx.y in part order (deterministic) into its y.
struct SumMats {
    const f4* part[GEMM_MATS];
    f4* y[GEMM_MATS];
    size_t n4[GEMM_MATS];
};
__global__ __launch_bounds__(256) void k_splitk_sum(const SumMats S, int ks) {
    const f4* __restrict__ part = S.part[blockIdx.y];
    f4* __restrict__ y = S.y[blockIdx.y];
    const size_t n4 = S.n4[blockIdx.y];
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n4; i += (size_t)gridDim.x * 256) {
        f4 v = part[i];
        for (int j = 1; j < ks; j++) v += part[j * n4 + i];
        y[i] = v;
    }
}

// The gate/up pair's output: part holds [2][ks][m][n] (gate, then up); each thread adds the ks parts
// of four consecutive rows of both in part order and stores silu(g) u (silu(v) = v / (1 + e^-v), as
// the GEMV's GLU output) in yfmt: fp32, or fp16 (round to nearest even) at the plain or xperm position.
__global__ __launch_bounds__(256) void k_glu_sum(const f4* __restrict__ part, int ks, size_t n4, int n4row, void* y,
                                                 int yfmt) {
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n4; i += (size_t)gridDim.x * 256) {
        f4 g = part[i], u = part[(size_t)ks * n4 + i];
        for (int j = 1; j < ks; j++) {
            g += part[j * n4 + i];
            u += part[(size_t)(ks + j) * n4 + i];
        }
        const int t = (int)(i / n4row), r = 4 * (int)(i % n4row);
        for (int e = 0; e < 4; e++) store_act(y, yfmt, (size_t)n4row * 4, t, r + e, g[e] / (1.0f + expf(-g[e])) * u[e]);
    }
}

// One call: x already fp16 (plain or xperm).  nz matrices of one type and k (w[z], n[z] rows): with glu,
// w[0] / w[1] are gate / up and y[0] receives silu(g) u in yfmt; otherwise y[z] is fp32 [m][n[z]].
// Partials ([ks][m][n[z]] per matrix, one matrix after another) sit in part.
struct GemmCall {
    int nz;
    const uint8_t* w[GEMM_MATS];
    int n[GEMM_MATS];
    void* y[GEMM_MATS];
    int nsb;
    const _Float16* xh;
    int xperm, m;
    int yfmt;
    bool glu;
    float* part;
    size_t part_cap;
    int cus;
    hipStream_t s;
};

template <int TYPE, int P, int NTB>
int launch_p(const GemmCall& c, int ks) {
    constexpr size_t lds = GemmLds<TYPE, P, NTB>::TOTAL;
    const int mblocks = (c.m + 32 * NTB - 1) / (32 * NTB);
    const int map = mblocks > 1 && g_map == 1 && XCDS % mblocks == 0 ? 1 : 0;
    const int rep = XCDS / mblocks;
    const bool parts = ks > 1 || c.glu;
    GemmMats M{};
    SumMats S{};
    int grid = 0;
    size_t off = 0;
    for (int z = 0; z < c.nz; z++) {
        const int npx = (c.n[z] / 16 + 2 * P - 1) / (2 * P);
        grid = std::max(grid, map == 1 ? (npx * ks + rep - 1) / rep * XCDS
                                       : (npx * ks + XCDS - 1) / XCDS * XCDS * mblocks);  // idle ids exit at once
        M.w[z] = c.w[z];
        M.n[z] = c.n[z];
        M.y[z] = parts ? c.part + off : (float*)c.y[z];
        S.part[z] = (const f4*)(c.part + off);
        S.y[z] = (f4*)c.y[z];
        S.n4[z] = (size_t)c.m * c.n[z] / 4;  // n % 16 == 0
        off += (size_t)ks * c.m * c.n[z];
    }
    hipLaunchKernelGGL((k_gemm<TYPE, P, NTB>), dim3(grid, 1, c.nz), dim3(THREADS), lds, c.s, M, c.nsb,
                       c.xh, c.xperm, c.m, map, parts ? 1 : 0, ks);
    if (hipGetLastError() != hipSuccess) return -1;
    size_t n4max = 0;
    for (int z = 0; z < c.nz; z++) n4max = std::max(n4max, S.n4[z]);
    const int blocks = (int)std::min<size_t>((n4max + 255) / 256, 4096);
    if (c.glu)
        hipLaunchKernelGGL(k_glu_sum, dim3(blocks), dim3(256), 0, c.s, (const f4*)c.part, ks, S.n4[0], c.n[0] / 4, c.y[0],
                           c.yfmt);
    else if (ks > 1)
        hipLaunchKernelGGL(k_splitk_sum, dim3(blocks, c.nz), dim3(256), 0, c.s, S, ks);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

// Plan: 32-token blocks per work-group NTB (1 up to 32 tokens, 2 up to 64, else 4), then the tile pairs
// per work-group P and K-parts ks of least estimated time: the busiest CU's work-groups (ceil(work-
// groups / CUs)) times one work-group's time, ~0.03 us per KiB its steps move (4 KiB of activations
// per token block and P pairs' weight pieces) plus ~5 us of pipeline fill and drain; split K adds the
// partials' traffic (ks + 1 passes over m x n fp32 at ~5 TB/s) and one more launch.  P = 5 and 9
// leave a pair to the DMA waves, which then multiply as well as issue the weight DMAs: their steps
// count 1.3 times.  The constants rank (P, ks) as a sweep of every pair measured them on 26 shapes
// (5 to 1024 tokens, four types, a gate/up pair): the plans are within 0.6 % of the fastest measured
// in sum, where the former rule (fewest rounds of work-groups over the CUs first, then ~0.05 us per
// KiB) was 5 % off (14 % on the 19 shapes of 5..512 tokens: Q6_K K=17408 N=5120 at 8 tokens 39.6 ->
// 30.9 us, Q5_K at 13 tokens 33.1 -> 23.4; every M=512 plan unchanged).  With fewer than four token
// blocks only P = 4 and 8 are planned: they give each compute wave whole pairs, where P = 5 and 9
// leave one pair to a single DMA wave (the others wait for it at every step) and P = 2 and 3 repeat
// pairs over the compute waves.  Small P is costly per pair (the activations are shared by fewer
// pairs), so long-K, narrow-N shapes split K rather than shrink P.
constexpr int P_CHOICES[] = {2, 3, 4, 5, 8, 9};
constexpr int MAX_KS = 16;

std::atomic<int> g_gemm_p{0};   // tuning override of the tile pairs per work-group (0 = planned)
std::atomic<int> g_gemm_ks{0};  // tuning override of the K-parts (0 = planned)

template <int TYPE, int NTB>
int launch_ntb(const GemmCall& c) {
    const int nsb = c.nsb, m = c.m, cus = c.cus;
    const double wkib = (GT<TYPE>::RP * 512.0 + GT<TYPE>::SP * 128.0) / 1024.0;  // per pair and step
    const int mblocks = (m + 32 * NTB - 1) / (32 * NTB);
    size_t nsum = 0;  // rows of all the matrices
    for (int z = 0; z < c.nz; z++) nsum += (size_t)c.n[z];
    int best_p = 0, best_ks = 0;
    double best_t = 0.0;
    for (int p : P_CHOICES) {
        if (g_gemm_p ? p != g_gemm_p : NTB < 4 && p != 4 && p != 8) continue;
        for (int ks = 1; ks <= MAX_KS && ks <= nsb; ks++) {
            if (g_gemm_ks && ks != g_gemm_ks) continue;
            if ((ks > 1 || c.glu) && (size_t)ks * m * nsum > c.part_cap) continue;
            long long wgs = 0;
            for (int z = 0; z < c.nz; z++) wgs += (long long)(((c.n[z] / 16 + 1) / 2 + p - 1) / p) * mblocks * ks;
            const long long busy = (wgs + cus - 1) / cus;
            const int sbw = (nsb + ks - 1) / ks;
            double step = sbw * 4 * (4.0 * NTB + p * wkib) * 0.03;
            if (p % 4 == 1) step *= 1.3;  // P = 5, 9: the DMA waves also multiply a pair
            const double t = busy * (step + 5.0) +
                             (ks > 1 || c.glu ? (ks + 1) * 4.0 * m * (double)nsum / 5e6 + 2.0 : 0.0);
            if (!best_p || t < best_t) {
                best_p = p;
                best_ks = ks;
                best_t = t;
            }
        }
    }
    switch (best_p) {
        case 2: return launch_p<TYPE, 2, NTB>(c, best_ks);
        case 3: return launch_p<TYPE, 3, NTB>(c, best_ks);
        case 4: return launch_p<TYPE, 4, NTB>(c, best_ks);
        case 5: return launch_p<TYPE, 5, NTB>(c, best_ks);
        case 8: return launch_p<TYPE, 8, NTB>(c, best_ks);
        case 9: return launch_p<TYPE, 9, NTB>(c, best_ks);
    }
    return -1;
}

template <int TYPE>
int launch_type(const GemmCall& c) {
    const int m = c.m;
    if (m <= 32) return launch_ntb<TYPE, 1>(c);
    if (m <= 64) return launch_ntb<TYPE, 2>(c);
    return launch_ntb<TYPE, 4>(c);
}

}  // namespace

void gemm_set_map(int map) { g_map = map; }

bool gemm_set_pairs(int p) {
    if (p != 0) {
        bool ok = false;
        for (int c : P_CHOICES) ok = ok || c == p;
        if (!ok) return false;
    }
    g_gemm_p = p;
    return true;
}

size_t gemm_image_bytes(int m, int k) { return (size_t)m * k * 2; }

bool gemm_set_ksplit(int ks) {
    if (ks < 0 || ks > MAX_KS) return false;
    g_gemm_ks = ks;
    return true;
}

namespace {
int launch_call(int type, GemmCall& c, int k, const void* x, int xfmt, uint8_t* ximg) {
    if (xfmt != ACT_F16 && xfmt != ACT_F16_XPERM && xfmt != ACT_F32) return -1;
    c.xh = (const _Float16*)x;  // fp16 x (plain or xperm, k % 1024 == 0) is read where it lies
    c.xperm = xfmt == ACT_F16_XPERM ? 1 : 0;
    if (xfmt == ACT_F32) {
        const size_t n8 = (size_t)c.m * k / 8;  // k % 256 == 0
        const int blocks = (int)std::min<size_t>((n8 + 255) / 256, 2048);
        hipLaunchKernelGGL(k_gemm_cvt_x, dim3(blocks), dim3(256), 0, c.s, (const float*)x, n8, (u4*)ximg);
        if (hipGetLastError() != hipSuccess) return -1;
        c.xh = (const _Float16*)ximg;
    }
    c.nsb = k / 256;
    c.cus = current_cus();
    if (type == T_Q4_K) return launch_type<T_Q4_K>(c);
    if (type == T_Q6_K) return launch_type<T_Q6_K>(c);
    if (type == T_Q5_K) return launch_type<T_Q5_K>(c);
    if (type == T_Q8_0) return launch_type<T_Q8_0>(c);
    return -1;
}
}  // namespace

int launch_gemm(int type, const uint8_t* w, int k, int n, const void* x, int xfmt, int m, uint8_t* ximg, float* y,
                float* part, size_t part_cap, hipStream_t s) {
    const uint8_t* ws[1] = {w};
    const int ns[1] = {n};
    float* ys[1] = {y};
    return launch_gemm_group(type, ws, ns, ys, 1, k, x, xfmt, m, ximg, part, part_cap, s);
}

int launch_gemm_group(int type, const uint8_t* const* ws, const int* ns, float* const* ys, int cnt, int k, const void* x,
                      int xfmt, int m, uint8_t* ximg, float* part, size_t part_cap, hipStream_t s) {
    if (cnt < 1 || cnt > GEMM_MATS) return -1;
    GemmCall c{};
    c.nz = cnt;
    for (int z = 0; z < cnt; z++) {
        c.w[z] = ws[z];
        c.n[z] = ns[z];
        c.y[z] = ys[z];
    }
    c.m = m;
    c.yfmt = ACT_F32;
    c.glu = false;
    c.part = part;
    c.part_cap = part_cap;
    c.s = s;
    return launch_call(type, c, k, x, xfmt, ximg);
}

int launch_gemm_glu(int type, const uint8_t* wg, const uint8_t* wu, int k, int n, const void* x, int xfmt, int m,
                    uint8_t* ximg, void* y, int yfmt, float* part, size_t part_cap, hipStream_t s) {
    if ((size_t)2 * m * n > part_cap || (yfmt != ACT_F32 && yfmt != ACT_F16 && yfmt != ACT_F16_XPERM)) return -1;
    GemmCall c{};
    c.nz = 2;
    c.w[0] = wg;
    c.w[1] = wu;
    c.n[0] = c.n[1] = n;
    c.y[0] = y;
    c.m = m;
    c.yfmt = yfmt;
    c.glu = true;
    c.part = part;
    c.part_cap = part_cap;
    c.s = s;
    return launch_call(type, c, k, x, xfmt, ximg);
}

}  // namespace qk
