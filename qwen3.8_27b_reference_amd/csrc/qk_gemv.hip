// Decode GEMV (m <= 4 through qk_matmul and grouped launches, m <= 8 per launch under the gemm_min_m
// knob) with the GGUF block dequant fused into CDNA4 MFMA.
//
// Replaces the reference's k_gemv / k_gemv1 / k_gemv_glu (qwen_cuda/kernels.cu:191-295, 403-438)
// with matrix-core, persistent kernels for 64-lane wavefronts instead of one warp per row.  Weights
// are in the T16 layout (qk_device.h): 16-row tiles whose per-super-block groups each 64-lane load
// reads as one contiguous 1 KiB run; a "unit" is one tile x one super-block column.
//
// Two kernels; launch_gemv picks (qk_gemv_plan reports which):
//  * k_gemv1 (the int8 kernel, the default for m = 1..8 per launch, all four quantized types): one
//    launch, no prepass.  Each work-group converts its slices of x into an LDS image of three int8
//    parts per element with fp32 scales (within max|x| / 16387064), then its waves take units from an
//    LDS counter, stream them through per-wave LDS-DMA rings and run v_mfma_i32_16x16x64_i8 with the
//    weights as the B operand; unit sums are added in unit order per group and shared tiles / K-slices
//    combine through device-scope exchanges (deterministic).  Described in detail above k_gemv1.
//  * k_gemv_q4k / k_gemv_q6k (the general kernel) after the k_prep_q4 / q6 prepass: Q4_K / Q6_K only,
//    under the gemv_fused = 0, gemv_waves and gemv_min_waves tuning knobs (and for a shape no int8
//    plan fits, which the planner's small-matrix plans leave none of).  Its domain is narrower than
//    the int8 kernel's: the prepass writes x as an exact pair of fp16 halves (x == hi + lo to 2^-22,
//    |x| < 65504; Q4_K also its 32-element sub-block sums) in MFMA B-operand records; each
//    wave owns an equal contiguous range of units (stream-K), streams them through an LDS-DMA ring and
//    runs v_mfma_f32_16x16x32_f16 on exact fp16 integer A operands (Q4_K: A = sc*q with the min term
//    on one more MFMA, the reference's hoisting d1*sum(x*q) - m1*sum(x), kernels.cu:193, 281-290;
//    Q6_K: A = 1024 + q, y += d*sc*(D - 1056*Sx)).  Split tiles are summed by whichever contributor
//    completes them, in wave order, through per-tile counters that reset themselves.
#include <algorithm>
#include <atomic>
#include <type_traits>

#include "qk_device.h"
#include "qk_internal.h"

namespace qk {
namespace {

constexpr int LDS_PER_CU = 160 * 1024;
constexpr int LDS_GRANULE = 1024;

#define LDS_AS __attribute__((address_space(3)))

// Wait until at most N vector-memory operations of this wave are outstanding.  The compiler does
// not track LDS-DMA completion for later LDS reads, so the ring waits explicitly; the memory
// clobber keeps the compiler from moving LDS accesses across the wait.
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

template <int STEP>
__device__ inline void wait_vm_units(int k) {  // k = units still allowed in flight (0..2)
    if (k <= 0) wait_vm<0>();
    else if (k == 1) wait_vm<STEP>();
    else wait_vm<2 * STEP>();
}

// Lanes of one wave exchange data through LDS: keep stores and later loads in program order.
__device__ inline void lds_order() { asm volatile("" ::: "memory"); }

// LDS counters shared by the waves of a work-group.  The compiler puts a full vmcnt(0) wait in front
// of every LDS atomic issued while an LDS-DMA may be in flight, which would drain the DMA ring at
// each use; this form waits only for the LDS access itself.  A CU's LDS performs the accesses of one
// wave in program order and those of all waves in one order, so an add that returns the last count
// of a tile comes after every other wave's unit-sum stores to that tile.
__device__ inline uint32_t lds_addr(const void* p) { return (uint32_t)(uintptr_t)(LDS_AS const void*)p; }
// LDS stores the compiler does not see: it would otherwise wait for every in-flight LDS-DMA
// (vmcnt(0)) before a store it cannot prove disjoint from the DMA's destination.
__device__ inline void lds_st32(void* p, uint32_t v) { asm volatile("ds_write_b32 %0, %1" ::"v"(lds_addr(p)), "v"(v) : "memory"); }
__device__ inline void lds_st64(void* p, uint64_t v) { asm volatile("ds_write_b64 %0, %1" ::"v"(lds_addr(p)), "v"(v) : "memory"); }
__device__ inline void lds_st128(void* p, u4 v) { asm volatile("ds_write_b128 %0, %1" ::"v"(lds_addr(p)), "v"(v) : "memory"); }
// Work-group barrier that waits only for this wave's LDS operations (not for its LDS-DMAs, as the
// release fence of __syncthreads() would); the empty asm keeps memory accesses on their side.
__device__ inline void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

__device__ inline void lds_write(int* p, int v) { asm volatile("ds_write_b32 %0, %1" ::"v"(lds_addr(p)), "v"(v) : "memory"); }
__device__ inline int lds_add(int* p, int v) {  // returns the old value
    int old;
    asm volatile("ds_add_rtn_u32 %0, %1, %2\n\ts_waitcnt lgkmcnt(0)" : "=v"(old) : "v"(lds_addr(p)), "v"(v) : "memory");
    return old;
}

// 16 bytes per lane from global memory into LDS (M0 + 16 * lane), without VGPRs.  Issued from inline
// assembly: the compiler then never holds a pending LDS-DMA, which it would otherwise wait out
// (vmcnt(0), the whole ring) before every LDS access it cannot prove disjoint from the destination,
// and before the lane-masked ones it could not count at all.  Every read of DMA'd bytes follows an
// explicit wait_vm*; an operation the compiler does not count only makes its own waits (for the
// loads it issued earlier) more conservative.  The LDS base goes in M0 (an input the compiler
// sets); s_nop: M0 written by the SALU needs one wait state before an LDS-DMA reads it.
__device__ inline void dma16(const void* g, uint8_t* lds) {
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "{m0}"(lds_addr(lds)) : "memory");
}
// The same for weight bytes, which a call reads exactly once: non-temporal, so that the stream does
// not push the activation (read by every CU) out of L2.  Measured on MI355X: the single-token GEMV
// takes 13.0 us instead of 14.4 (K=5120, N=17408) and 19.2 instead of 20.5 (K=17408, N=5120).
__device__ inline void dma16_stream(const void* g, uint8_t* lds) {
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off nt" ::"v"(g), "{m0}"(lds_addr(lds)) : "memory");
}

__device__ inline float silu(float v) { return v / (1.0f + expf(-v)); }

// Four fp32 -> the four hi (or lo) fp16 halves of their exact split.
__device__ inline uint2 pack4(const f4& v, bool lo_part) {
    _Float16 h[4];
#pragma unroll
    for (int e = 0; e < 4; e++) {
        _Float16 hi, lo;
        split_h(v[e], hi, lo);
        h[e] = lo_part ? lo : hi;
    }
    return uint2{as_u32(h2{h[0], h[1]}), as_u32(h2{h[2], h[3]})};
}

// Everything indexed by a wave-uniform value stays in scalar registers: a kernel-argument array is
// read through a select chain, never a computed address (that would turn into a vector load and a
// full vmcnt(0) wait in the middle of the DMA ring).
template <typename T>
__device__ inline T pick(const T* v, int i) {  // v[i] for i < GEMV_MAX_CNT
    static_assert(GEMV_MAX_CNT == 4, "select chain covers four entries");
    return i == 0 ? v[0] : i == 1 ? v[1] : i == 2 ? v[2] : v[3];
}

__device__ inline int tile_matrix(const GemvParams& P, int tile) {  // tile0 is ascending
    if (P.glu) return 0;
    return (P.cnt > 1 && tile >= P.tile0[1]) + (P.cnt > 2 && tile >= P.tile0[2]) + (P.cnt > 3 && tile >= P.tile0[3]);
}

__device__ inline const uint8_t* unit_group(const GemvParams& P, int a, int tile, int sb, int gbytes) {
    const int mi = tile_matrix(P, tile);
    const uint8_t* w = pick(P.w, P.glu ? a : mi);
    return w + ((size_t)(tile - pick(P.tile0, mi)) * P.nsb + sb) * gbytes;
}

__device__ inline int wave_first_unit(const GemvParams& P, int w) {
    return (int)((long long)w * P.units / P.waves);
}
__device__ inline int wave_of_unit(const GemvParams& P, int u) {  // largest w with first_unit(w) <= u
    return (int)(((long long)(u + 1) * P.waves - 1) / P.units);
}

// Single-token kernel ranges: the first rrem work-groups own rq + 1 units, the others rq.
__device__ inline int range_start(const GemvParams& P, int b) { return b * P.rq + min(b, P.rrem); }

// Final value of row `row` of tile `tile`, token t, from the per-stream sums v[0..NA).
template <int NA>
__device__ inline void store_row(const GemvParams& P, int tile, int t, int row, const float (&v)[NA]) {
    const int mi = tile_matrix(P, tile);
    const int n = pick(P.n, mi), r = (tile - pick(P.tile0, mi)) * 16 + row;
    if (P.glu) store_act(pick(P.y, mi), P.yfmt, n, t, r, silu(v[0]) * v[NA - 1]);
    else ((float*)pick(P.y, mi))[(size_t)t * n + r] = v[0];
}

// Pairwise combine through a device-scope exchange on a 64-bit slot holding (stream 0, stream 1):
// the first of the two partners to arrive leaves its value in the slot and is done; the second takes
// it, adds it to its own (old + v == v + old bitwise, so the sum does not depend on who came first)
// and empties the slot for the next launch.  Returns whether this lane carries the sum on.  One
// round trip per combine, instead of a piece store, its wait, a counter add and the piece loads.
// An empty slot is all zeros, so zero-initialised memory (a static device array, a cleared buffer)
// is already in the state every launch leaves behind.  A value is stored complemented: NaNs are
// canonicalised first, so the all-ones pattern never occurs and a stored low word is never zero.
__device__ inline uint32_t canon(float v) { return v != v ? 0x7FC00000u : __builtin_bit_cast(uint32_t, v); }
template <int NA>
__device__ inline bool xcombine(uint64_t* slot, float (&v)[NA]) {
    const uint64_t mine = (uint64_t)~canon(v[0]) | ((uint64_t)(NA == 2 ? ~canon(v[NA - 1]) : 0u) << 32);
    const uint64_t old = __hip_atomic_exchange(slot, mine, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if ((uint32_t)old == 0u) return false;
    __hip_atomic_store(slot, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    v[0] = __builtin_bit_cast(float, ~(uint32_t)old) + v[0];
    if constexpr (NA == 2) v[1] = __builtin_bit_cast(float, ~(uint32_t)(old >> 32)) + v[1];
    return true;
}

// Lane-held result of a finished tile piece: token t, rows 4g..4g+3, one f4 per stream.
template <int NA>
__device__ inline void store_tile(const GemvParams& P, int tile, int t, int g, const f4 (&v)[NA]) {
    const int mi = tile_matrix(P, tile);
    const int n = pick(P.n, mi), r = (tile - pick(P.tile0, mi)) * 16 + 4 * g;
    f4 o;
#pragma unroll
    for (int i = 0; i < 4; i++) o[i] = P.glu ? silu(v[0][i]) * v[NA - 1][i] : v[0][i];
    if (!P.glu || P.yfmt == ACT_F32) {
        *(f4*)((float*)pick(P.y, mi) + (size_t)t * n + r) = o;
        return;
    }
#pragma unroll
    for (int i = 0; i < 4; i++) store_act(pick(P.y, mi), P.yfmt, n, t, r + i, o[i]);
}

// Pieces of split tiles (at most two per wave), handled once the wave's range is done.
template <int NA, int MT>
__device__ inline void finish_pieces(const GemvParams& P, int w, int npend, const int (&ptile)[2],
                                     const int (&punits)[2], const f4 (&pend)[2][NA], bool holds, int t_lane, int g) {
    if (npend == 0) return;
    const int lane = threadIdx.x & 63;
    const int first_tile = wave_first_unit(P, w) / P.nsb;
    for (int k = 0; k < npend; k++) {
        // slot 0: the piece of the wave's first tile, slot 1: of its last tile (what readers expect)
        const int slot = ptile[k] == first_tile ? 0 : 1;
        if (holds) {
#pragma unroll
            for (int a = 0; a < NA; a++) {
                float* dst = P.part + ((((size_t)w * 2 + slot) * NA + a) * MT + t_lane) * 16 + 4 * g;
#pragma unroll
                for (int i = 0; i < 4; i++)
                    __hip_atomic_store(dst + i, pend[k][a][i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
    }
    wait_vm<0>();  // the write-through piece stores have completed before any counter moves
    for (int k = 0; k < npend; k++) {
        const int tile = ptile[k];
        int old = 0;
        if (lane == 0)
            old = __hip_atomic_fetch_add(P.counters + tile, punits[k], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        old = __shfl(old, 0);
        if (old + punits[k] != P.nsb) continue;
        // this wave completed the tile: add every contributor's piece in wave order
        const int wa = wave_of_unit(P, tile * P.nsb), wb = wave_of_unit(P, (tile + 1) * P.nsb - 1);
        const int t = lane >> 4, row = lane & 15;
        if (t < P.m) {
            float v[NA];
#pragma unroll
            for (int a = 0; a < NA; a++) v[a] = 0.0f;
            // contributor wa's piece is its last (slot 1) unless its range starts at this tile;
            // every later contributor starts inside the tile (slot 0)
            const int ka = wave_first_unit(P, wa) < tile * P.nsb ? 1 : 0;
            for (int c0 = wa; c0 <= wb; c0 += 8) {  // issue up to 8 contributors' loads, then add in order
                float pv[8][NA];
#pragma unroll
                for (int q = 0; q < 8; q++) {
                    const int c = min(c0 + q, wb), kc = c == wa ? ka : 0;
#pragma unroll
                    for (int a = 0; a < NA; a++)
                        pv[q][a] = __hip_atomic_load(P.part + ((((size_t)c * 2 + kc) * NA + a) * MT + t) * 16 + row,
                                                     __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
#pragma unroll
                for (int q = 0; q < 8; q++)
#pragma unroll
                    for (int a = 0; a < NA; a++) v[a] += c0 + q <= wb ? pv[q][a] : 0.0f;
            }
            store_row<NA>(P, tile, t, row, v);
        }
        if (lane == 0) __hip_atomic_store(P.counters + tile, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// ================================================================================================
// Activation images.  Per super-block sb the image holds IMG bytes (a multiple of 16), formatted for
// the weight type; the GEMV copies the unit's IMG bytes into its ring slot next to the weights.
template <int MT>
constexpr int q4_img() { return 1152 * MT + 144; }
template <int MT>
constexpr int q6_img() { return MT * (2 * 528 + 128); }

// ================================================================================================
// Q4_K
//
// Activation image of one super-block: 16-byte records at ((g*2MT + col)*9 + j)*16,
// col = 2t + {0: hi, 1: lo}, then a 144-byte zero run:
//   j < 8: x[t][sb*256 + 64g + 32(j>>2) + 8(j&3) + 0..7]   (matches A-operand slot order)
//   j = 8: (Sx[2g], Sx[2g+1], 0 x 6), Sx[i] = sum of x over sub-block i of the super-block.
// A lane reads its nine records from one base address; columns beyond the tokens point at the zero
// run, so no read is exec-masked.  One wave of the prepass writes one (super-block, token).
struct RawQ4 {
    u4 q0, q1;            // qs_r[32g .. 32g+31]
    uint32_t s0, s1, s2;  // scales_r[0..11]
    u4 dd;                // (d, dmin) of rows 4g .. 4g+3
};

constexpr int Q4_DMA = 3;  // LDS-DMA instructions per 2304-byte group
__device__ inline void dma_q4(const uint8_t* G, uint8_t* slot, int lane) {
    dma16_stream(G + 16 * lane, slot);
    dma16_stream(G + 1024 + 16 * lane, slot + 1024);
    if (lane < 16) dma16_stream(G + 2048 + 16 * lane, slot + 2048);
}

__device__ inline RawQ4 load_q4(const uint8_t* G, int lane, int r, int g) {  // G: an LDS ring slot
    RawQ4 w;
    w.q0 = ld16(G + 16 * lane);
    w.q1 = ld16(G + 1024 + 16 * lane);
    w.s0 = ld4(G + 2112 + 12 * r);
    w.s1 = ld4(G + 2116 + 12 * r);
    w.s2 = ld4(G + 2120 + 12 * r);
    w.dd = ld16(G + 2048 + 16 * g);
    return w;
}

__device__ inline f4 q4_step(const RawQ4& w, const h8 (&B)[9], f4 acc, int g) {
    // 6-bit scales/mins of sub-blocks 2g (low nibbles) and 2g+1 (high nibbles): the four j<4 values
    // are bytes of s0/s1, the four j>=4 values are rebuilt bytewise (qwen_cpu/quants.h:33-41).
    const uint32_t Slo = w.s0 & 0x3F3F3F3Fu, Mlo = w.s1 & 0x3F3F3F3Fu;
    const uint32_t Shi = (w.s2 & 0x0F0F0F0Fu) | ((w.s0 >> 2) & 0x30303030u);
    const uint32_t Mhi = ((w.s2 >> 4) & 0x0F0F0F0Fu) | ((w.s1 >> 2) & 0x30303030u);
    const uint32_t S4 = g < 2 ? Slo : Shi, M4 = g < 2 ? Mlo : Mhi;
    const int sh = (g & 1) * 16;
    const float sca = (float)((S4 >> sh) & 0xFFu), scb = (float)((S4 >> (sh + 8)) & 0xFFu);
    const float ma = (float)((M4 >> sh) & 0xFFu), mb = (float)((M4 >> (sh + 8)) & 0xFFu);
    // (1024 + q)*sc - 1024*sc = q*sc and (1024 + 16q)*(sc/16) - 64*sc = q*sc, exact in fp16.
    const _Float16 hla = (_Float16)sca, hlb = (_Float16)(-1024.0f * sca);
    const _Float16 hha = (_Float16)(scb * 0.0625f), hhb = (_Float16)(-64.0f * scb);
    const h2 mlo = {hla, hla}, alo = {hlb, hlb}, mhi = {hha, hha}, ahi = {hhb, hhb};
    const uint32_t W[8] = {w.q0.x, w.q0.y, w.q0.z, w.q0.w, w.q1.x, w.q1.y, w.q1.z, w.q1.w};
    f4 c1 = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const uint32_t a = W[2 * j] & 0x0F0F0F0Fu, b = W[2 * j + 1] & 0x0F0F0F0Fu;
        const h8 A = make_h8(pk_fma(perm_lo(a), mlo, alo), pk_fma(perm_hi(a), mlo, alo), pk_fma(perm_lo(b), mlo, alo),
                             pk_fma(perm_hi(b), mlo, alo));
        c1 = mfma(A, B[j], c1);
    }
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const uint32_t a = W[2 * j] & 0xF0F0F0F0u, b = W[2 * j + 1] & 0xF0F0F0F0u;
        const h8 A = make_h8(pk_fma(perm_lo(a), mhi, ahi), pk_fma(perm_hi(a), mhi, ahi), pk_fma(perm_lo(b), mhi, ahi),
                             pk_fma(perm_hi(b), mhi, ahi));
        c1 = mfma(A, B[4 + j], c1);
    }
    const h2 mm = {(_Float16)ma, (_Float16)mb};
    const h8 Am = make_h8(as_u32(mm), 0u, 0u, 0u);
    const f4 c2 = mfma(Am, B[8], f4{0.0f, 0.0f, 0.0f, 0.0f});
    const uint32_t dd[4] = {w.dd.x, w.dd.y, w.dd.z, w.dd.w};
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float d = h2f_bits(dd[i] & 0xFFFFu), dmin = h2f_bits(dd[i] >> 16);
        acc[i] = fmaf(d, c1[i], acc[i]);
        acc[i] = fmaf(-dmin, c2[i], acc[i]);
    }
    return acc;
}

// One wave writes the image of (super-block sb, token t) at bimg (global or LDS) from its 256
// x values (v: elements 4*lane .. 4*lane+3 of the super-block).
template <int MT>
__device__ inline void prep_q4_store(const f4& v, int t, int lane, uint8_t* bimg) {
    if (t == 0 && lane < 9) *(u4*)(bimg + MT * 1152 + 16 * lane) = u4{0u, 0u, 0u, 0u};
    const int gg = lane >> 4, j = 4 * ((lane >> 3) & 1) + ((lane >> 1) & 3);
    *(uint2*)(bimg + ((gg * 2 * MT + 2 * t) * 9 + j) * 16 + 8 * (lane & 1)) = pack4(v, false);
    *(uint2*)(bimg + ((gg * 2 * MT + 2 * t + 1) * 9 + j) * 16 + 8 * (lane & 1)) = pack4(v, true);
    // sub-block sums: 8 lanes per 32-element sub-block; lane 16gg collects 2gg and 2gg+1
    const float sum = sum8((v.x + v.y) + (v.z + v.w));
    const float odd = dpp_down8(sum);
    if ((lane & 15) == 0) {
        _Float16 h0, l0, h1, l1;
        split_h(sum, h0, l0);
        split_h(odd, h1, l1);
        *(u4*)(bimg + ((gg * 2 * MT + 2 * t) * 9 + 8) * 16) = u4{as_u32(h2{h0, h1}), 0u, 0u, 0u};
        *(u4*)(bimg + ((gg * 2 * MT + 2 * t + 1) * 9 + 8) * 16) = u4{as_u32(h2{l0, l1}), 0u, 0u, 0u};
    }
}

// Issue-only loads, from inline assembly so that the compiler does not count them (its own waits would
// otherwise fall back to vmcnt(0) with LDS-DMAs pending); use only after wait_x.
__device__ inline u4 load16_async_u(const void* p) {
    u4 v;
    asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(v) : "v"(p) : "memory");
    return v;
}
__device__ inline u2 load8_async(const void* p) {
    u2 v;
    asm volatile("global_load_dwordx2 %0, %1, off" : "=v"(v) : "v"(p) : "memory");
    return v;
}
// Wait until at most N vector-memory operations are in flight; v is tied to the wait, so no use of
// it can be placed before.
template <int N, typename V>
__device__ inline void wait_x(V& v) {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%1)" : "+v"(v) : "n"(N) : "memory");
}

__device__ inline f4 load_x_sb(const void* __restrict__ x, int xfmt, int ldx, int sb, int t, int lane) {
    return load_act4(x, xfmt, ldx, t, sb * 256 + 4 * lane);
}

template <int MT>
__device__ inline void prep_q4_sb(const void* __restrict__ x, int xfmt, int ldx, int sb, int t, int lane,
                                  uint8_t* bimg) {
    prep_q4_store<MT>(load_x_sb(x, xfmt, ldx, sb, t, lane), t, lane, bimg);
}

template <int MT>
__global__ __launch_bounds__(64) void k_prep_q4(const void* __restrict__ x, int xfmt, int ldx,
                                                uint8_t* __restrict__ img) {
    prep_q4_sb<MT>(x, xfmt, ldx, blockIdx.x, blockIdx.y, threadIdx.x, img + (size_t)blockIdx.x * q4_img<MT>());
}

// Copies `bytes` (a multiple of 16) from g to lds with LDS-DMA, 1 KiB per instruction.
template <int BYTES>
__device__ inline void dma_bytes(const uint8_t* g, uint8_t* lds, int lane) {
#pragma unroll
    for (int c = 0; c < (BYTES + 1023) / 1024; c++) {
        const int left = BYTES - c * 1024;
        if (left >= 1024 || lane < left / 16) dma16(g + c * 1024 + 16 * lane, lds + c * 1024);
    }
}

template <int NA, int MT, int D>
struct Q4Cfg {
    static constexpr int IMG = q4_img<MT>();
    static constexpr int SLOT = NA * Q4K_GROUP + IMG;
    static constexpr int WAVE_LDS = D * SLOT;
    static constexpr int NDMA = NA * Q4_DMA + (IMG + 1023) / 1024;
};

template <int NA, int MT, int D, int WPG>
__global__ __launch_bounds__(64 * WPG) void k_gemv_q4k(const GemvParams P) {
    using C = Q4Cfg<NA, MT, D>;
    extern __shared__ __align__(16) uint8_t smem[];
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r = lane & 15, g = lane >> 4;
    const int w = blockIdx.x * WPG + wave;
    if (w >= P.waves) return;
    const int u0 = wave_first_unit(P, w), nu = wave_first_unit(P, w + 1) - u0;
    const int M = P.m, nsb = P.nsb;
    uint8_t* ring = smem + wave * C::WAVE_LDS;

    auto issue = [&](int i) {  // unit u0+i -> slot i % D: weight group(s) + the image of its super-block
        const int u = u0 + i, tile = u / nsb, sb = u - tile * nsb;
        uint8_t* slot = ring + (i % D) * C::SLOT;
#pragma unroll
        for (int a = 0; a < NA; a++) dma_q4(unit_group(P, a, tile, sb, Q4K_GROUP), slot + a * Q4K_GROUP, lane);
        dma_bytes<C::IMG>(P.ximg + (size_t)sb * C::IMG, slot + NA * Q4K_GROUP, lane);
    };
    for (int i = 0; i < D - 1 && i < nu; i++) issue(i);

    const int boff = r < 2 * M ? (g * 2 * MT + r) * 144 : MT * 1152;
    const bool holds = (r & 1) == 0 && (r >> 1) < M;  // after the hi/lo pair sum: token r>>1
    f4 acc[NA], pend[2][NA];
#pragma unroll
    for (int a = 0; a < NA; a++) acc[a] = f4{0.0f, 0.0f, 0.0f, 0.0f};
    int ptile[2] = {0, 0}, punits[2] = {0, 0}, npend = 0, piece0 = u0;

    for (int i = 0; i < nu; i++) {
        if (i + D - 1 < nu) {
            issue(i + D - 1);
            wait_vm<(D - 1) * C::NDMA>();
        } else {
            wait_vm_units<C::NDMA>(nu - 1 - i);
        }
        const uint8_t* slot = ring + (i % D) * C::SLOT;
        const uint8_t* bp = slot + NA * Q4K_GROUP + boff;
        h8 B[9];
#pragma unroll
        for (int j = 0; j < 9; j++) B[j] = __builtin_bit_cast(h8, *(const u4*)(bp + 16 * j));
#pragma unroll
        for (int a = 0; a < NA; a++) acc[a] = q4_step(load_q4(slot + a * Q4K_GROUP, lane, r, g), B, acc[a], g);
        lds_order();

        const int u = u0 + i, tile = u / nsb, sb = u - tile * nsb;
        if (sb == nsb - 1 || i == nu - 1) {  // end of this wave's piece of the tile
            f4 v[NA];
#pragma unroll
            for (int a = 0; a < NA; a++)
#pragma unroll
                for (int e = 0; e < 4; e++) v[a][e] = sum2(acc[a][e]);  // hi + lo columns
            if (piece0 == tile * nsb && sb == nsb - 1) {
                if (holds) store_tile<NA>(P, tile, r >> 1, g, v);
            } else {
#pragma unroll
                for (int a = 0; a < NA; a++) pend[npend][a] = v[a];
                ptile[npend] = tile;
                punits[npend] = u - piece0 + 1;
                npend++;
            }
#pragma unroll
            for (int a = 0; a < NA; a++) acc[a] = f4{0.0f, 0.0f, 0.0f, 0.0f};
            piece0 = u + 1;
        }
    }
    finish_pieces<NA, MT>(P, w, npend, ptile, punits, pend, holds, r >> 1, g);
}

// ================================================================================================
// Q6_K
//
// Lane (r, g) holds, per half n of the super-block, ql_r[64n + 32(g>>1) + 16(g&1) + 0..15] and
// qh_r[32n + 16(g&1) + 0..15]: 32 elements of sub-blocks u = g (low nibbles, s = g>>1) and u = g+4
// (high nibbles, s = (g>>1)+2) of the half.  MFMA p (0..3) of the half uses bytes 8(p&1)..+7 and
// nibble p>>1, i.e. sub-block u = g + 4(p>>1).  B columns 2u + {hi, lo}: a lane of column c feeds
// MFMA p only when c>>1 == g + 4(p>>1); all other B lanes read a zero record.
//
// Activation image of one super-block: per (token t, half n) 528 bytes: 16-byte records
// (p*4 + g)*2 + part = x^part[t][sb*256 + 128n + 32*((g>>1) + 2(p>>1)) + 16(g&1) + 8(p&1) + 0..7] and
// a zero record at 512; then floats ((t*2 + n)*8 + u)*2 + part = sum of x^part over sub-block u of
// half n.
struct RawQ6 {
    u4 ql[2], qh[2];
    uint32_t sc[2];  // int8 scales of rows 4g..4g+3 for sub-block 8n + (r>>1)
    u2 dd;           // d of rows 4g..4g+3
};

constexpr int Q6_DMA = 4;  // LDS-DMA instructions per 3360-byte group
__device__ inline void dma_q6(const uint8_t* G, uint8_t* slot, int lane) {
    dma16_stream(G + 16 * lane, slot);
    dma16_stream(G + 1024 + 16 * lane, slot + 1024);
    dma16_stream(G + 2048 + 16 * lane, slot + 2048);
    if (lane < 18) dma16_stream(G + 3072 + 16 * lane, slot + 3072);  // scales (256 B) + d (32 B)
}

__device__ inline RawQ6 load_q6(const uint8_t* G, int lane, int r, int g) {  // G: an LDS ring slot
    RawQ6 w;
    w.ql[0] = ld16(G + 16 * lane);
    w.ql[1] = ld16(G + 1024 + 16 * lane);
    w.qh[0] = ld16(G + 2048 + 16 * (r + 16 * (g & 1)));
    w.qh[1] = ld16(G + 2560 + 16 * (r + 16 * (g & 1)));
    w.sc[0] = ld4(G + 3072 + 32 * g + 4 * (r >> 1));
    w.sc[1] = ld4(G + 3200 + 32 * g + 4 * (r >> 1));
    w.dd = ld8(G + 3328 + 8 * g);
    return w;
}

__device__ inline uint32_t q6_byte(uint32_t L, uint32_t H, int hi_nib, int sp) {
    return hi_nib ? (((L >> 4) & 0x0F0F0F0Fu) | ((H >> (2 * sp)) & 0x30303030u))
                  : ((L & 0x0F0F0F0Fu) | ((H << (4 - 2 * sp)) & 0x30303030u));
}

__device__ inline h8 q6_operand(const u4& L, const u4& H, int p, int sp) {
    const uint32_t lw[4] = {L.x, L.y, L.z, L.w}, hw[4] = {H.x, H.y, H.z, H.w};
    const int w0 = 2 * (p & 1), hn = p >> 1;
    const uint32_t a = q6_byte(lw[w0], hw[w0], hn, sp), b = q6_byte(lw[w0 + 1], hw[w0 + 1], hn, sp);
    return make_h8(perm_lo(a), perm_hi(a), perm_lo(b), perm_hi(b));
}

template <int MT>
__device__ inline void prep_q6_store(const f4& v, int t, int lane, uint8_t* bimg) {
    float* sums = (float*)(bimg + MT * 2 * 528);
    if (lane < 2) *(u4*)(bimg + (t * 2 + lane) * 528 + 512) = u4{0u, 0u, 0u, 0u};
    const int n = lane >> 5, sq = (lane & 31) >> 3;
    const int gg = 2 * (sq & 1) + ((lane & 7) >> 2), p = 2 * (sq >> 1) + ((lane >> 1) & 1);
    uint8_t* rec = bimg + (t * 2 + n) * 528 + ((p * 4 + gg) * 2) * 16 + 8 * (lane & 1);
    *(uint2*)rec = pack4(v, false);
    *(uint2*)(rec + 16) = pack4(v, true);
    float sh = 0.0f, sl = 0.0f;  // sums of the fp16 parts over the 16-element sub-block (4 lanes)
#pragma unroll
    for (int e = 0; e < 4; e++) {
        _Float16 h, l;
        split_h(v[e], h, l);
        sh += (float)h;
        sl += (float)l;
    }
    sh = sum4(sh);
    sl = sum4(sl);
    if ((lane & 3) == 0) {
        const int u = (lane & 31) >> 2;
        sums[((t * 2 + n) * 8 + u) * 2 + 0] = sh;
        sums[((t * 2 + n) * 8 + u) * 2 + 1] = sl;
    }
}

template <int MT>
__device__ inline void prep_q6_sb(const void* __restrict__ x, int xfmt, int ldx, int sb, int t, int lane,
                                  uint8_t* bimg) {
    prep_q6_store<MT>(load_x_sb(x, xfmt, ldx, sb, t, lane), t, lane, bimg);
}

template <int MT>
__global__ __launch_bounds__(64) void k_prep_q6(const void* __restrict__ x, int xfmt, int ldx,
                                                uint8_t* __restrict__ img) {
    prep_q6_sb<MT>(x, xfmt, ldx, blockIdx.x, blockIdx.y, threadIdx.x, img + (size_t)blockIdx.x * q6_img<MT>());
}

template <int NA, int MT, int D>
struct Q6Cfg {
    static constexpr int IMG = q6_img<MT>();
    static constexpr int SLOT = NA * Q6K_GROUP + IMG;
    static constexpr int WAVE_LDS = D * SLOT;
    static constexpr int NDMA = NA * Q6_DMA + (IMG + 1023) / 1024;
};

template <int NA, int MT, int D, int WPG>
__global__ __launch_bounds__(64 * WPG) void k_gemv_q6k(const GemvParams P) {
    using C = Q6Cfg<NA, MT, D>;
    extern __shared__ __align__(16) uint8_t smem[];
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r = lane & 15, g = lane >> 4;
    const int w = blockIdx.x * WPG + wave;
    if (w >= P.waves) return;
    const int u0 = wave_first_unit(P, w), nu = wave_first_unit(P, w + 1) - u0;
    const int M = P.m, nsb = P.nsb;
    uint8_t* ring = smem + wave * C::WAVE_LDS;

    auto issue = [&](int i) {
        const int u = u0 + i, tile = u / nsb, sb = u - tile * nsb;
        uint8_t* slot = ring + (i % D) * C::SLOT;
#pragma unroll
        for (int a = 0; a < NA; a++) dma_q6(unit_group(P, a, tile, sb, Q6K_GROUP), slot + a * Q6K_GROUP, lane);
        dma_bytes<C::IMG>(P.ximg + (size_t)sb * C::IMG, slot + NA * Q6K_GROUP, lane);
    };
    for (int i = 0; i < D - 1 && i < nu; i++) issue(i);

    const int sp = g >> 1, part = r & 1, u = r >> 1;
    int boff[4];  // per MFMA p: this lane's record in a (t, n) group, or the group's zero record
#pragma unroll
    for (int p = 0; p < 4; p++) boff[p] = u == g + 4 * (p >> 1) ? ((p * 4 + g) * 2 + part) * 16 : 512;
    const bool holds = r < M;  // after the 16-column sum: lane r holds token r
    f4 acc[NA][MT], pend[2][NA];
#pragma unroll
    for (int a = 0; a < NA; a++)
#pragma unroll
        for (int t = 0; t < MT; t++) acc[a][t] = f4{0.0f, 0.0f, 0.0f, 0.0f};
    int ptile[2] = {0, 0}, punits[2] = {0, 0}, npend = 0, piece0 = u0;

    for (int i = 0; i < nu; i++) {
        if (i + D - 1 < nu) {
            issue(i + D - 1);
            wait_vm<(D - 1) * C::NDMA>();
        } else {
            wait_vm_units<C::NDMA>(nu - 1 - i);
        }
        const uint8_t* slot = ring + (i % D) * C::SLOT;
        const uint8_t* bimg = slot + NA * Q6K_GROUP;
        const float* sums = (const float*)(bimg + MT * 2 * 528);
        RawQ6 src[NA];
#pragma unroll
        for (int a = 0; a < NA; a++) src[a] = load_q6(slot + a * Q6K_GROUP, lane, r, g);
        h8 A[NA][2][4];
#pragma unroll
        for (int a = 0; a < NA; a++)
#pragma unroll
            for (int n = 0; n < 2; n++)
#pragma unroll
                for (int p = 0; p < 4; p++) A[a][n][p] = q6_operand(src[a].ql[n], src[a].qh[n], p, sp);
#pragma unroll
        for (int t = 0; t < MT; t++) {
            if (MT == 1 || t < M) {
#pragma unroll
                for (int n = 0; n < 2; n++) {
                    const uint8_t* grp = bimg + (t * 2 + n) * 528;
                    h8 B[4];
#pragma unroll
                    for (int p = 0; p < 4; p++) B[p] = __builtin_bit_cast(h8, *(const u4*)(grp + boff[p]));
                    const float sx = 1056.0f * sums[((t * 2 + n) * 8 + u) * 2 + part];
#pragma unroll
                    for (int a = 0; a < NA; a++) {
                        f4 c = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                        for (int p = 0; p < 4; p++) c = mfma(A[a][n][p], B[p], c);
                        const uint32_t scw = src[a].sc[n];
                        const uint32_t dw[2] = {src[a].dd.x, src[a].dd.y};
#pragma unroll
                        for (int e = 0; e < 4; e++) {
                            const float d = h2f_bits((dw[e >> 1] >> (16 * (e & 1))) & 0xFFFFu);
                            const float sc = (float)(int)(int8_t)(scw >> (8 * e));
                            acc[a][t][e] = fmaf(d * sc, c[e] - sx, acc[a][t][e]);
                        }
                    }
                }
            }
        }
        lds_order();

        const int uu = u0 + i, tile = uu / nsb, sb = uu - tile * nsb;
        if (sb == nsb - 1 || i == nu - 1) {
            f4 v[NA];  // lane r keeps token r after summing the 16 (sub-block, hi/lo) columns
#pragma unroll
            for (int a = 0; a < NA; a++) {
                v[a] = f4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int t = 0; t < MT; t++)
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        const float x = sum16(acc[a][t][e]);
                        if (r == t) v[a][e] = x;
                    }
            }
            if (piece0 == tile * nsb && sb == nsb - 1) {
                if (holds) store_tile<NA>(P, tile, r, g, v);
            } else {
#pragma unroll
                for (int a = 0; a < NA; a++) pend[npend][a] = v[a];
                ptile[npend] = tile;
                punits[npend] = uu - piece0 + 1;
                npend++;
            }
#pragma unroll
            for (int a = 0; a < NA; a++)
#pragma unroll
                for (int t = 0; t < MT; t++) acc[a][t] = f4{0.0f, 0.0f, 0.0f, 0.0f};
            piece0 = uu + 1;
        }
    }
    finish_pieces<NA, MT>(P, w, npend, ptile, punits, pend, holds, r, g);
}

// ================================================================================================
// Single-token GEMV (m <= 4): x in LDS as three int8 parts, integer MFMA, a static split of the units.
//
// Units are ordered slice-major: k is cut into S slices of cs super-blocks, and group q = s * ntiles
// + tile holds the cs units (tile, s*cs + j).  One work-group per CU owns a contiguous range of
// units, so it touches one or two slices and converts only those super-blocks of x into the A-
// operand image in LDS (no prepass kernel).  Wave w of W takes positions w, w + W, w + 2W, ... of the
// range (the same every run), keeping D units' weights in flight through its LDS-DMA ring; a table
// built in the prologue gives each position's weight address and fields, which the wave holds in
// registers 64 positions at a time.  Each unit's 16 row sums go to an LDS slot indexed by the unit,
// and after the loop one wave per group adds that group's unit sums in unit order (deterministic).
// A tile held whole by the range is stored; otherwise the sums pair up by device-scope exchanges
// (xcombine): a group's two pieces, when two ranges share it, then the slices' sums along a binary
// tree, each pair added by whichever partner arrives second (one round trip per level,
// deterministic).
// ------------------------------------------------------------------------------------------------
// Integer form of a unit for the single-token kernel, for MT (1, 2 or 4) tokens.  The weights are the
// B operand of v_mfma_i32_16x16x64_i8: lane (g, r) holds 16 int8 weights of row r for the MFMA's k-
// group g.  x is the A operand, each token split into XP = 3 int8 parts with one triple of scales per
// super-block,
//   x ~= s0 x_0 + s1 x_1 + s2 x_2,  s0 = max|x| / 127,  s1 = s0 / 254,  s2 = s1 / 254,
//   |error| <= max|x| / 16387064 per element,
// so an element far below its super-block's largest (an outlier 10^5 times the rest) still keeps ~24
// bits.  (Token u, part h) is slot i = 3u + h; slot i sits in A row 4g + (i & 3) of MFMA i >> 2, and
// only for the k-group g it multiplies, so that D row 4g + (i & 3) of lane (g, r) is row r's dot
// product of that part with the 16 elements lane group g holds.  NP = ceil(3 MT / 4) MFMAs per step:
// one token (rows 4g + 3 stay at zero), two tokens in two MFMAs, four in three.  Each lane then
// applies its row's sub-block scale in int32 (exact) and d, dmin and the x scales in fp32.
//
// Image of one super-block (img8<TYPE, MT>() bytes; A8 = a8_t<MT>() bytes per MFMA step):
//   [t*A8 + ((g*MT + u)*3 + h)*16, +16): x_h of token u at the 16 elements k-group g supplies to step t,
//   [t*A8 + 192*MT, +16): zeros (read by the A lanes of rows that carry no x),
//   [S + 16u, +16): s0, s1, s2, f of token u (fp32), S = 4*A8; a non-finite x makes s0..s2 NaN; f is
//     2^-100 for a super-block converted from x * 2^100 (largest |x| below 2^-100), else 1,
//   Q4_K/Q5_K [SX + 32u, +32): sums of x over the eight 32-element sub-blocks (fp32, the min term),
//   Q6_K [SX + 64u, +64): sums of x over the sub-block of (g, t), fp32 [g][t] (the -32 offset);
//   SX = S + 16*MT.
// Elements of (g, t): Q4_K/Q5_K 64g + 32(t >> 1) + 16(t & 1) + e (chunk g of the 128 qs bytes: low
// nibbles are sub-block 2g, high nibbles 2g + 1; qwen_cpu/quants.h:53-94), Q6_K 128(g >> 1) + 32t +
// 16(g & 1) + e (quarter t of half g >> 1; qwen_cpu/quants.h:96-121), Q8_0 64t + 16g + e (block
// 2t + (g >> 1) of the run; qwen_cpu/quants.h:45-51).
typedef int i4 __attribute__((ext_vector_type(4)));
constexpr int XP = 3;  // int8 parts per activation element
template <int MT>
constexpr int np_of() { return (XP * MT + 3) / 4; }  // MFMAs per step
template <int MT>
constexpr int a8_t() { return 64 * XP * MT + 16; }
template <int MT>
constexpr int img8_s() { return 4 * a8_t<MT>(); }
template <int MT>
constexpr int img8_sx() { return img8_s<MT>() + 16 * MT; }
template <int TYPE, int MT>
constexpr int img8() {
    return TYPE == T_Q8_0 ? img8_sx<MT>() : img8_sx<MT>() + (TYPE == T_Q6_K ? 64 : 32) * MT;
}
static_assert(img8<T_Q4_K, 1>() == 880 && img8<T_Q6_K, 1>() == 912 && img8<T_Q8_0, 1>() == 848, "image sizes");

__device__ inline i4 mfma8(const i4& a, const i4& b, const i4& c) {
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}
__device__ inline i4 ld16i(const uint8_t* p) { return *(const i4*)p; }

// A-operand offset of this lane inside a super-block's image for MFMA p of a step: row 4g + j of
// k-group g reads the record of slot 4p + j (token u, part h), every other lane the zero record.
template <int MT>
__device__ inline int a8_offset(int lane, int p) {
    const int m = lane & 15, kg = lane >> 4, i = 4 * p + (m & 3);
    const bool live = (m >> 2) == kg && i < XP * MT;
    return live ? (kg * MT * XP + i) * 16 : 64 * XP * MT;
}

// Cross-row exchanges without the LDS: permlane16/32_swap(x, x) return the two halves whose sum
// (or max) is the xor-16 (xor-32) reduction in every lane.
__device__ inline float xor16_sum(float v) {
    const auto p = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(int, v), __builtin_bit_cast(int, v), false, false);
    return __builtin_bit_cast(float, (int)p[0]) + __builtin_bit_cast(float, (int)p[1]);
}
__device__ inline float xor32_sum(float v) {
    const auto p = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(int, v), __builtin_bit_cast(int, v), false, false);
    return __builtin_bit_cast(float, (int)p[0]) + __builtin_bit_cast(float, (int)p[1]);
}
__device__ inline uint32_t xor16_umax(uint32_t v) {
    const auto p = __builtin_amdgcn_permlane16_swap((int)v, (int)v, false, false);
    return max((uint32_t)p[0], (uint32_t)p[1]);
}
__device__ inline uint32_t xor32_umax(uint32_t v) {
    const auto p = __builtin_amdgcn_permlane32_swap((int)v, (int)v, false, false);
    return max((uint32_t)p[0], (uint32_t)p[1]);
}
// Sum over the four 16-lane groups (lanes r, r + 16, r + 32, r + 48), in every lane.
__device__ inline float sum_groups(float v) { return xor32_sum(xor16_sum(v)); }
// Two values reduced at once: lanes 0..31 get a[l] + a[l + 32], lanes 32..63 get b[l - 32] + b[l]
// (one permlane32 swap and one add for both).
__device__ inline float swap32_sum(float a, float b) {
    const auto p = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(int, a), __builtin_bit_cast(int, b), false, false);
    return __builtin_bit_cast(float, (int)p[0]) + __builtin_bit_cast(float, (int)p[1]);
}
// The same over 16-lane rows: rows 0 and 2 get a summed with the next row, rows 1 and 3 b summed
// with the row before.
__device__ inline float swap16_sum(float a, float b) {
    const auto p = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(int, a), __builtin_bit_cast(int, b), false, false);
    return __builtin_bit_cast(float, (int)p[0]) + __builtin_bit_cast(float, (int)p[1]);
}
// A unit's NC columns of row partial sums (lane group g holds k-group g's part of row r) summed over
// the four lane groups and stored at part[c * 16 + r].  A reduce-scatter: the xor-32 level pairs
// column i with i + NC/2 and the xor-16 level column j with j + NC/4, each swap reducing two columns
// at once, so that lane group G ends with columns 2G, 2G + 1 (NC = 8), column G (NC = 4) or column
// G >> 1 (NC = 2, groups 0 and 2 store): 12 operations for eight columns where eight full
// reductions took 48.  Each sum adds (g0 + g2) + (g1 + g3), the same order in every lane.
template <int NC>
__device__ inline void store_sums(const float (&c)[NC], float* part, int lane) {
    const int r = lane & 15, G = lane >> 4;
    if constexpr (NC == 1) {
        const float v = sum_groups(c[0]);
        if (lane < 16) part[r] = v;
    } else if constexpr (NC == 2) {
        const float v = xor16_sum(swap32_sum(c[0], c[1]));
        if ((G & 1) == 0) part[(G >> 1) * 16 + r] = v;
    } else if constexpr (NC == 4) {
        part[G * 16 + r] = swap16_sum(swap32_sum(c[0], c[2]), swap32_sum(c[1], c[3]));
    } else if constexpr (NC == 8) {
        float w[4];
#pragma unroll
        for (int i = 0; i < 4; i++) w[i] = swap32_sum(c[i], c[i + 4]);
        part[(2 * G) * 16 + r] = swap16_sum(w[0], w[2]);
        part[(2 * G + 1) * 16 + r] = swap16_sum(w[1], w[3]);
    } else {
        // sixteen columns (the gate/up pair at eight tokens): the xor-32 level pairs i with i + 8, the
        // xor-16 level j with j + 4, so that lane group G ends with columns i + 4G, i = 0..3
        static_assert(NC == 16, "columns");
        float w[8];
#pragma unroll
        for (int i = 0; i < 8; i++) w[i] = swap32_sum(c[i], c[i + 8]);
#pragma unroll
        for (int i = 0; i < 4; i++) part[(i + 4 * G) * 16 + r] = swap16_sum(w[i], w[i + 4]);
    }
}
// Largest of the wave's unsigned values, in every lane.
template <int CTRL>
__device__ inline uint32_t dpp_max_u(uint32_t v) {
    const uint32_t o = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, false);
    return v > o ? v : o;
}
__device__ inline uint32_t wave_max_u(uint32_t v) {
    v = dpp_max_u<0xB1>(v);   // quad_perm xor 1
    v = dpp_max_u<0x4E>(v);   // quad_perm xor 2
    v = dpp_max_u<0x141>(v);  // row_half_mirror
    v = dpp_max_u<0x140>(v);  // row_mirror
    return xor32_umax(xor16_umax(v));
}
// Low bytes of four ints, in order, with two byte permutes.
__device__ inline uint32_t pack_i8(int a, int b, int c, int d) {
    const uint32_t lo = __builtin_amdgcn_perm((uint32_t)b, (uint32_t)a, 0x0C0C0400u);  // a.b0, b.b0, 0, 0
    const uint32_t hi = __builtin_amdgcn_perm((uint32_t)d, (uint32_t)c, 0x04000C0Cu);  // 0, 0, c.b0, d.b0
    return lo | hi;
}
__device__ inline uint32_t abs_bits(float v) { return __builtin_bit_cast(uint32_t, v) & 0x7FFFFFFFu; }

// One wave writes token u's part of the image of one super-block from its 256 x values (v: elements
// 4 lane .. 4 lane + 3).
template <int TYPE, int MT>
__device__ inline void prep8_store(const f4& v0, int lane, uint8_t* img, int u) {
    constexpr int A8 = a8_t<MT>(), S = img8_s<MT>(), SX = img8_sx<MT>();
    // largest |x| as a bit pattern, where NaN orders above inf above every finite value (a float
    // max would drop a NaN)
    const uint32_t amb = wave_max_u(max(max(abs_bits(v0.x), abs_bits(v0.y)), max(abs_bits(v0.z), abs_bits(v0.w))));
    // A super-block whose largest |x| is below 2^-100 (fp32 subnormals included) is converted from x
    // times 2^100, which is exact, so that s0, s1 and s2 stay normal; its fourth scale 2^-100 (else
    // 1) multiplies the unit's result back, and its x sums are of the scaled values too.  One with a
    // NaN or an inf gets NaN scales, so every output it feeds is NaN, as the reference's float paths
    // give a non-finite result (its parts are zeros).
    const bool fin = amb < 0x7F800000u, tiny = amb != 0u && amb < 0x0D800000u;  // 0x0D800000 = 2^-100
    const float up = tiny ? 0x1p100f : 1.0f;
    const f4 v = {v0.x * up, v0.y * up, v0.z * up, v0.w * up};
    const float am = __builtin_bit_cast(float, amb) * up;
    // |x| * r0 stays below 127.0001, and each residual times the next reciprocal below 127.02
    // (1-ulp reciprocals, round-to-nearest products, fused residuals), so every part rounds to at
    // most 127 in magnitude without a clamp; the parts are rebuilt with s0, s1, s2 themselves, so
    // the reciprocals need not be exact.
    const bool nz = fin && amb != 0u;
    const float s0 = !fin ? __builtin_nanf("") : nz ? am * (1.0f / 127.0f) : 1.0f;
    const float s1 = s0 * (1.0f / 254.0f), s2 = s1 * (1.0f / 254.0f);
    const float r0 = nz ? 127.0f * __builtin_amdgcn_rcpf(am) : 0.0f;
    const float r1 = fin ? 254.0f * __builtin_amdgcn_rcpf(s0) : 0.0f, r2 = fin ? 254.0f * __builtin_amdgcn_rcpf(s1) : 0.0f;
    // Rounding by the 1.5 * 2^23 shift: fma(v, r, M) rounds v * r to the nearest integer (ties to even)
    // and holds it in its low mantissa bits, so its low byte is already that integer as int8 (|h| <=
    // 127) and (t - M) is the integer as a float, exactly: three instructions per part instead of
    // a multiply, a rint and a conversion.
    constexpr float M = 12582912.0f;
    uint32_t x0[4], x1[4], x2[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float t0 = fmaf(v[i], r0, M);
        const float e0 = fmaf(-s0, t0 - M, v[i]);
        const float t1 = fmaf(e0, r1, M);
        const float e1 = fmaf(-s1, t1 - M, e0);
        x0[i] = __builtin_bit_cast(uint32_t, t0);
        x1[i] = __builtin_bit_cast(uint32_t, t1);
        x2[i] = __builtin_bit_cast(uint32_t, fmaf(e1, r2, M));
    }
    const int e0 = 4 * lane;
    constexpr bool K4 = TYPE == T_Q4_K || TYPE == T_Q5_K;
    const int kg = K4 ? e0 >> 6 : TYPE == T_Q8_0 ? (e0 >> 4) & 3 : 2 * (e0 >> 7) + ((e0 >> 4) & 1);
    const int t = K4 ? (e0 >> 4) & 3 : TYPE == T_Q8_0 ? e0 >> 6 : (e0 >> 5) & 3;
    uint8_t* rec = img + t * A8 + (kg * MT + u) * (16 * XP) + (e0 & 15);
    lds_st32(rec, pack_i8((int)x0[0], (int)x0[1], (int)x0[2], (int)x0[3]));
    lds_st32(rec + 16, pack_i8((int)x1[0], (int)x1[1], (int)x1[2], (int)x1[3]));
    lds_st32(rec + 32, pack_i8((int)x2[0], (int)x2[1], (int)x2[2], (int)x2[3]));
    if (u == 0 && lane < 4) lds_st128(img + lane * A8 + 64 * XP * MT, u4{0u, 0u, 0u, 0u});
    if (lane == 0)
        lds_st128(img + S + 16 * u, u4{__builtin_bit_cast(uint32_t, s0), __builtin_bit_cast(uint32_t, s1),
                                       __builtin_bit_cast(uint32_t, s2), tiny ? 0x0D800000u : 0x3F800000u});
    if constexpr (K4) {
        const float sum = sum8((v.x + v.y) + (v.z + v.w));  // 32-element sub-block of lanes 8j .. 8j + 7
        if ((lane & 7) == 0) lds_st32(img + SX + 32 * u + 4 * (lane >> 3), __builtin_bit_cast(uint32_t, sum));
    } else if constexpr (TYPE == T_Q6_K) {
        const float sum = sum4((v.x + v.y) + (v.z + v.w));  // 16-element sub-block of lanes 4j .. 4j + 3
        if ((lane & 3) == 0) lds_st32(img + SX + 64 * u + (kg * 4 + t) * 4, __builtin_bit_cast(uint32_t, sum));
    }
}

// A operand of MFMA p of step t, read from the LDS image where it is used (keeping all NP x 4 of them
// live pushes the four-token gate/up pair past 128 VGPRs).
template <int MT>
__device__ inline i4 a_op(const uint8_t* simg, const int (&aoff)[np_of<MT>()], int p, int t) {
    return ld16i(simg + aoff[p] + t * a8_t<MT>());
}

// Int8 dot product of slot i = 3u + h (token u, part h) among the NP results of one MFMA step (i is a
// constant after unrolling).
template <int NP>
__device__ inline int slot_of(const i4 (&c)[NP], int i) { return c[i >> 2][i & 3]; }

// Sums of one unit: v[a][u] = lane (g, r)'s part of row r of stream a, token u (the caller adds the
// four groups).
// Q4_K, and Q5_K with the fifth bit of each quant or-ed in from the qh plane (qh_r[l] bit 2g + h for
// element 64g + 32h + l; qwen_cpu/quants.h:73-94): lane (g, r) reads qh_r[0..15] and qh_r[16..31]
// and its four MFMA steps take bits 2g (t < 2) and 2g + 1 (t >= 2) of them.
template <int TYPE, int NA, int MT>
__device__ inline void q45_unit8(const uint8_t* slot, const uint8_t* simg, const int (&aoff)[np_of<MT>()], int lane,
                                 int r, int g, float (&v)[NA][MT]) {
    constexpr int NP = np_of<MT>(), GB = group_bytes(TYPE);
    const int sh = 16 * (g & 1);
    const uint32_t M = 0x0F0F0F0Fu, B1 = 0x01010101u;
    const i4 zero = {0, 0, 0, 0};
#pragma unroll
    for (int a = 0; a < NA; a++) {
        if (a > 0) lds_order();  // the second stream reads its A operands again
        const uint8_t* G = slot + a * GB;
        const u4 q0 = ld16(G + 16 * lane), q1 = ld16(G + 1024 + 16 * lane);  // qs of row r, chunk g
        const uint32_t s0 = ld4(G + 2112 + 12 * r), s1 = ld4(G + 2116 + 12 * r), s2 = ld4(G + 2120 + 12 * r);
        const uint32_t dd = ld4(G + 2048 + 4 * r);
        // B operand of step t, built right before its MFMAs: low (t < 2) or high nibbles of qs half
        // t & 1, with Q5_K's fifth bit (its qh half read where used: the four-token gate/up pair has
        // no registers to hold both halves through the unit)
        auto bop = [&](int t) __attribute__((always_inline)) {
            const u4 q = (t & 1) ? q1 : q0;
            u4 b = (t < 2 ? q : q >> 4) & M;
            if constexpr (TYPE == T_Q5_K) {
                const u4 h = ld16(G + 2304 + 256 * (t & 1) + 16 * r) >> (2 * g);
                b |= t < 2 ? (h & B1) << 4 : (h << 3) & (B1 << 4);
            }
            return __builtin_bit_cast(i4, b);
        };
        // 6-bit scales and mins of sub-blocks 2g, 2g + 1 (qwen_cpu/quants.h:33-41, four at a time)
        const uint32_t S = g < 2 ? s0 & 0x3F3F3F3Fu : (s2 & 0x0F0F0F0Fu) | ((s0 >> 2) & 0x30303030u);
        const uint32_t Mn = g < 2 ? s1 & 0x3F3F3F3Fu : ((s2 >> 4) & 0x0F0F0F0Fu) | ((s1 >> 2) & 0x30303030u);
        const int sc0 = (S >> sh) & 0xFF, sc1 = (S >> (sh + 8)) & 0xFF;
        const float m0 = (float)((Mn >> sh) & 0xFF), m1 = (float)((Mn >> (sh + 8)) & 0xFF);
        const float d = h2f_bits(dd & 0xFFFFu), dmin = h2f_bits(dd >> 16);
        // Eight token slots run as two halves of four tokens (MFMAs 3h .. 3h + 2 carry tokens 4h ..
        // 4h + 3), so that only half the int32 sums are live at a time (all six MFMAs' sums of both
        // sub-blocks spilled the gate/up pair); each half's A operands are loaded where its MFMAs run.
        constexpr int NH = MT == 8 ? 2 : 1, NPH = NP / NH, TPH = MT / NH;
        static_assert(NH == 1 || (NPH * NH == NP && TPH * XP == 4 * NPH), "a half holds whole tokens");
#pragma unroll
        for (int hh = 0; hh < NH; hh++) {
            auto step_fence = [&]() __attribute__((always_inline)) {
                if constexpr (MT == 8) __builtin_amdgcn_sched_barrier(0);
            };
            i4 c0[NPH], c1[NPH];
#pragma unroll
            for (int p = 0; p < NPH; p++) c0[p] = mfma8(a_op<MT>(simg, aoff, hh * NPH + p, 0), bop(0), zero);
            step_fence();
#pragma unroll
            for (int p = 0; p < NPH; p++) c0[p] = mfma8(a_op<MT>(simg, aoff, hh * NPH + p, 1), bop(1), c0[p]);  // sub-block 2g
            step_fence();
#pragma unroll
            for (int p = 0; p < NPH; p++) c1[p] = mfma8(a_op<MT>(simg, aoff, hh * NPH + p, 2), bop(2), zero);
            step_fence();
#pragma unroll
            for (int p = 0; p < NPH; p++) c1[p] = mfma8(a_op<MT>(simg, aoff, hh * NPH + p, 3), bop(3), c1[p]);  // sub-block 2g + 1
            step_fence();
#pragma unroll
            for (int uu = 0; uu < TPH; uu++) {
                const int u = hh * TPH + uu;
                // x scales and the x sums of sub-blocks 2g, 2g + 1, read where used
                const f4 xs = *(const f4*)(simg + img8_s<MT>() + 16 * u);
                const float2 sx = *(const float2*)(simg + img8_sx<MT>() + 32 * u + 8 * g);
                float part[XP];
#pragma unroll
                for (int h = 0; h < XP; h++)
                    part[h] = (float)(__mul24(sc0, slot_of(c0, XP * uu + h)) + __mul24(sc1, slot_of(c1, XP * uu + h)));
                v[a][u] = xs[3] * fmaf(d, fmaf(xs[0], part[0], fmaf(xs[1], part[1], xs[2] * part[2])),
                                       -dmin * fmaf(m0, sx.x, m1 * sx.y));
            }
        }
    }
}

// Q8_0: the quants are the int8 B operand as stored; step t covers block 2t + (g >> 1) of the run, whose
// fp16 d scales that step's dot products (qwen_cpu/quants.h:45-51).
template <int NA, int MT>
__device__ inline void q8_unit8(const uint8_t* slot, const uint8_t* simg, const int (&aoff)[np_of<MT>()], int lane,
                                int r, int g, float (&v)[NA][MT]) {
    constexpr int NP = np_of<MT>();
    const i4 zero = {0, 0, 0, 0};
#pragma unroll
    for (int a = 0; a < NA; a++) {
        if (a > 0) lds_order();  // the second stream reads its A operands again
        const uint8_t* G = slot + a * Q8_GROUP;
        const u2 dd = ld8(G + 4096 + 16 * r + 8 * (g >> 1));  // d of blocks g >> 1, 2 + .., 4 + .., 6 + ..
        float acc[MT][XP];
#pragma unroll
        for (int u = 0; u < MT; u++)
#pragma unroll
            for (int h = 0; h < XP; h++) acc[u][h] = 0.0f;
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const i4 B = ld16i(G + 1024 * t + 16 * lane);
            const float d = h2f_bits((dd[t >> 1] >> (16 * (t & 1))) & 0xFFFFu);
            i4 c[NP];
#pragma unroll
            for (int p = 0; p < NP; p++) c[p] = mfma8(a_op<MT>(simg, aoff, p, t), B, zero);
#pragma unroll
            for (int u = 0; u < MT; u++)
#pragma unroll
                for (int h = 0; h < XP; h++) acc[u][h] = fmaf(d, (float)slot_of(c, XP * u + h), acc[u][h]);
        }
#pragma unroll
        for (int u = 0; u < MT; u++) {
            const f4 xs = *(const f4*)(simg + img8_s<MT>() + 16 * u);
            v[a][u] = xs[3] * fmaf(xs[0], acc[u][0], fmaf(xs[1], acc[u][1], xs[2] * acc[u][2]));
        }
    }
}

// Q6_K: B = the 6-bit quants q (0..63) as bytes; a step's dot products take the int8 scale of the
// step's 16-element sub-block in int32, and the -32 offset of q enters as 32 * sc * (sum of x over
// the sub-block) in fp32: w x = d sc (q x - 32 x) (qwen_cpu/quants.h:96-121).
template <int NA, int MT>
__device__ inline void q6_unit8(const uint8_t* slot, const uint8_t* simg, const int (&aoff)[np_of<MT>()], int lane,
                                int r, int g, float (&v)[NA][MT]) {
    constexpr int NP = np_of<MT>();
    const int n2 = g >> 1, gb = g & 1;
    const uint32_t M = 0x0F0F0F0Fu, H = 0x30303030u;
    const i4 zero = {0, 0, 0, 0};
#pragma unroll
    for (int a = 0; a < NA; a++) {
        if (a > 0) lds_order();  // the second stream reads its A operands again
        const uint8_t* G = slot + a * Q6K_GROUP;
        const u4 La = ld16(G + 1024 * n2 + 16 * (16 * gb + r));        // ql[l],      l = 16 gb + e
        const u4 Lb = ld16(G + 1024 * n2 + 16 * (16 * (2 + gb) + r));  // ql[l + 32]
        const u4 Q = ld16(G + 2048 + 512 * n2 + 16 * (r + 16 * gb));    // qh[l]
        const uint8_t* scp = G + 3072 + 128 * n2 + 32 * (r >> 2) + 4 * gb + (r & 3);  // sc[8 n2 + 2t + gb]
        const float d = h2f_bits(*(const uint16_t*)(G + 3328 + 2 * r));
        const u4 B[4] = {(La & M) | ((Q << 4) & H), (Lb & M) | ((Q << 2) & H), ((La >> 4) & M) | (Q & H),
                         ((Lb >> 4) & M) | ((Q >> 2) & H)};
        int acc[MT][XP];
        float scs[4];
#pragma unroll
        for (int u = 0; u < MT; u++)
#pragma unroll
            for (int h = 0; h < XP; h++) acc[u][h] = 0;
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const int sc = (int)*(const int8_t*)(scp + 8 * t);
            i4 c[NP];
#pragma unroll
            for (int p = 0; p < NP; p++) c[p] = mfma8(a_op<MT>(simg, aoff, p, t), __builtin_bit_cast(i4, B[t]), zero);
#pragma unroll
            for (int u = 0; u < MT; u++)
#pragma unroll
                for (int h = 0; h < XP; h++) acc[u][h] += __mul24(sc, slot_of(c, XP * u + h));
            scs[t] = (float)sc;
        }
#pragma unroll
        for (int u = 0; u < MT; u++) {
            const f4 xs = *(const f4*)(simg + img8_s<MT>() + 16 * u);
            const f4 sx = *(const f4*)(simg + img8_sx<MT>() + 64 * u + 16 * g);  // x sums of this group's sub-blocks
            const float off = fmaf(scs[0], sx[0], fmaf(scs[1], sx[1], fmaf(scs[2], sx[2], scs[3] * sx[3])));
            v[a][u] = xs[3] * (d * fmaf(xs[0], (float)acc[u][0],
                                        fmaf(xs[1], (float)acc[u][1], fmaf(xs[2], (float)acc[u][2], -32.0f * off))));
        }
    }
}

template <int TYPE, int MT>
struct G1 {
    static constexpr int GB = group_bytes(TYPE);
    static constexpr int IMG = img8<TYPE, MT>();
    static constexpr int DMA = (GB + 1023) / 1024;  // LDS-DMA instructions per group
};

// dma16_stream on lanes 0 .. LANES - 1 only, with the lane mask applied inside the assembly: a
// lane-masked call in C++ becomes an exec-skip branch around the DMA, and on that (never taken)
// path the vmcnt waits that count this DMA would no longer cover the loads they wait for, so the
// code could not be checked path by path.  exec is restored before the statement ends.
template <int LANES>
__device__ inline void dma16_stream_lanes(const void* g, uint8_t* lds) {
    static_assert(LANES > 0 && LANES < 64, "a partial wave");
    constexpr uint64_t MASK = (1ull << LANES) - 1;
    uint64_t saved;
    asm volatile("s_and_saveexec_b64 %0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off nt\n\ts_mov_b64 exec, %0"
                 : "=&s"(saved)
                 : "v"(g), "s"(MASK), "{m0}"(lds_addr(lds))
                 : "memory", "scc");
}

// One weight group into an LDS slot: 1 KiB per instruction, the last one on the lanes it needs
// (every instruction has live lanes, so each one counts once on vmcnt), with no branch.
template <int GB>
__device__ inline void dma_group(const uint8_t* G, uint8_t* slot, int lane) {
    static_assert(GB % 16 == 0, "16-byte pieces");
    constexpr int FULL = GB / 1024, TAIL = (GB % 1024) / 16;
#pragma unroll
    for (int c = 0; c < FULL; c++) dma16_stream(G + c * 1024 + 16 * lane, slot + c * 1024);
    if constexpr (TAIL > 0) dma16_stream_lanes<TAIL>(G + FULL * 1024 + 16 * lane, slot + FULL * 1024);
}

// Eight token slots: at most 12 waves per work-group (170 VGPRs; the gate/up pair needs more than
// 128, and the LDS leaves such a plan fewer waves than that anyway).
template <int MT>
constexpr int gemv1_max_waves() { return MT == 8 ? 12 : 16; }

template <int TYPE, int NA, int D, int XM, int ST, int MT>
__global__ __launch_bounds__(64 * gemv1_max_waves<MT>()) void k_gemv1(const GemvParams P) {
    static_assert(D <= 3, "ring units are packed into one 64-bit register");
    // ST static units per wave (positions wave + i * waves): PRE of them go out ahead of the x
    // conversion, the rest right after it, before the barrier
    static_assert((ST == 2 || ST == 3) && ST <= D, "static units fit the ring");
    constexpr int PRE = ST == 3 ? 1 : 2;
    using C = G1<TYPE, MT>;
    constexpr int NP = np_of<MT>();
    constexpr int NDMA = NA * C::DMA;
    extern __shared__ __align__(16) uint8_t smem[];
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nwaves = P.wpg;
    const int r = lane & 15, g = lane >> 4;
    // units in slice-major order: group q = s * ntiles + tile holds the CS units (tile, s*CS + j)
    const int CS = P.cs, S = P.slices, ntiles = P.ntiles, b = blockIdx.x;
    const int u0 = range_start(P, b), u1 = range_start(P, b + 1), nu = u1 - u0;
    const int qf = u0 / CS, ql = (u1 - 1) / CS;  // groups of this work-group's range
    const int sb0 = (qf / ntiles) * CS, nimg = (ql / ntiles - qf / ntiles + 1) * CS;  // its super-blocks
    uint8_t* img = smem;
    float* part = (float*)(smem + P.lds_part);  // [unit][NA][MT][16] row sums
    u4* tab = (u4*)(smem + P.lds_tab);          // per position: the unit's entry (below)
    int* next = (int*)(smem + P.lds_cnt);       // hand-out counter of the dynamic positions
    uint8_t* ring = smem + P.lds_ring + wave * (D * NA * C::GB);
    constexpr int SLOT = NA * C::GB;
    // matrix 1 of a GLU pair sits at the same offset from its own base
    const ptrdiff_t wdelta = NA == 2 ? P.w[1] - P.w[0] : 0;

    // position order: the last group's units first when that group is shared with the next range
    const int nb = (ql > qf && u1 % CS) ? u1 - ql * CS : 0;
    auto rel_of = [&](int p) __attribute__((always_inline)) { return p < nb ? (ql * CS - u0) + p : p - nb; };
    // Positions [0, SC * W) are static, wave w taking w, w + W, w + 2W, ...: no hand-out and no table
    // read before their DMAs.  The last ~nu >> dshift go out from an LDS counter, so that the waves
    // a SIMD serves late (the youngest) take fewer of them.
    const int SC = max(ST, (nu - (nu >> P.dshift)) / nwaves);
    const int nst = wave < nu ? min(SC, (nu - 1 - wave) / nwaves + 1) : 0;  // this wave's static units

    // DMA of this wave's unit i < ST into ring slot i, before the table exists; for i >= nst a
    // stand-in (the range's last unit, into a slot no unit reads) that keeps the prologue's memory
    // operations unconditional, so that the waits below can count them exactly
    auto issue_static = [&](int i) __attribute__((always_inline)) {
        const int ru = rel_of(min(wave + i * nwaves, nu - 1)), u = u0 + ru, q = u / CS, s = q / ntiles,
                  tile = q - s * ntiles;
        const int sb = s * CS + (u - q * CS);
        const uint8_t* G = unit_group(P, 0, tile, sb, C::GB);
#pragma unroll
        for (int a = 0; a < NA; a++) dma_group<C::GB>(G + a * wdelta, ring + i * SLOT + a * C::GB, lane);
    };

    // x first: its loads go out ahead of this wave's weight DMAs (returns are in order) instead of
    // queueing behind the GPU-wide burst of them.  The DMAs of each wave's first ST units go out
    // before the table exists: PRE of them with the x loads, the others as soon as this wave's part of
    // the image is written, so that the whole ring is in flight when the barrier publishes the image
    // and the table.  (With three units ahead, the first x loads would wait behind three units'
    // DMAs: one goes ahead, two after.  Measured on MI355X, K=17408 N=5120 Q6_K: 17.4 us against 19.2
    // with two units issued ahead of x; waves with fewer than three units keep two ahead of x.)
    // XM conversion jobs per wave, job j = wave + i * waves = MT * sb + u (token u, super-block sb;
    // nimg * MT <= XM * waves, see plan; MT is a power of two, so no division); loads past the last
    // job repeat it, tokens past m read token m - 1 and convert zeros.  The prologue is instantiated
    // once per activation width (fp32: 16 bytes per lane, fp16: 8), so that each form holds only its
    // own load registers and both issue one load per job (the waits below count them).
    auto prologue = [&](auto half) __attribute__((always_inline)) {
        constexpr bool H = decltype(half)::value;
        using XR = std::conditional_t<H, u2, u4>;
        XR xv[XM];
#pragma unroll
        for (int i = 0; i < XM; i++) {
            const int j = min(wave + i * nwaves, nimg * MT - 1), u = j & (MT - 1);
            const size_t row = MT == 1 ? 0 : (size_t)min(u, P.m - 1) * P.ldx;
            const int e = (sb0 + j / MT) * 256 + 4 * lane;
            if constexpr (H)
                xv[i] = load8_async((const _Float16*)P.x + row + (P.xfmt == ACT_F16_XPERM ? xperm_pos(e) : e));
            else
                xv[i] = load16_async_u((const float*)P.x + row + e);
        }
        static_for<PRE>([&](auto ic) __attribute__((always_inline)) { issue_static(decltype(ic)::value); });
        if (threadIdx.x == 0) lds_write(next, min(SC * nwaves, nu));
        // table entry of position p, written while the loads above are in flight and published by the
        // barrier: global address of the unit's weight group (matrix 0), then ru | (sb - sb0) << 16
        // (both below 2^16, see plan)
        for (int p = threadIdx.x; p < nu; p += 64 * nwaves) {
            const int ru = rel_of(p), u = u0 + ru, q = u / CS, s = q / ntiles, tile = q - s * ntiles;
            const int sb = s * CS + (u - q * CS);
            const uint64_t G = (uint64_t)unit_group(P, 0, tile, sb, C::GB);
            lds_st128(tab + p, u4{(uint32_t)G, (uint32_t)(G >> 32), (uint32_t)(ru | ((sb - sb0) << 16)), 0u});
        }
        // load i is followed by XM - 1 - i loads and the PRE * NDMA DMA instructions of the first units
        // (issued unconditionally; the masked ones still issue, lanes 0..15 being live)
        static_for<XM>([&](auto ic) __attribute__((always_inline)) {
            constexpr int i = decltype(ic)::value;
            wait_x<XM - 1 - i + PRE * NDMA>(xv[i]);
            const int j = wave + i * nwaves, u = j & (MT - 1);
            if (j < nimg * MT) {
                f4 v;
                if constexpr (H)
                    v = f4{h2f_bits(xv[i].x & 0xFFFFu), h2f_bits(xv[i].x >> 16), h2f_bits(xv[i].y & 0xFFFFu),
                           h2f_bits(xv[i].y >> 16)};
                else
                    v = __builtin_bit_cast(f4, xv[i]);
                const f4 xz = {0.0f, 0.0f, 0.0f, 0.0f};
                prep8_store<TYPE, MT>(MT == 1 || u < P.m ? v : xz, lane, img + (j / MT) * C::IMG, u);
            }
        });
        static_for<ST - PRE>([&](auto ic) __attribute__((always_inline)) { issue_static(PRE + decltype(ic)::value); });
    };
    if (P.xfmt == ACT_F32) prologue(std::false_type{});
    else prologue(std::true_type{});
    lds_barrier();  // publishes the image and the table; waits only for LDS operations

    // Weight addresses of this wave's static units, 64 at a time (ta: lane l holds unit 64 * batch
    // + l's), taken by v_readlane, so that no static unit waits on an LDS read before its DMA.  (The
    // gate/up pair at four tokens has no two registers to spare: it reads each address where used.)
    constexpr bool REGTAB = !(NA == 2 && MT >= 4) && MT < 8;
    auto tab_at = [&](int i0) __attribute__((always_inline)) {
        return (const uint2*)(tab + min(wave + (i0 + (REGTAB ? lane : 0)) * nwaves, nu - 1));
    };
    uint2 ta = {0u, 0u};
    if constexpr (REGTAB) ta = *tab_at(0);
    int issued = min(ST, nst), done = 0, cslot = 0, islot = issued == D ? 0 : issued * SLOT;
    bool more = true;
    // positions of the units in this wave's ring, 21 bits each, oldest in the low bits
    uint64_t ring_units = 0;
    for (int i = 0; i < issued; i++) ring_units |= (uint64_t)(wave + i * nwaves) << (21 * i);
    // the next unit's DMA: static unit `issued` while there is one, then a position from the counter
    auto issue = [&]() __attribute__((always_inline)) {
        int p;
        uint64_t G;
        if (issued < nst) {
            const int j = issued;
            p = wave + j * nwaves;
            if constexpr (REGTAB) {
                if ((j & 63) == 0) ta = *tab_at(j);
                G = ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)ta.y, j & 63) << 32) |
                    (uint32_t)__builtin_amdgcn_readlane((int)ta.x, j & 63);
            } else {
                const uint2 e = *tab_at(j);
                G = ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)e.y) << 32) |
                    (uint32_t)__builtin_amdgcn_readfirstlane((int)e.x);
            }
        } else {
            if (SC * nwaves >= nu) {  // every position was static
                more = false;
                return;
            }
            uint2 e = {0u, 0u};
            p = 0;
            if (lane == 0) {
                p = lds_add(next, 1);
                e = *(const uint2*)(tab + min(p, nu - 1));
            }
            p = __builtin_amdgcn_readfirstlane(p);
            if (p >= nu) {
                more = false;
                return;
            }
            G = ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)e.y) << 32) |
                (uint32_t)__builtin_amdgcn_readfirstlane((int)e.x);
        }
#pragma unroll
        for (int a = 0; a < NA; a++) dma_group<C::GB>((const uint8_t*)G + a * wdelta, ring + islot + a * C::GB, lane);
        ring_units |= (uint64_t)p << (21 * (issued - done));
        issued++;
        islot = islot + SLOT == D * SLOT ? 0 : islot + SLOT;
    };
    int aoff[NP];
#pragma unroll
    for (int p = 0; p < NP; p++) aoff[p] = a8_offset<MT>(lane, p);
    while (done < issued) {
        if (more && issued - done < D) issue();
        const int pos = (int)(ring_units & 0x1FFFFF);
        ring_units >>= 21;
        // ru | (super-block - sb0) << 16, read while the unit's DMA may still be in flight
        const uint32_t ent = (uint32_t)__builtin_amdgcn_readfirstlane((int)((const uint32_t*)(tab + pos))[2]);
        // units issued after this one and still allowed in flight (stand-ins of the prologue
        // follow the real units, so counting only real ones waits longer, never shorter)
        wait_vm_units<NDMA>(issued - done - 1);
        const uint8_t* slot = ring + cslot;
        cslot = cslot + SLOT == D * SLOT ? 0 : cslot + SLOT;
        const uint8_t* simg = img + (ent >> 16) * C::IMG;
        const int ru = (int)(ent & 0xFFFFu);

        float v[NA][MT];
        if constexpr (TYPE == T_Q4_K || TYPE == T_Q5_K) q45_unit8<TYPE, NA, MT>(slot, simg, aoff, lane, r, g, v);
        else if constexpr (TYPE == T_Q8_0) q8_unit8<NA, MT>(slot, simg, aoff, lane, r, g, v);
        else q6_unit8<NA, MT>(slot, simg, aoff, lane, r, g, v);
        float cols[NA * MT];  // column a * MT + u
#pragma unroll
        for (int a = 0; a < NA; a++)
#pragma unroll
            for (int u = 0; u < MT; u++) cols[a * MT + u] = v[a][u];
        lds_order();
        done++;
        store_sums<NA * MT>(cols, part + ru * NA * MT * 16, lane);
    }

    // Every unit's sums are in the LDS after this barrier.  Wave w completes groups w, w + waves, ...
    // of the range: it adds the group's unit sums in unit order.  Column c = a * MT + u of the sums;
    // lane (row, c % CW) sums the units of its lane group (NGRP groups, units grp, grp + NGRP, ...),
    // then the groups add in a fixed order; with more than four columns a lane does NC / 4 of them.
    lds_barrier();
    // the lane index again (mbcnt), so that nothing derived from it stays live across the loop
    const int lane_e = (int)__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
    for (int gi = wave; gi <= ql - qf; gi += nwaves) {
        const int q = qf + gi, s = q / ntiles, tile = q - s * ntiles;
        const int ta0 = max(u0, q * CS) - u0, tb = min(u1, (q + 1) * CS) - u0;
        constexpr int NC = NA * MT, CW = NC < 4 ? NC : 4, NCL = NC > 4 ? NC / 4 : 1, NGRP = 4 / CW;
        const int row = lane_e & 15, cl = (lane_e >> 4) % CW, grp = (lane_e >> 4) / CW;
        float sums[NCL];
#pragma unroll
        for (int i = 0; i < NCL; i++) {
            float sum = 0.0f;
            for (int j = ta0 + grp; j < tb; j += NGRP) sum += part[(j * NC + cl + 4 * i) * 16 + row];
            if constexpr (NGRP >= 2) sum += __shfl_xor(sum, 32);
            if constexpr (NGRP == 4) sum += __shfl_xor(sum, 16);
            sums[i] = sum;
        }
        const bool whole = q * CS >= u0 && (q + 1) * CS <= u1;
        // tokens in passes of four (eight token slots: two passes); lane (row, u) takes its token's
        // columns a * MT + u: with eight slots lane group G holds columns G + 4i, i.e. tokens G and
        // G + 4 of each stream; with up to four its own sums for a = 0 (and for a = 1 with eight
        // columns), the up column of lane (MT + u, row) otherwise
        constexpr int NH = MT == 8 ? 2 : 1;
#pragma unroll
        for (int h = 0; h < NH; h++) {
            const int u = MT == 1 ? 0 : (lane_e >> 4) + 4 * h;
            float vals[NA];
            if constexpr (MT == 8) {
                vals[0] = sums[h];
                if constexpr (NA == 2) vals[1] = sums[2 + h];
            } else {
                vals[0] = sums[0];
                if constexpr (NA == 2) vals[1] = NC > 4 ? sums[NCL - 1] : __shfl(sums[0], (MT + u) * 16 + row);
            }
            if (MT == 1 ? lane_e < 16 : (lane_e < 16 * MT || MT == 8) && u < P.m) {
                // a group shared with a neighbouring range first pairs with its other piece (node s of
                // level 0); then slice sums pair up a binary tree over the slices (node s >> l of level
                // l); whoever completes the root stores the row.  Slots: [tile][node][token][row].
                uint64_t* xs = P.xslot + ((size_t)tile * P.xnodes * MT + u) * 16 + row;
                bool carry = whole || xcombine<NA>(xs + (size_t)s * MT * 16, vals);
                int lo = S;  // first node of level l
                for (int l = 1; (1 << (l - 1)) < S; l++) {
                    const int sib = ((s >> (l - 1)) ^ 1) << (l - 1);  // first slice of the sibling subtree
                    if (carry && sib < S) carry = xcombine<NA>(xs + (size_t)(lo + (s >> l)) * MT * 16, vals);
                    lo += (S + (1 << l) - 1) >> l;
                }
                if (carry) store_row<NA>(P, tile, u, row, vals);
            }
        }
    }
}

// ------------------------------------------------------------------------------------------------
// Launch plumbing: one instantiation per (type, streams, token bucket); ring depth 3 for a single
// stream, 2 for the GLU pair (two groups per slot).
template <int NA>
constexpr int ring_of() { return NA == 1 ? 3 : 2; }

// Waves per work-group: as many as the LDS of one CU holds (at most 16), so that a CU runs one
// work-group whose waves were all dispatched together.  Waves of one age share the memory pipeline
// fairly; several work-groups per CU would be served oldest-first and finish one after another.
constexpr int lds_round(int b) { return (b + LDS_GRANULE - 1) / LDS_GRANULE * LDS_GRANULE; }
constexpr int waves_per_wg(int wave_lds, int cap) {
    int w = cap;
    while (w > 1 && lds_round(w * wave_lds) > LDS_PER_CU) w--;
    return w;
}

template <int TYPE, int NA, int MT>
struct Kern {
    static constexpr int D = ring_of<NA>();
    static constexpr int WAVE_LDS = TYPE == T_Q4_K ? Q4Cfg<NA, MT, D>::WAVE_LDS : Q6Cfg<NA, MT, D>::WAVE_LDS;
    // the Q6_K GLU kernels with 2 or 4 tokens need more than 128 VGPRs: at most 2 waves per SIMD
    static constexpr int WPG = waves_per_wg(WAVE_LDS, TYPE == T_Q6_K && NA == 2 && MT >= 2 ? 8 : 16);
    static constexpr size_t LDS = (size_t)WPG * WAVE_LDS;
    static const void* fn() {
        if constexpr (TYPE == T_Q4_K) return (const void*)&k_gemv_q4k<NA, MT, D, WPG>;
        else return (const void*)&k_gemv_q6k<NA, MT, D, WPG>;
    }
    static constexpr int IMG = TYPE == T_Q4_K ? q4_img<MT>() : q6_img<MT>();
    static int launch(const GemvParams& p, hipStream_t s) {
        if constexpr (TYPE == T_Q4_K)
            hipLaunchKernelGGL((k_prep_q4<MT>), dim3(p.nsb, p.m), dim3(64), 0, s, p.x, p.xfmt, p.ldx, (uint8_t*)p.ximg);
        else
            hipLaunchKernelGGL((k_prep_q6<MT>), dim3(p.nsb, p.m), dim3(64), 0, s, p.x, p.xfmt, p.ldx, (uint8_t*)p.ximg);
        if (hipGetLastError() != hipSuccess) return -1;
        const int grid = (p.waves + WPG - 1) / WPG;
        if constexpr (TYPE == T_Q4_K)
            hipLaunchKernelGGL((k_gemv_q4k<NA, MT, D, WPG>), dim3(grid), dim3(64 * WPG), LDS, s, p);
        else
            hipLaunchKernelGGL((k_gemv_q6k<NA, MT, D, WPG>), dim3(grid), dim3(64 * WPG), LDS, s, p);
        return hipGetLastError() == hipSuccess ? 0 : -1;
    }
    static int resident_wgs() {  // work-groups of this kernel resident per CU, per device
        static std::atomic<int> cache[MAX_DEVICES];
        const int dev = current_device() % MAX_DEVICES;
        if (int c = cache[dev].load(std::memory_order_relaxed)) return c;
        int n = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, fn(), 64 * WPG, LDS) != hipSuccess || n < 1) n = 1;
        // LDS is granted in blocks; the occupancy query does not round, so bound it here (a grid
        // larger than what is resident would leave waves waiting for a whole wave lifetime)
        const int by_lds = (int)(LDS_PER_CU / ((LDS + LDS_GRANULE - 1) / LDS_GRANULE * LDS_GRANULE));
        if (n > by_lds) n = by_lds;
        n = n < 1 ? 1 : n;
        cache[dev].store(n, std::memory_order_relaxed);
        return n;
    }
};

template <int TYPE, int NA, typename F>
int dispatch_mt(int m, F&& f) {
    if (m <= 1) return f(Kern<TYPE, NA, 1>{});
    if (m <= 2) return f(Kern<TYPE, NA, 2>{});
    return f(Kern<TYPE, NA, 4>{});
}

template <typename F>
int dispatch(int type, int na, int m, F&& f) {
    if (type == T_Q4_K) return na == 1 ? dispatch_mt<T_Q4_K, 1>(m, f) : dispatch_mt<T_Q4_K, 2>(m, f);
    if (type == T_Q6_K) return na == 1 ? dispatch_mt<T_Q6_K, 1>(m, f) : dispatch_mt<T_Q6_K, 2>(m, f);
    return -1;
}

// Tuning overrides (qk_set_tuning), process-wide; atomics so that a setter racing a launch is not a
// data race (which value a concurrent launch sees is unspecified).
std::atomic<int> g_tune_waves{0};
std::atomic<bool> g_fused{true};  // m <= 4 through the int8 kernel where its plan applies
std::atomic<int> g_wpg{0};        // at most this many waves per int8 work-group (0 = as many as fit)
std::atomic<int> g_img_kib{32};   // largest activation image per range before the K-slices double
std::atomic<int> g_dshift{1};     // int8 kernel: about nu >> g_dshift of a range's units handed out dynamically
std::atomic<int> g_min_waves{0};  // int8 kernel at m >= 2: the fewest waves per work-group it is planned with
std::atomic<int> g_max_slots{8};  // int8 kernel: the most token slots per launch (4 or 8)

// Single-token plan: one work-group per CU (more when a group's unit sums would not fit its LDS),
// as many waves as the LDS left after the activation image and the unit sums can feed (<= 16).
// Combine slots per tile row and token for S slices: S at level 0 (a group's two pieces), then
// ceil(S / 2^l) at level l of the binary tree over the slices, levels stored one after another.
inline int xnodes_of(int S) {
    int n = S;
    for (int l = 1; (1 << (l - 1)) < S; l++) n += (S + (1 << l) - 1) >> l;
    return n;
}

template <int TYPE, int NA, int MT>
struct Fused {
    // ring depth: 3 units per wave; 2 for the gate/up pair at four tokens, whose unit sums take a
    // third of the LDS (a 2-deep ring leaves room for 10 waves instead of 6), and for eight tokens
    static constexpr int D = (NA == 2 && MT == 4) || MT == 8 ? 2 : 3;
    static size_t align16(size_t v) { return (v + 15) & ~(size_t)15; }
    // Plan for `groups` work-groups and S slices: LDS bytes, or 0 when it does not apply.
    static size_t layout(GemvParams& p, int groups, int S, int waves) {
        using C = G1<TYPE, MT>;
        const int cs = p.nsb / S, ntiles = p.units / p.nsb;
        // table fields: unit indices below 2^16 (the super-block offsets are smaller still, see jobs)
        const int maxnu = (p.units + groups - 1) / groups;
        if (p.units / groups < cs || maxnu >= (1 << 16)) return 0;
        // the most super-blocks any range covers
        int span = 0;
        const int rq = p.units / groups, rrem = p.units % groups;
        for (int b = 0; b < groups; b++) {
            const int u0 = b * rq + std::min(b, rrem), u1 = u0 + rq + (b < rrem ? 1 : 0);
            const int qf = u0 / cs, ql = (u1 - 1) / cs;
            span = std::max(span, (ql / ntiles - qf / ntiles + 1) * cs);
        }
        const int jobs = span * MT;  // x conversions: (token, super-block)
        if (jobs > 12 * waves) return 0;  // at most 12 conversions per wave
        p.xm = jobs <= 2 * waves ? 2 : jobs <= 4 * waves ? 4 : jobs <= 6 * waves ? 6 : 12;
        p.slices = S;
        p.dshift = g_dshift.load();
        p.xnodes = xnodes_of(S);
        p.rq = rq;
        p.rrem = rrem;
        p.cs = cs;
        p.ntiles = ntiles;
        p.waves = groups;
        p.lds_part = (int)align16((size_t)span * C::IMG);
        p.lds_cnt = (int)align16(p.lds_part + (size_t)maxnu * NA * MT * 64);
        p.lds_tab = p.lds_cnt + 16;
        p.lds_ring = (int)align16(p.lds_tab + 16 * (size_t)maxnu);
        return p.lds_ring + (size_t)waves * D * NA * C::GB;
    }
    // Slices: the fewest whose range image fits 32 KB (else the smallest image), then as many waves
    // (<= 16) as the LDS left feeds.
    static bool plan(GemvParams& p, int cus, bool small, int& wpg, size_t& lds) {
        // one work-group per CU; more (smaller ranges, run in rounds) when one range's tables do not
        // fit the LDS, or leave it room for fewer than WANT waves: a range's unit sums and table grow
        // with its units (a 248320-row matrix left four waves per CU at one work-group per CU, and
        // nine at two, in two rounds)
        constexpr int WANT = 8;
        GemvParams best = p;
        int best_w = 0;
        size_t best_lds = 0;
        for (int groups = std::min(p.units, cus), tries = 0;; groups = std::min(p.units, 2 * groups), tries++) {
            GemvParams t = p;
            int w = 0;
            size_t l = 0;
            if (plan_groups(t, groups, MT == 8 ? 32 : 16, w, l) && w > best_w) {
                best = t;
                best_w = w;
                best_lds = l;
            }
            // eight token slots: one round only (the gate/up pair at K=5120 N=17408 planned four
            // rounds of 9 waves, 66 us at eight tokens against 50 for four tokens and then four)
            if (best_w >= WANT || groups == p.units || (best_w > 0 && tries >= 2) || MT == 8) break;
        }
        // eight token slots with fewer than WANT waves: four tokens and then the rest is faster
        if (MT == 8 && best_w > 0 && best_w < WANT) return false;
        if (best_w > 0) {
            p = best;
            wpg = best_w;
            lds = best_lds;
            return true;
        }
        if (!small) return false;
        // small matrices (fewer units than CUs times a slice): fewer work-groups, each range holding
        // at least one group of cs units.  Per S, estimated time = a unit's share of one CU's stream
        // (~25 ns) times the units of a range, plus one exchange round trip (~1 us) per level of
        // the slice tree; the cheapest S wins.
        // the cheapest S whose plan fits (a range converting many super-blocks of several tokens
        // needs many waves, whose rings may not fit the LDS)
        struct Cand {
            double t;
            int g, S;
        };
        Cand cands[128];  // divisors of nsb (at most 128 for any k the ABI accepts here)
        int nc = 0;
        for (int S = 1; S <= p.nsb && nc < 128; S++) {
            if (p.nsb % S) continue;
            const int g = std::min(cus, p.units / (p.nsb / S));
            int levels = 0;
            while ((1 << levels) < S) levels++;
            cands[nc++] = {0.025 * ((p.units + g - 1) / g) + 1.0 * levels, g, S};
        }
        std::stable_sort(cands, cands + nc, [](const Cand& a, const Cand& b) { return a.t < b.t; });
        for (int ci = 0; ci < nc; ci++) {
            const Cand& c = cands[ci];
            GemvParams t = p;
            if (plan_groups(t, c.g, c.S, wpg, lds, c.S)) {
                p = t;
                return true;
            }
        }
        return false;
    }
    // Plan for `groups` work-groups: the fewest slices (from smin, at most smax) whose range image
    // fits 32 KB, else the smallest image.
    static bool plan_groups(GemvParams& p, int groups, int smax, int& wpg, size_t& lds, int smin = 1) {
        const int ntiles = p.units / p.nsb;
        int best = 0;
        size_t best_img = 0;
        for (int S = smin; S <= smax && S <= p.nsb; S++) {
            GemvParams t = p;
            if (p.nsb % S || (size_t)ntiles * xnodes_of(S) * MT * 16 > p.xslot_cap ||
                !layout(t, groups, S, gemv1_max_waves<MT>()))
                continue;
            const size_t img = (size_t)t.lds_part;
            if (!best || img < best_img) {
                best = S;
                best_img = img;
            }
            // eight token slots: an image twice the size (the slices' exchange levels cost more than
            // the waves the larger image takes)
            if (img <= (size_t)g_img_kib.load() * 1024 * (MT == 8 ? 2 : 1)) break;
        }
        if (!best) return false;
        for (int waves = std::min(g_wpg.load() > 0 ? g_wpg.load() : 16, gemv1_max_waves<MT>()); waves >= 4; waves--) {
            GemvParams t = p;
            const size_t total = layout(t, groups, best, waves);
            if (total && total <= (size_t)LDS_PER_CU) {
                p = t;
                wpg = waves;
                lds = total;
                return true;
            }
        }
        return false;
    }
    template <int ST>
    static void launch_xm(const GemvParams& p, dim3 grid, dim3 block, size_t lds, hipStream_t s) {
        switch (p.xm) {
            case 2: hipLaunchKernelGGL((k_gemv1<TYPE, NA, D, 2, ST, MT>), grid, block, lds, s, p); break;
            case 4: hipLaunchKernelGGL((k_gemv1<TYPE, NA, D, 4, ST, MT>), grid, block, lds, s, p); break;
            case 6: hipLaunchKernelGGL((k_gemv1<TYPE, NA, D, 6, ST, MT>), grid, block, lds, s, p); break;
            default: hipLaunchKernelGGL((k_gemv1<TYPE, NA, D, 12, ST, MT>), grid, block, lds, s, p); break;
        }
    }
    static int launch(GemvParams p, hipStream_t s, int cus, bool small, int min_waves, GemvPlan* info) {
        int wpg = 0;
        size_t lds = 0;
        // not applicable: the caller uses the general kernel
        if (!plan(p, cus, small, wpg, lds) || wpg < min_waves) return 1;
        if (info) {
            info->kernel = GEMV_KERNEL_INT8;
            info->work_groups = p.waves;
            info->waves_per_group = wpg;
            info->ring_depth = D;
            info->slices = p.slices;
            info->token_slots = MT;
            info->lds_bytes = (int)lds;
            return 0;  // plan only
        }
        p.wpg = wpg;
        const dim3 grid(p.waves), block(64 * wpg);
        // three static units per wave when the waves have at least three units each
        if (D >= 3 && p.rq >= 3 * wpg) launch_xm<D >= 3 ? 3 : 2>(p, grid, block, lds, s);
        else launch_xm<2>(p, grid, block, lds, s);
        return hipGetLastError() == hipSuccess ? 0 : -1;
    }
};

}  // namespace

void gemv_set_waves(int waves) { g_tune_waves = waves; }
void gemv_set_fused(bool on) { g_fused = on; }
void gemv_set_wpg(int w) { g_wpg = w; }
void gemv_set_img_kib(int kib) { g_img_kib = kib > 0 ? kib : 32; }
void gemv_set_dshift(int sh) { g_dshift = sh; }
void gemv_set_min_waves(int w) { g_min_waves = w; }
void gemv_set_max_slots(int t) { g_max_slots = t; }

// Q5_K / Q8_0 run only the single-token kernel, which plans its own grid: the general kernel's
// figures of Q4_K stand in for them here.
inline int general_type(int type) { return type == T_Q5_K || type == T_Q8_0 ? T_Q4_K : type; }

int gemv_plan_waves(int type, int na, int m, int units) {
    type = general_type(type);
    const int cus = current_cus();
    int waves = g_tune_waves;
    if (waves <= 0)
        waves = dispatch(type, na, m, [](auto k) { return decltype(k)::resident_wgs() * decltype(k)::WPG; }) * cus;
    return waves < units ? waves : units;
}

size_t gemv_image_bytes(int type, int m, int nsb) {
    type = general_type(type);
    return (size_t)nsb * dispatch(type, 1, m, [](auto k) { return decltype(k)::IMG; });
}

size_t gemv_part_floats(int waves, int na, int m) {
    const int mt = m <= 1 ? 1 : m <= 2 ? 2 : 4;
    return (size_t)waves * 2 * na * mt * 16;
}

// The int8 kernel for p.m <= 8 tokens (1, 2, 4 or 8 token slots).  small: also plan matrices too small
// for one work-group per CU.  min_waves: the fewest waves per work-group to accept (0 by default; the
// gemv_min_waves knob hands plans with fewer waves to the general kernel, for comparisons).
// info != nullptr: plan only, nothing is launched.
// Returns 0, 1 when no plan applies, -1 on a launch error.
template <int TYPE>
int launch_fused(const GemvParams& p, hipStream_t s, bool small, int min_waves, GemvPlan* info) {
    auto go = [&](auto mt) {
        constexpr int MT = decltype(mt)::value;
        const int cus = current_cus();
        return p.glu ? Fused<TYPE, 2, MT>::launch(p, s, cus, small, min_waves, info)
                     : Fused<TYPE, 1, MT>::launch(p, s, cus, small, min_waves, info);
    };
    if (p.m <= 1) return go(std::integral_constant<int, 1>{});
    if (p.m <= 2) return go(std::integral_constant<int, 2>{});
    if (p.m <= 4) return go(std::integral_constant<int, 4>{});
    if (g_max_slots.load() < 8) return 1;  // the caller runs four tokens, then the rest
    return go(std::integral_constant<int, 8>{});
}

int launch_gemv(int type, const GemvParams& p, hipStream_t s, GemvPlan* info) {
    if (type == T_Q5_K || type == T_Q8_0)  // the int8 kernel only: 1 = no plan for this shape
        return type == T_Q5_K ? launch_fused<T_Q5_K>(p, s, true, 0, info) : launch_fused<T_Q8_0>(p, s, true, 0, info);
    if (g_fused && !g_tune_waves) {
        // The int8 kernel takes every shape it can plan, small matrices included (at two to four
        // tokens it was measured faster than the general kernel even where its plan leaves six to
        // eight waves per work-group: K=17408 N=5120 Q6_K at four tokens 22.5 against 32.7 us, the
        // output projection at two 177 against 225 us).  It also carries any finite x, where the
        // general kernel's fp16 pair needs |x| < 65504 and Q4_K sub-block sums below that too.
        const int mw = p.m > 1 ? g_min_waves.load() : 0;
        int rc = 1;
        if (type == T_Q4_K) rc = launch_fused<T_Q4_K>(p, s, mw == 0, mw, info);
        if (type == T_Q6_K) rc = launch_fused<T_Q6_K>(p, s, mw == 0, mw, info);
        if (rc <= 0) return rc;
    }
    if (p.m > 4) return 1;  // the general kernel carries at most four tokens: the caller splits
    if (info) {
        info->kernel = GEMV_KERNEL_GENERAL;
        info->work_groups = dispatch(type, p.glu ? 2 : 1, p.m, [&](auto k) {
            return (p.waves + decltype(k)::WPG - 1) / decltype(k)::WPG;
        });
        info->waves_per_group = dispatch(type, p.glu ? 2 : 1, p.m, [](auto k) { return decltype(k)::WPG; });
        info->ring_depth = dispatch(type, p.glu ? 2 : 1, p.m, [](auto k) { return decltype(k)::D; });
        info->slices = 1;
        info->token_slots = p.m <= 1 ? 1 : p.m <= 2 ? 2 : 4;
        info->lds_bytes = dispatch(type, p.glu ? 2 : 1, p.m, [](auto k) { return (int)decltype(k)::LDS; });
        return 0;
    }
    return dispatch(type, p.glu ? 2 : 1, p.m, [&](auto k) { return decltype(k)::launch(p, s); });
}

}  // namespace qk
