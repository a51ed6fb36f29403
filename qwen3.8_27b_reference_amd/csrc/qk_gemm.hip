// Prefill GEMM (m >= 16) for Q4_K / Q6_K weights: super-blocks dequantized to fp16 feeding CDNA4
// MFMA (v_mfma_f32_32x32x16_f16), fp32 accumulate.
//
// Replaces the reference's k_gemm_q4k / k_gemm_q6k (qwen_cuda/kernels.cu:307-361, 394, 397-401:
// 64x64x64 tiles, 2x2 warps of mma.m16n8k16, dequant via dq8h into shared memory) with a design
// for 256-CU CDNA4:
//
//  * The 32x32x16 MFMA: on MI355X it runs at about twice the rate of 16x16x32 (measured
//    ~2.07 vs ~1.19 PFLOP/s fp16).  Its 32 A rows are a pair of T16 tiles.
//  * A work-group owns P tile pairs x 128 tokens; P is chosen per shape so that the work-groups
//    fill whole rounds of CUs (N=17408, M=512: 544 pairs = 60 x 9 + 4, 61 x 4 token blocks =
//    244 work-groups on 256 CUs).  Each of the 4 waves owns P/4 pairs for all 128 tokens and
//    takes one 32-token block of each of the P%4 remaining pairs, so all waves issue the same
//    number of MFMAs.
//  * K advances 64 elements (a quarter super-block) per step.  The raw T16 bytes of the step and
//    the fp16 activation tile arrive in LDS by LDS-DMA two steps ahead (three stages).  Each wave
//    dequantizes its own A fragments in registers (the reference's tolerance path,
//    kernels.cu:127-181: scales rounded to fp16, one packed FMA per pair of weights), so the
//    dequantized weights never travel through LDS.
//  * x is rounded to fp16 once per call into MFMA B-operand order by k_gemm_prep_x.
//  * y is fp32 [m][n] row-major like the reference's GEMM output (y[tok*n + row]).
#include "qk_device.h"
#include "qk_internal.h"

namespace qk {
namespace {

#define LDS_AS __attribute__((address_space(3)))

typedef float f16v __attribute__((ext_vector_type(16)));

constexpr int BM = GEMM_BM;   // tokens per work-group (four 32-token blocks)
constexpr int THREADS = 256;  // 4 waves
constexpr int STAGES = 3;

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

__device__ inline void dma16(const void* g, uint8_t* lds) {
    __builtin_amdgcn_global_load_lds(g, (LDS_AS void*)lds, 16, 0, 0);
}

// D(32x32 f32) += A(32x16 f16) * B(16x32 f16).  Lane l holds A[l & 31][8*(l >> 5) .. +7],
// B[8*(l >> 5) .. +7][l & 31] and D[8*(v/4) + 4*(l >> 5) + v%4][l & 31] in register v (checked
// on the device against a host product).
__device__ inline f16v mfma32(const h8& a, const h8& b, const f16v& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// ------------------------------------------------------------------------------------------------
// Activation image: x fp32 [m][k] -> fp16 records; record (tb, kc, l) at ((tb * K/16 + kc) * 64 + l)
// * 16 holds x[32*tb + (l & 31)][16*kc + 8*(l >> 5) + 0..7] rounded to nearest even (zeros for
// tokens >= m): one 64-lane 16-byte read per (32-token block, K/16 chunk) is a B operand.
__global__ __launch_bounds__(64) void k_gemm_prep_x(const float* __restrict__ x, int m, int k,
                                                     uint8_t* __restrict__ img) {
    const int kc = blockIdx.x, tb = blockIdx.y, l = threadIdx.x;
    const int tok = 32 * tb + (l & 31), k0 = 16 * kc + 8 * (l >> 5);
    f4 a = {0.0f, 0.0f, 0.0f, 0.0f}, b = a;
    if (tok < m) {
        a = *(const f4*)(x + (size_t)tok * k + k0);
        b = *(const f4*)(x + (size_t)tok * k + k0 + 4);
    }
    const h2 p0 = {(_Float16)a.x, (_Float16)a.y}, p1 = {(_Float16)a.z, (_Float16)a.w};
    const h2 p2 = {(_Float16)b.x, (_Float16)b.y}, p3 = {(_Float16)b.z, (_Float16)b.w};
    *(u4*)(img + (((size_t)tb * (k / 16) + kc) * 64 + l) * 16) = u4{as_u32(p0), as_u32(p1), as_u32(p2), as_u32(p3)};
}

__device__ inline uint32_t pk_sub1024(uint32_t v) {  // (1024 + q) - 1024, exact
    return as_u32(as_h2(v) + h2{(_Float16)-1024.0f, (_Float16)-1024.0f});
}

// ------------------------------------------------------------------------------------------------
// Raw bytes of one step (quarter q of super-block sb) of one tile, staged in LDS by LDS-DMA as
// 256-byte pieces.
//   Q4_K: piece 0/1 = the two 256-byte qs runs of the quarter (T16 bytes 1024i + 256q ..),
//         piece 2 = d/dmin (offset 0) and scales (offset 64) (T16 bytes 2048..2303).
//   Q6_K: pieces 0..3 = ql half-plane n = q/2 (T16 1024n ..), 4..5 = qh plane n (2048 + 512n ..),
//         piece 6 = scales of half n (offset 0, T16 3072 + 128n) and d (offset 128, T16 3328).
constexpr int Q4_PIECES = 3, Q6_PIECES = 7;

__device__ inline const uint8_t* q4_piece_src(const uint8_t* G, int q, int j, int li) {
    return (j < 2 ? G + 1024 * j + 256 * q : G + 2048) + 16 * li;
}

__device__ inline const uint8_t* q6_piece_src(const uint8_t* G, int q, int j, int li) {
    const int n = q >> 1;
    if (j < 4) return G + 1024 * n + 256 * j + 16 * li;
    if (j < 6) return G + 2048 + 512 * n + 256 * (j - 4) + 16 * li;
    return li < 8 ? G + 3072 + 128 * n + 16 * li : G + 3328 + 16 * (li & 1);  // lanes 10..15 repeat d
}

// Per super-block, per lane (row r): the eight sub-blocks' (half(d*sc_j), half(-dmin*m_j)) pairs.
// fp16 products of exact fp16 factors round once, as the reference's half(d * sc) does
// (kernels.cu:127-181).  6-bit unpack as in qwen_cpu/quants.h:33-41, bytewise on whole dwords.
struct Q4Scales {
    uint32_t dm[8];
};

__device__ inline Q4Scales q4_scales(const uint8_t* R, int r) {
    const uint32_t dd = ld4(R + 512 + 4 * r);
    const uint32_t s0 = ld4(R + 576 + 12 * r), s1 = ld4(R + 580 + 12 * r), s2 = ld4(R + 584 + 12 * r);
    const uint32_t Slo = s0 & 0x3F3F3F3Fu, Mlo = s1 & 0x3F3F3F3Fu;
    const uint32_t Shi = (s2 & 0x0F0F0F0Fu) | ((s0 >> 2) & 0x30303030u);
    const uint32_t Mhi = ((s2 >> 4) & 0x0F0F0F0Fu) | ((s1 >> 2) & 0x30303030u);
    const h2 dmn = {__builtin_bit_cast(_Float16, (uint16_t)(dd & 0xFFFFu)),
                    (_Float16)-__builtin_bit_cast(_Float16, (uint16_t)(dd >> 16))};
    Q4Scales o;
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const uint32_t S = j < 4 ? Slo : Shi, M = j < 4 ? Mlo : Mhi;
        const int b = 8 * (j & 3);
        // bytes (sc_j, m_j) under the fp16 exponent of 1024: (1024 + sc, 1024 + m), exact
        const uint32_t packed = ((S >> b) & 0xFFu) | (((M >> b) & 0xFFu) << 16) | 0x64006400u;
        o.dm[j] = as_u32((as_h2(packed) + h2{(_Float16)-1024.0f, (_Float16)-1024.0f}) * dmn);
    }
    return o;
}

// A fragments of one tile pair for quarter q: lane l = 32h + 16u + r (row 16u + r of the pair,
// K half h) gets W[row][16c + 8h + 0..7] for the four K/16 chunks c of the quarter.
//   Q4_K: chunks 0,1 = low nibbles of qs_r[32q + 16c + 8h ..] (sub-block 2q), chunks 2,3 = high
//   nibbles of the same bytes (sub-block 2q+1) (qwen_cpu/quants.h:53-71 element order).
__device__ inline void q4_frags(const uint8_t* R, const Q4Scales& S, int q, int r, int h, h8 (&a)[4]) {
    const u2 lo = ld8(R + 16 * r + 8 * h);        // qs_r[32q + 8h + 0..7]
    const u2 hi = ld8(R + 256 + 16 * r + 8 * h);  // qs_r[32q + 16 + 8h + 0..7]
#pragma unroll
    for (int c = 0; c < 4; c++) {
        const h2 v = as_h2(S.dm[2 * q + (c >> 1)]);
        const h2 vds = {v.x, v.x}, vdm = {v.y, v.y};
        const u2 src = (c & 1) ? hi : lo;
        const uint32_t n0 = (c >> 1) ? (src.x >> 4) & 0x0F0F0F0Fu : src.x & 0x0F0F0F0Fu;
        const uint32_t n1 = (c >> 1) ? (src.y >> 4) & 0x0F0F0F0Fu : src.y & 0x0F0F0F0Fu;
        a[c] = make_h8(pk_fma(pk_sub1024(perm_lo(n0)), vds, vdm), pk_fma(pk_sub1024(perm_hi(n0)), vds, vdm),
                       pk_fma(pk_sub1024(perm_lo(n1)), vds, vdm), pk_fma(pk_sub1024(perm_hi(n1)), vds, vdm));
    }
}

//   Q6_K: chunk c holds elements 128n + 32s + l' with s = 2(q&1) + c/2, l' = 16(c&1) + 8h + 0..7:
//   ql_r[64n + 16c + 8h ..] (nibble s >= 2), qh_r[32n + 16(c&1) + 8h ..] (crumb s), scale
//   8n + 4(q&1) + c (qwen_cpu/quants.h:96-121).
__device__ inline void q6_frags(const uint8_t* R, int q, int r, int h, h8 (&a)[4]) {
    const int hn = q & 1;
    const float d = h2f_bits(*(const uint16_t*)(R + 1664 + 2 * r));
    const h2 m1056 = {(_Float16)-1056.0f, (_Float16)-1056.0f};
    u2 qh[2];
#pragma unroll
    for (int i = 0; i < 2; i++) qh[i] = ld8(R + 1024 + 16 * (r + 16 * i) + 8 * h);
#pragma unroll
    for (int c = 0; c < 4; c++) {
        const u2 ql = ld8(R + 16 * (16 * c + r) + 8 * h);
        const int sc = (int)(int8_t)R[1536 + 32 * (r >> 2) + 4 * (4 * hn + c) + (r & 3)];
        const _Float16 ds = (_Float16)(d * (float)sc);
        const h2 vds = {ds, ds};
        const int sh = 2 * (2 * hn + (c >> 1));
        uint32_t v[2];
#pragma unroll
        for (int e = 0; e < 2; e++) {
            const uint32_t L = e ? ql.y : ql.x, H = e ? qh[c & 1].y : qh[c & 1].x;
            const uint32_t lo = hn ? (L >> 4) & 0x0F0F0F0Fu : L & 0x0F0F0F0Fu;
            v[e] = lo | (((H >> sh) & 0x03030303u) << 4);
        }
        // (1024 + q) - 1056 = q - 32 exactly, then one rounding of (q - 32) * half(d * sc)
        a[c] = make_h8(as_u32((as_h2(perm_lo(v[0])) + m1056) * vds), as_u32((as_h2(perm_hi(v[0])) + m1056) * vds),
                       as_u32((as_h2(perm_lo(v[1])) + m1056) * vds), as_u32((as_h2(perm_hi(v[1])) + m1056) * vds));
    }
}

template <int TYPE>
struct Gcfg {
    static constexpr int GBYTES = TYPE == T_Q4_K ? Q4K_GROUP : Q6K_GROUP;
    static constexpr int PIECES = TYPE == T_Q4_K ? Q4_PIECES : Q6_PIECES;
};

// LDS of one work-group: three stages of activations and raw weights (LDS-DMA runs two steps ahead
// of the step being multiplied).
template <int TYPE, int P>
struct GemmLds {
    static constexpr int X = (BM / 32) * 4 * 1024;                         // fp16 activations of one step
    static constexpr int RAW_DMA = (2 * P * Gcfg<TYPE>::PIECES + 3) / 4;  // 1 KiB DMAs of raw weights
    static constexpr int RAW = RAW_DMA * 1024;
    static constexpr int TOTAL = STAGES * (X + RAW);
};

// Work-group id -> (pair group px, token block ty).  Work-groups are dealt to the 8 XCDs round-robin
// (id % 8); all token blocks of one pair group get the same XCD and consecutive slots there, so the
// group's weights stream from HBM into that XCD's L2 once and serve every token block.
constexpr int XCDS = 8;
__device__ inline bool wg_coords(int id, int npx, int mblocks, int& px, int& ty) {
    const int xcd = id % XCDS, j = id / XCDS;
    px = (j / mblocks) * XCDS + xcd;
    ty = j % mblocks;
    return px < npx;
}

template <int TYPE, int P>
__global__ __launch_bounds__(THREADS) void k_gemm(const uint8_t* __restrict__ w, int ntiles, int nsb, int n,
                                                  const uint8_t* __restrict__ ximg, int m, float* __restrict__ y) {
    using C = Gcfg<TYPE>;
    using L = GemmLds<TYPE, P>;
    static_assert(L::TOTAL <= 160 * 1024, "work-group LDS");
    constexpr int OWN = P / 4, SH = P % 4, NPL = OWN + SH;  // pairs whose fragments a wave builds
    constexpr int XDMA = (BM / 32) * 4 / 4;                  // activation DMAs per wave
    extern __shared__ __align__(16) uint8_t smem[];
    auto sX = [&](int st) { return smem + st * L::X; };
    auto sR = [&](int st) { return smem + STAGES * L::X + st * L::RAW; };

    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int r = lane & 15, u = (lane >> 4) & 1, h = lane >> 5;
    int px, ty;
    if (!wg_coords(blockIdx.x, (ntiles + 2 * P - 1) / (2 * P), (m + BM - 1) / BM, px, ty)) return;
    const int tile0 = px * 2 * P, tn = min(2 * P, ntiles - tile0);
    const int tb0 = ty * (BM / 32);
    const int kchunks = nsb * 16;  // K / 16
    const int steps = nsb * 4;
    const int rcnt = (L::RAW_DMA - wave + 3) / 4;  // raw-weight DMAs this wave issues per step

    auto issue_raw = [&](int s) {  // raw weights of step s -> stage s % 3, 4 pieces per DMA
        const int sb = s >> 2, q = s & 3;
        uint8_t* dst = sR(s % STAGES);
        for (int d = wave; d < L::RAW_DMA; d += 4) {
            const int piece = min(4 * d + (lane >> 4), 2 * P * C::PIECES - 1), li = lane & 15;
            const int t = min(piece / C::PIECES, tn - 1), j = piece % C::PIECES;  // idle tiles re-read a valid one
            const uint8_t* G = w + ((size_t)(tile0 + t) * nsb + sb) * C::GBYTES;
            const uint8_t* src;
            if constexpr (TYPE == T_Q4_K) src = q4_piece_src(G, q, j, li);
            else src = q6_piece_src(G, q, j, li);
            dma16(src, dst + d * 1024);
        }
    };
    auto issue_x = [&](int s) {  // 4 token blocks x K/16 chunks 4s..4s+3 -> stage s % 3
        uint8_t* dst = sX(s % STAGES);
#pragma unroll
        for (int j = 0; j < XDMA; j++) {
            const int rec = wave * XDMA + j, tb = rec >> 2, c = rec & 3;
            dma16(ximg + (((size_t)(tb0 + tb) * kchunks + 4 * s + c) * 64 + lane) * 16, dst + rec * 1024);
        }
    };
    auto pair_of = [&](int i) { return i < OWN ? wave * OWN + i : 4 * OWN + (i - OWN); };

    f16v acc[OWN > 0 ? OWN : 1][4], accs[SH > 0 ? SH : 1];
#pragma unroll
    for (int i = 0; i < (OWN > 0 ? OWN : 1); i++)
#pragma unroll
        for (int b = 0; b < 4; b++)
#pragma unroll
            for (int e = 0; e < 16; e++) acc[i][b][e] = 0.0f;
#pragma unroll
    for (int i = 0; i < (SH > 0 ? SH : 1); i++)
#pragma unroll
        for (int e = 0; e < 16; e++) accs[i][e] = 0.0f;

    // prologue: step 0 landed, step 1 in flight
    issue_raw(0);
    issue_x(0);
    wait_vm<0>();
    if (steps > 1) {
        issue_raw(1);
        issue_x(1);
    }
    __syncthreads();

    Q4Scales sc4[TYPE == T_Q4_K ? NPL : 1];
    for (int sb = 0; sb < nsb; sb++) {
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const int s = 4 * sb + q;
            // step s reads stage s % 3 and issues step s + 2 into the stage step s - 1 released
            int issued = 0;
            if (s + 2 < steps) {
                issue_raw(s + 2);
                issue_x(s + 2);
                issued = rcnt + XDMA;
            }
            const uint8_t* raw = sR(s % STAGES);
            const uint8_t* xl = sX(s % STAGES);
            // raw bytes of this lane's tile (pair i's half u) within the stage
            auto tile_raw = [&](int i) { return raw + (2 * pair_of(i) + u) * C::PIECES * 256; };
            if constexpr (TYPE == T_Q4_K) {
                if (q == 0) {
#pragma unroll
                    for (int i = 0; i < NPL; i++) sc4[i] = q4_scales(tile_raw(i), r);
                }
            }
            auto frags = [&](int i, h8(&a)[4]) {
                if constexpr (TYPE == T_Q4_K) q4_frags(tile_raw(i), sc4[i], q, r, h, a);
                else q6_frags(tile_raw(i), q, r, h, a);
            };
            if constexpr (OWN > 0) {
                h8 b[4][4];
#pragma unroll
                for (int tb = 0; tb < 4; tb++)
#pragma unroll
                    for (int c = 0; c < 4; c++)
                        b[tb][c] = __builtin_bit_cast(h8, *(const u4*)(xl + (tb * 4 + c) * 1024 + 16 * lane));
#pragma unroll
                for (int i = 0; i < OWN; i++) {
                    h8 a[4];
                    frags(i, a);
#pragma unroll
                    for (int c = 0; c < 4; c++)
#pragma unroll
                        for (int tb = 0; tb < 4; tb++) acc[i][tb] = mfma32(a[c], b[tb][c], acc[i][tb]);
                }
            }
            if constexpr (SH > 0) {
                h8 bs[4];  // this wave's token block, read by address (no register indexing)
#pragma unroll
                for (int c = 0; c < 4; c++)
                    bs[c] = __builtin_bit_cast(h8, *(const u4*)(xl + (wave * 4 + c) * 1024 + 16 * lane));
#pragma unroll
                for (int i = 0; i < SH; i++) {
                    h8 a[4];
                    frags(OWN + i, a);
#pragma unroll
                    for (int c = 0; c < 4; c++) accs[i] = mfma32(a[c], bs[c], accs[i]);
                }
            }
            wait_vm_le<16>(issued);  // step s + 1 (issued one step earlier) has landed
            __syncthreads();
        }
    }

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
#pragma unroll
    for (int i = 0; i < OWN; i++)
#pragma unroll
        for (int tb = 0; tb < 4; tb++) store(acc[i][tb], wave * OWN + i, tb);
#pragma unroll
    for (int i = 0; i < SH; i++) store(accs[i], 4 * OWN + i, wave);
}

template <int TYPE, int P>
int launch_p(const uint8_t* w, int ntiles, int nsb, int n, const uint8_t* ximg, int m, float* y, hipStream_t s) {
    constexpr size_t lds = GemmLds<TYPE, P>::TOTAL;
    const int npx = (ntiles + 2 * P - 1) / (2 * P), mblocks = (m + BM - 1) / BM;
    const int grid = (npx + XCDS - 1) / XCDS * XCDS * mblocks;  // ids whose px >= npx exit at once
    hipLaunchKernelGGL((k_gemm<TYPE, P>), dim3(grid), dim3(THREADS), lds, s, w, ntiles, nsb, n, ximg, m, y);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

// Tile pairs per work-group: the candidate that minimises (work-group rounds over the CUs) x P,
// i.e. the time of the busiest CU, preferring larger P (fewer work-groups) on ties.
constexpr int P_CHOICES[] = {2, 3, 4, 5, 8, 9};

int g_gemm_p = 0;  // tuning override (0 = planned)

template <int TYPE>
int launch_type(const uint8_t* w, int ntiles, int nsb, int n, const uint8_t* ximg, int m, float* y, int cus,
                hipStream_t s) {
    int best = 0;
    long long best_cost = 0;
    const int mblocks = (m + BM - 1) / BM, npairs = (ntiles + 1) / 2;
    for (int p : P_CHOICES) {
        if (g_gemm_p && p != g_gemm_p) continue;
        const long long wgs = (long long)((npairs + p - 1) / p) * mblocks;
        const long long cost = (wgs + cus - 1) / cus * p;
        if (!best || cost < best_cost || (cost == best_cost && p > best)) {
            best = p;
            best_cost = cost;
        }
    }
    switch (best) {
        case 2: return launch_p<TYPE, 2>(w, ntiles, nsb, n, ximg, m, y, s);
        case 3: return launch_p<TYPE, 3>(w, ntiles, nsb, n, ximg, m, y, s);
        case 4: return launch_p<TYPE, 4>(w, ntiles, nsb, n, ximg, m, y, s);
        case 5: return launch_p<TYPE, 5>(w, ntiles, nsb, n, ximg, m, y, s);
        case 8: return launch_p<TYPE, 8>(w, ntiles, nsb, n, ximg, m, y, s);
        case 9: return launch_p<TYPE, 9>(w, ntiles, nsb, n, ximg, m, y, s);
    }
    return -1;
}

int g_cus = 0;

}  // namespace

bool gemm_set_pairs(int p) {
    if (p != 0) {
        bool ok = false;
        for (int c : P_CHOICES) ok = ok || c == p;
        if (!ok) return false;
    }
    g_gemm_p = p;
    return true;
}

size_t gemm_image_bytes(int m, int k) { return (size_t)((m + BM - 1) / BM) * BM * k * 2; }

int launch_gemm(int type, const uint8_t* w, int k, int n, const float* x, int m, uint8_t* ximg, float* y,
                hipStream_t s) {
    if (!g_cus) {
        int dev = 0;
        hipDeviceProp_t prop;
        g_cus = (hipGetDevice(&dev) == hipSuccess && hipGetDeviceProperties(&prop, dev) == hipSuccess)
                    ? prop.multiProcessorCount
                    : 256;
    }
    const int mpad = (m + BM - 1) / BM * BM;
    hipLaunchKernelGGL(k_gemm_prep_x, dim3(k / 16, mpad / 32), dim3(64), 0, s, x, m, k, ximg);
    if (hipGetLastError() != hipSuccess) return -1;
    const int ntiles = n / 16, nsb = k / 256;
    if (type == T_Q4_K) return launch_type<T_Q4_K>(w, ntiles, nsb, n, ximg, m, y, g_cus, s);
    if (type == T_Q6_K) return launch_type<T_Q6_K>(w, ntiles, nsb, n, ximg, m, y, g_cus, s);
    return -1;
}

}  // namespace qk
