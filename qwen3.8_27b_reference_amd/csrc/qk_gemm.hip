// Prefill GEMM (m >= 16) for Q4_K / Q6_K weights: super-blocks dequantized into LDS as fp16 tiles
// feeding CDNA4 MFMA (v_mfma_f32_16x16x32_f16), fp32 accumulate.
//
// Replaces the reference's k_gemm_q4k / k_gemm_q6k (qwen_cuda/kernels.cu:307-361, 394, 397-401:
// 64x64x64 tiles, 2x2 warps of mma.m16n8k16, dequant via dq8h into shared memory) with a design
// for 256-CU CDNA4:
//
//  * A work-group owns TN 16-row tiles of W (a T16 tile each) x 128 tokens, so that the number of
//    work-groups is a whole multiple of the CU count for the model's shapes (e.g. N=17408, M=512:
//    1088 tiles = 64 x 17, 64 x 4 token blocks = 256 work-groups, one per CU, no tail round).
//  * K advances 64 elements (a quarter super-block) per step.  Each step the 256 threads read the
//    raw T16 bytes of the quarter into registers, dequantize them to fp16 (the reference's
//    tolerance path, kernels.cu:127-181: scales rounded to fp16, one packed FMA per pair) and
//    store them in LDS already in MFMA A-operand order; the fp16 activation tiles arrive by
//    LDS-DMA from an image written once per call by k_gemm_prep_x (x rounded to fp16, RNE).
//  * 4 waves split the 128 tokens (32 each); every wave multiplies all TN tiles with its two
//    16-token blocks, so each A fragment read from LDS feeds two MFMAs.  Double-buffered LDS:
//    the next step's weights and activations load while the current step's MFMAs run.
//  * y is fp32 [m][n] row-major like the reference's GEMM output (y[tok*n + row]).
#include <type_traits>

#include "qk_device.h"
#include "qk_internal.h"

namespace qk {
namespace {

#define LDS_AS __attribute__((address_space(3)))

constexpr int BM = GEMM_BM;   // tokens per work-group
constexpr int BK = 64;        // K per step (a quarter super-block)
constexpr int THREADS = 256;  // 4 waves

template <int N>
__device__ inline void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

__device__ inline void dma16(const void* g, uint8_t* lds) {
    __builtin_amdgcn_global_load_lds(g, (LDS_AS void*)lds, 16, 0, 0);
}

// ------------------------------------------------------------------------------------------------
// Activation image: x fp32 [m][k] -> fp16 records; record (tb, kc, l) at ((tb * K/32 + kc) * 64 + l)
// * 16 holds x[16*tb + (l & 15)][32*kc + 8*(l >> 4) + 0..7] rounded to nearest even (zeros for
// tokens >= m).  This is the B-operand layout of v_mfma_f32_16x16x32_f16, so one 64-lane 16-byte
// LDS read per (token block, K/32 chunk) feeds an MFMA.
__global__ __launch_bounds__(64) void k_gemm_prep_x(const float* __restrict__ x, int m, int k,
                                                     uint8_t* __restrict__ img) {
    const int kc = blockIdx.x, tb = blockIdx.y, l = threadIdx.x;
    const int tok = 16 * tb + (l & 15), k0 = 32 * kc + 8 * (l >> 4);
    f4 a = {0.0f, 0.0f, 0.0f, 0.0f}, b = a;
    if (tok < m) {
        a = *(const f4*)(x + (size_t)tok * k + k0);
        b = *(const f4*)(x + (size_t)tok * k + k0 + 4);
    }
    const h2 p0 = {(_Float16)a.x, (_Float16)a.y}, p1 = {(_Float16)a.z, (_Float16)a.w};
    const h2 p2 = {(_Float16)b.x, (_Float16)b.y}, p3 = {(_Float16)b.z, (_Float16)b.w};
    *(u4*)(img + (((size_t)tb * (k / 32) + kc) * 64 + l) * 16) = u4{as_u32(p0), as_u32(p1), as_u32(p2), as_u32(p3)};
}

// ------------------------------------------------------------------------------------------------
// Weight tile in LDS: record (t, c, g, r) at ((t*2 + c)*64 + 16g + r)*16 holds
// W[16*tile + r][step*64 + 32c + 8g + 0..7] as fp16: the A operand of lane 16g + r.
__device__ inline uint32_t pk_sub1024(uint32_t v) {  // (1024 + q) - 1024, exact
    return as_u32(as_h2(v) + h2{(_Float16)-1024.0f, (_Float16)-1024.0f});
}

// Q4_K: task (tile t, row r, i) covers qs_r[32q + 16i + 0..15] of quarter q: low nibbles are
// elements 16i + 0..15 of sub-block 2q (chunk 0), high nibbles the same of sub-block 2q+1 (chunk 1)
// (qwen_cpu/quants.h:53-71 element order).
struct Q4Task {
    u4 qs;
    uint32_t dd;          // d | dmin << 16
    uint32_t s0, s1, s2;  // the 12 scale bytes
};

__device__ inline void q4_load(Q4Task& T, const uint8_t* G, int q, int r, int i) {
    T.qs = ld16(G + 1024 * i + 16 * (16 * q + r));
    T.dd = ld4(G + 2048 + 4 * r);
    T.s0 = ld4(G + 2112 + 12 * r);
    T.s1 = ld4(G + 2116 + 12 * r);
    T.s2 = ld4(G + 2120 + 12 * r);
}

// 6-bit scale/min of sub-block j (qwen_cpu/quants.h:33-41) from the 12 scale bytes held as three
// dwords, with shifts only (j is a run-time value; no indexed local array).
__device__ inline void scale_min_dw(int j, uint32_t s0, uint32_t s1, uint32_t s2, int& sc, int& m) {
    const int b = 8 * (j & 3);
    if (j < 4) {
        sc = (s0 >> b) & 63;
        m = (s1 >> b) & 63;
    } else {
        sc = ((s2 >> b) & 0xF) | (((s0 >> b) >> 6 & 3) << 4);
        m = ((s2 >> b) >> 4 & 0xF) | (((s1 >> b) >> 6 & 3) << 4);
    }
}

__device__ inline void q4_store(const Q4Task& T, uint8_t* sw, int t, int q, int r, int i) {
    const float d = h2f_bits(T.dd & 0xFFFFu), dmin = h2f_bits(T.dd >> 16);
    const uint32_t w[4] = {T.qs.x, T.qs.y, T.qs.z, T.qs.w};
#pragma unroll
    for (int c = 0; c < 2; c++) {
        int sc, m;
        scale_min_dw(2 * q + c, T.s0, T.s1, T.s2, sc, m);
        const _Float16 ds = (_Float16)(d * (float)sc), dm = (_Float16)(-(dmin * (float)m));
        const h2 vds = {ds, ds}, vdm = {dm, dm};
        uint32_t o[8];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint32_t nib = c ? (w[j] >> 4) & 0x0F0F0F0Fu : w[j] & 0x0F0F0F0Fu;
            o[2 * j] = pk_fma(pk_sub1024(perm_lo(nib)), vds, vdm);
            o[2 * j + 1] = pk_fma(pk_sub1024(perm_hi(nib)), vds, vdm);
        }
        // elements 16i + 0..7 -> g = 2i, 16i + 8..15 -> g = 2i + 1
        uint8_t* rec = sw + ((t * 2 + c) * 64 + 16 * (2 * i) + r) * 16;
        *(u4*)rec = u4{o[0], o[1], o[2], o[3]};
        *(u4*)(rec + 256) = u4{o[4], o[5], o[6], o[7]};
    }
}

// Q6_K: task (tile t, row r, s1, i) covers elements 32*s1 + 16i + 0..15 of quarter q (= 128n + 32s
// + l' with n = q/2, s = 2(q&1) + s1, l' = 16i + 0..15; qwen_cpu/quants.h:96-121).
struct Q6Task {
    u4 ql, qh;
    uint32_t sc;  // int8 scale (low byte) | d << 16
};

__device__ inline void q6_load(Q6Task& T, const uint8_t* G, int q, int r, int s1, int i) {
    const int n = q >> 1, u = 4 * (q & 1) + 2 * s1 + i;
    T.ql = ld16(G + 1024 * n + 16 * (16 * (2 * s1 + i) + r));
    T.qh = ld16(G + 2048 + 512 * n + 16 * (r + 16 * i));
    const uint32_t scb = G[3072 + 128 * n + 32 * (r >> 2) + 4 * u + (r & 3)];
    const uint32_t d = *(const uint16_t*)(G + 3328 + 2 * r);
    T.sc = scb | (d << 16);
}

__device__ inline void q6_store(const Q6Task& T, uint8_t* sw, int t, int q, int r, int s1, int i) {
    const int hn = q & 1, sh = 2 * (2 * hn + s1);
    const float d = h2f_bits(T.sc >> 16);
    const _Float16 ds = (_Float16)(d * (float)(int)(int8_t)(T.sc & 0xFFu));
    const h2 vds = {ds, ds}, m1056 = {(_Float16)-1056.0f, (_Float16)-1056.0f};
    const uint32_t L[4] = {T.ql.x, T.ql.y, T.ql.z, T.ql.w}, H[4] = {T.qh.x, T.qh.y, T.qh.z, T.qh.w};
    uint32_t o[8];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const uint32_t lo = hn ? (L[j] >> 4) & 0x0F0F0F0Fu : L[j] & 0x0F0F0F0Fu;
        const uint32_t q6 = lo | (((H[j] >> sh) & 0x03030303u) << 4);
        // (1024 + q) - 1056 = q - 32 exactly, then one rounding of (q - 32) * half(d * sc)
        o[2 * j] = as_u32((as_h2(perm_lo(q6)) + m1056) * vds);
        o[2 * j + 1] = as_u32((as_h2(perm_hi(q6)) + m1056) * vds);
    }
    uint8_t* rec = sw + ((t * 2 + s1) * 64 + 16 * (2 * i) + r) * 16;
    *(u4*)rec = u4{o[0], o[1], o[2], o[3]};
    *(u4*)(rec + 256) = u4{o[4], o[5], o[6], o[7]};
}

template <int TYPE>
struct Gcfg {
    static constexpr int TASKS_PER_TILE = TYPE == T_Q4_K ? 32 : 64;
    static constexpr int GBYTES = TYPE == T_Q4_K ? Q4K_GROUP : Q6K_GROUP;
    using Task = typename std::conditional<TYPE == T_Q4_K, Q4Task, Q6Task>::type;
};

template <int TYPE, int TN>
struct GemmLds {
    static constexpr int W = TN * 2 * 1024;     // one step of weights (fp16)
    static constexpr int X = (BM / 16) * 2 * 1024;  // one step of activations (fp16)
    static constexpr int TOTAL = 2 * (W + X);
};

template <int TYPE, int TN>
__global__ __launch_bounds__(THREADS) void k_gemm(const uint8_t* __restrict__ w, int ntiles, int nsb, int n,
                                                  const uint8_t* __restrict__ ximg, int m, float* __restrict__ y) {
    using C = Gcfg<TYPE>;
    using L = GemmLds<TYPE, TN>;
    constexpr int NT = (TN * C::TASKS_PER_TILE + THREADS - 1) / THREADS;  // tasks per thread
    extern __shared__ __align__(16) uint8_t smem[];
    auto sW = [&](int b) { return smem + b * L::W; };          // fp16 weight tile, buffer b
    auto sX = [&](int b) { return smem + 2 * L::W + b * L::X; };  // fp16 activation tile, buffer b

    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int tile0 = blockIdx.x * TN, tn = min(TN, ntiles - tile0);
    const int tb0 = blockIdx.y * (BM / 16);  // first 16-token block of this work-group
    const int kchunks = nsb * 8;             // K / 32
    const int steps = nsb * 4;

    typename C::Task task[NT];
    auto load_w = [&](int s) {
        const int sb = s >> 2, q = s & 3;
#pragma unroll
        for (int j = 0; j < NT; j++) {
            const int id = tid + j * THREADS, t = id / C::TASKS_PER_TILE, rem = id % C::TASKS_PER_TILE;
            if (t < tn) {
                const uint8_t* G = w + ((size_t)(tile0 + t) * nsb + sb) * C::GBYTES;
                if constexpr (TYPE == T_Q4_K) q4_load(task[j], G, q, rem & 15, rem >> 4);
                else q6_load(task[j], G, q, rem & 15, (rem >> 4) & 1, rem >> 5);
            }
        }
    };
    auto store_w = [&](int s, uint8_t* dst) {
        const int q = s & 3;
#pragma unroll
        for (int j = 0; j < NT; j++) {
            const int id = tid + j * THREADS, t = id / C::TASKS_PER_TILE, rem = id % C::TASKS_PER_TILE;
            if (t < tn) {
                if constexpr (TYPE == T_Q4_K) q4_store(task[j], dst, t, q, rem & 15, rem >> 4);
                else q6_store(task[j], dst, t, q, rem & 15, (rem >> 4) & 1, rem >> 5);
            }
        }
    };
    // activations of step s: token blocks tb0..tb0+7, K/32 chunks 2s, 2s+1 -> 16 records of 1 KiB,
    // four LDS-DMA instructions per wave
    constexpr int XDMA = (BM / 16) * 2 / 4;
    auto load_x = [&](int s, uint8_t* dst) {
#pragma unroll
        for (int j = 0; j < XDMA; j++) {
            const int rec = wave * XDMA + j, tb = rec >> 1, c = rec & 1;
            dma16(ximg + (((size_t)(tb0 + tb) * kchunks + 2 * s + c) * 64 + lane) * 16, dst + rec * 1024);
        }
    };

    f4 acc[TN][2];
#pragma unroll
    for (int t = 0; t < TN; t++) acc[t][0] = acc[t][1] = f4{0.0f, 0.0f, 0.0f, 0.0f};

    // prologue: step 0 into buffer 0
    load_w(0);
    load_x(0, sX(0));
    wait_vm<0>();
    store_w(0, sW(0));
    __syncthreads();

    for (int s = 0; s < steps; s++) {
        const int cur = s & 1, nxt = cur ^ 1;
        const bool more = s + 1 < steps;
        if (more) {
            load_w(s + 1);           // global -> registers, consumed after this step's MFMAs
            load_x(s + 1, sX(nxt));  // LDS-DMA into the idle buffer
        }
        const uint8_t* wl = sW(cur);
        const uint8_t* xl = sX(cur) + (2 * wave) * 2 * 1024;
#pragma unroll
        for (int c = 0; c < 2; c++) {
            const h8 b0 = __builtin_bit_cast(h8, *(const u4*)(xl + (0 * 2 + c) * 1024 + 16 * lane));
            const h8 b1 = __builtin_bit_cast(h8, *(const u4*)(xl + (1 * 2 + c) * 1024 + 16 * lane));
#pragma unroll
            for (int t = 0; t < TN; t++) {
                const h8 a = __builtin_bit_cast(h8, *(const u4*)(wl + ((t * 2 + c) * 64 + lane) * 16));
                acc[t][0] = mfma(a, b0, acc[t][0]);
                acc[t][1] = mfma(a, b1, acc[t][1]);
            }
        }
        if (more) {
            wait_vm<XDMA>();  // the weight loads (issued before the DMAs) have landed
            store_w(s + 1, sW(nxt));
            wait_vm<0>();
        }
        __syncthreads();
    }

    // lane holds rows 4g..4g+3 of tile t for token 16*tb + (lane & 15)
    const int g = lane >> 4;
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const int tok = 16 * (tb0 + 2 * wave + j) + (lane & 15);
        if (tok < m) {
#pragma unroll
            for (int t = 0; t < TN; t++)
                if (t < tn) *(f4*)(y + (size_t)tok * n + (size_t)(tile0 + t) * 16 + 4 * g) = acc[t][j];
        }
    }
}

template <int TYPE, int TN>
int launch_tn(const uint8_t* w, int ntiles, int nsb, int n, const uint8_t* ximg, int m, float* y, hipStream_t s) {
    constexpr size_t lds = GemmLds<TYPE, TN>::TOTAL;
    const dim3 grid((ntiles + TN - 1) / TN, (m + BM - 1) / BM);
    hipLaunchKernelGGL((k_gemm<TYPE, TN>), grid, dim3(THREADS), lds, s, w, ntiles, nsb, n, ximg, m, y);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

// Tiles per work-group: the candidate that minimises (work-group rounds over the CUs) x TN, i.e.
// the time of the slowest CU, preferring larger TN (more MFMAs per A read) on ties.
constexpr int TN_CHOICES[] = {4, 5, 8, 10, 16, 17};

int g_gemm_tn = 0;  // tuning override

template <int TYPE>
int launch_type(const uint8_t* w, int ntiles, int nsb, int n, const uint8_t* ximg, int m, float* y, int cus,
                hipStream_t s) {
    int best = 0;
    long long best_cost = 0;
    const int mblocks = (m + BM - 1) / BM;
    for (int tn : TN_CHOICES) {
        if (g_gemm_tn && tn != g_gemm_tn) continue;
        const long long wgs = (long long)((ntiles + tn - 1) / tn) * mblocks;
        const long long cost = (wgs + cus - 1) / cus * tn;
        if (!best || cost < best_cost || (cost == best_cost && tn > best)) {
            best = tn;
            best_cost = cost;
        }
    }
    switch (best) {
        case 4: return launch_tn<TYPE, 4>(w, ntiles, nsb, n, ximg, m, y, s);
        case 5: return launch_tn<TYPE, 5>(w, ntiles, nsb, n, ximg, m, y, s);
        case 8: return launch_tn<TYPE, 8>(w, ntiles, nsb, n, ximg, m, y, s);
        case 10: return launch_tn<TYPE, 10>(w, ntiles, nsb, n, ximg, m, y, s);
        case 16: return launch_tn<TYPE, 16>(w, ntiles, nsb, n, ximg, m, y, s);
        case 17: return launch_tn<TYPE, 17>(w, ntiles, nsb, n, ximg, m, y, s);
    }
    return -1;
}

int g_cus = 0;

}  // namespace

void gemm_set_tn(int tn) { g_gemm_tn = tn; }

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
    hipLaunchKernelGGL(k_gemm_prep_x, dim3(k / 32, mpad / 16), dim3(64), 0, s, x, m, k, ximg);
    if (hipGetLastError() != hipSuccess) return -1;
    const int ntiles = n / 16, nsb = k / 256;
    if (type == T_Q4_K) return launch_type<T_Q4_K>(w, ntiles, nsb, n, ximg, m, y, g_cus, s);
    if (type == T_Q6_K) return launch_type<T_Q6_K>(w, ntiles, nsb, n, ximg, m, y, g_cus, s);
    return -1;
}

}  // namespace qk
