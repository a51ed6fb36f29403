// TEST INFRASTRUCTURE — the parity oracle.  Only tests/, __graft_entry__.smoke() and bench.py's
// cpu_baseline leg may load this library, and only as the checker / the timed CPU baseline.  The
// product (libqk.so) never links, loads or calls it.
//
// A CPU restatement, written from the reference's behaviour, of its quantized-matmul path:
//   * GGUF block formats and row sizes ............ qwen_cpu/quants.h:13-31, docs/model.md:263-318
//   * exact fp16 -> fp32 widening with subnormals .. qwen_cuda/quants_ref.h:19-37
//   * 6-bit scale/min unpack ....................... qwen_cpu/quants.h:33-41
//   * scalar dequant Q8_0/Q4_K/Q5_K/Q6_K ........... qwen_cpu/quants.h:45-121 (Ref::*)
//   * AVX-512 dequant Q4_K/Q6_K (same bits) ........ qwen_cpu/quants.h:141-189
//   * matmul: 4-row tasks, each row dequantized once to fp32, NT<=4-token micro-kernels with
//     16-lane fp32 FMA accumulators and a tree reduction ... qwen_cpu/ops.h:34-76
//   * atomic-counter thread pool, caller participates ... qwen_cpu/pool.h:24-73
//   * splitmix64 mixing constants .................. qwen_cpu/qwen.cpp:314-319
//   * double-precision brute-force dot used as the error yardstick ... qwen_cpu/qwen.cpp:889-899
// Synthetic-input generators (counter-based splitmix64 streams) are this repository's own
// definition of the BASELINE configs' input distributions.
//
// Pinning (all in tests/test_oracle.py): fp16 widening is checked exhaustively against an exact
// double conversion; scale unpack against the pack/unpack bijection and the index formulas;
// dequant against the closed forms (d*sc)*q - dmin*m and (d*sc)*(q-32) computed in double and
// rounded once; matmul against the f64 brute force and bitwise against oracle/_ref (the
// reference's own AVX-512 code compiled from /root/reference) where that library is present.
#include <atomic>
#include <chrono>
#include <cmath>
#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <thread>
#include <vector>
#include <immintrin.h>

namespace {

enum : uint32_t { T_F32 = 0, T_Q8_0 = 8, T_Q4_K = 12, T_Q5_K = 13, T_Q6_K = 14 };
constexpr int KMAX = 17408;  // largest input dim of the model (ops.h:15)
constexpr int ROWS = 4;      // output rows per task (ops.h:16)

// ---------------------------------------------------------------- fp16 <-> fp32
float h2f(uint16_t h) {  // exact, subnormals included (quants_ref.h:19-37 semantics)
    uint32_t s = (uint32_t)(h >> 15) << 31, e = (h >> 10) & 31, m = h & 1023, bits;
    if (e == 31) {
        bits = s | 0x7f800000u | (m << 13);
    } else if (e) {
        bits = s | ((e + 112) << 23) | (m << 13);
    } else if (m) {  // subnormal: value m * 2^-24, renormalise
        int sh = 0;
        while (!(m & 1024)) { m <<= 1; sh++; }
        bits = s | ((uint32_t)(113 - sh) << 23) | ((m & 1023) << 13);
    } else {
        bits = s;
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

uint16_t f2h_rne(float f) {  // IEEE round-to-nearest-even, subnormals and overflow to inf handled
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u : 0));
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);  // rounds to >= 65520 -> inf
    int e = (int)(ax >> 23) - 127;
    uint32_t mant = (ax & 0x7fffffu) | 0x800000u;
    if (e >= -14) {  // normal half
        uint32_t hm = mant >> 13, rem = mant & 0x1fffu;
        uint32_t he = (uint32_t)(e + 15);
        uint32_t r = (he << 10) | (hm & 0x3ffu);
        if (rem > 0x1000u || (rem == 0x1000u && (r & 1))) r++;
        return (uint16_t)(sign | r);
    }
    if (e < -25) return (uint16_t)sign;  // below half of the smallest subnormal
    // subnormal half: value = mant * 2^(e-23); unit 2^-24 -> shift = -(e-23) - 24 = -e - 1
    int shift = -e - 1;  // in [14, 24]
    uint32_t hm = mant >> shift, rem = mant & ((1u << shift) - 1), half = 1u << (shift - 1);
    if (rem > half || (rem == half && (hm & 1))) hm++;
    return (uint16_t)(sign | hm);
}

// ---------------------------------------------------------------- block formats (quants.h:13-17)
struct BlockQ8_0 { uint16_t d; int8_t qs[32]; };
struct BlockQ4K { uint16_t d, dmin; uint8_t scales[12]; uint8_t qs[128]; };
struct BlockQ5K { uint16_t d, dmin; uint8_t scales[12]; uint8_t qh[32]; uint8_t qs[128]; };
struct BlockQ6K { uint8_t ql[128]; uint8_t qh[64]; int8_t scales[16]; uint16_t d; };
static_assert(sizeof(BlockQ8_0) == 34 && sizeof(BlockQ4K) == 144 && sizeof(BlockQ5K) == 176 &&
                  sizeof(BlockQ6K) == 210,
              "GGUF block sizes");

size_t row_bytes(uint32_t type, int64_t k) {  // quants.h:21-31; 0 for an unknown type
    switch (type) {
        case T_F32: return (size_t)k * 4;
        case T_Q8_0: return (size_t)(k / 32) * sizeof(BlockQ8_0);
        case T_Q4_K: return (size_t)(k / 256) * sizeof(BlockQ4K);
        case T_Q5_K: return (size_t)(k / 256) * sizeof(BlockQ5K);
        case T_Q6_K: return (size_t)(k / 256) * sizeof(BlockQ6K);
    }
    return 0;
}

// quants.h:33-41: sub-block j of 8; j<4 keep the low 6 bits of bytes j / j+4, j>=4 rebuild the
// 6-bit values from a nibble of byte j+4 and the top two bits of bytes j-4 / j.
void scale_min_k4(int j, const uint8_t* q, uint8_t* sc, uint8_t* m) {
    if (j < 4) {
        *sc = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *sc = (uint8_t)((q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4));
        *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

// ---------------------------------------------------------------- scalar dequant (quants.h:45-121)
void dq_q8_0(const void* src, float* y, int64_t k) {
    const BlockQ8_0* b = (const BlockQ8_0*)src;
    for (int64_t i = 0; i < k / 32; i++) {
        const float d = h2f(b[i].d);
        for (int e = 0; e < 32; e++) y[i * 32 + e] = (float)b[i].qs[e] * d;
    }
}

void dq_q4_k(const void* src, float* y, int64_t k) {
    const BlockQ4K* b = (const BlockQ4K*)src;
    for (int64_t i = 0; i < k / 256; i++) {
        const float d = h2f(b[i].d), dmin = h2f(b[i].dmin);
        float* out = y + i * 256;
        for (int g = 0; g < 4; g++) {  // 64 elements share 32 qs bytes: low nibbles then high nibbles
            for (int h = 0; h < 2; h++) {
                uint8_t sc, m;
                scale_min_k4(2 * g + h, b[i].scales, &sc, &m);
                const float d1 = d * (float)sc, m1 = dmin * (float)m;
                for (int l = 0; l < 32; l++) {
                    const int q = (b[i].qs[32 * g + l] >> (4 * h)) & 0xF;
                    out[64 * g + 32 * h + l] = d1 * (float)q - m1;
                }
            }
        }
    }
}

void dq_q5_k(const void* src, float* y, int64_t k) {
    const BlockQ5K* b = (const BlockQ5K*)src;
    for (int64_t i = 0; i < k / 256; i++) {
        const float d = h2f(b[i].d), dmin = h2f(b[i].dmin);
        float* out = y + i * 256;
        for (int g = 0; g < 4; g++) {
            for (int h = 0; h < 2; h++) {
                uint8_t sc, m;
                scale_min_k4(2 * g + h, b[i].scales, &sc, &m);
                const float d1 = d * (float)sc, m1 = dmin * (float)m;
                for (int l = 0; l < 32; l++) {
                    const int q = ((b[i].qs[32 * g + l] >> (4 * h)) & 0xF) + (((b[i].qh[l] >> (2 * g + h)) & 1) << 4);
                    out[64 * g + 32 * h + l] = d1 * (float)q - m1;
                }
            }
        }
    }
}

void dq_q6_k(const void* src, float* y, int64_t k) {
    const BlockQ6K* b = (const BlockQ6K*)src;
    for (int64_t i = 0; i < k / 256; i++) {
        const float d = h2f(b[i].d);
        float* out = y + i * 256;
        for (int e = 0; e < 256; e++) {  // e = 128n + 32s + l
            const int n = e >> 7, s = (e >> 5) & 3, l = e & 31;
            const int lo = (b[i].ql[64 * n + 32 * (s & 1) + l] >> (s >= 2 ? 4 : 0)) & 0xF;
            const int hi = (b[i].qh[32 * n + l] >> (2 * s)) & 3;
            const int q = (lo | (hi << 4)) - 32;
            out[e] = (d * (float)b[i].scales[e >> 4]) * (float)q;
        }
    }
}

int dequant_scalar(uint32_t type, const void* src, float* y, int64_t k) {
    switch (type) {
        case T_F32: memcpy(y, src, (size_t)k * 4); return 0;
        case T_Q8_0: dq_q8_0(src, y, k); return 0;
        case T_Q4_K: dq_q4_k(src, y, k); return 0;
        case T_Q5_K: dq_q5_k(src, y, k); return 0;
        case T_Q6_K: dq_q6_k(src, y, k); return 0;
    }
    return -1;
}

// ---------------------------------------------------------------- AVX-512 dequant (quants.h:141-189)
#define AVX512_TARGET __attribute__((target("avx512f,avx512bw,avx512dq,avx512vl,f16c,fma")))

AVX512_TARGET void avx_q4_k(const void* src, float* y, int64_t k) {
    const BlockQ4K* b = (const BlockQ4K*)src;
    const __m256i m4 = _mm256_set1_epi8(0xF);
    for (int64_t i = 0; i < k / 256; i++) {
        const float d = h2f(b[i].d), dmin = h2f(b[i].dmin);
        for (int g = 0; g < 4; g++) {
            uint8_t sc, m;
            scale_min_k4(2 * g, b[i].scales, &sc, &m);
            const __m512 dlo = _mm512_set1_ps(d * (float)sc), mlo = _mm512_set1_ps(dmin * (float)m);
            scale_min_k4(2 * g + 1, b[i].scales, &sc, &m);
            const __m512 dhi = _mm512_set1_ps(d * (float)sc), mhi = _mm512_set1_ps(dmin * (float)m);
            const __m256i raw = _mm256_loadu_si256((const __m256i*)(b[i].qs + 32 * g));
            const __m256i lo = _mm256_and_si256(raw, m4);
            const __m256i hi = _mm256_and_si256(_mm256_srli_epi16(raw, 4), m4);
            float* out = y + i * 256 + 64 * g;
            _mm512_storeu_ps(out + 0, _mm512_fmsub_ps(dlo, _mm512_cvtepi32_ps(_mm512_cvtepu8_epi32(_mm256_castsi256_si128(lo))), mlo));
            _mm512_storeu_ps(out + 16, _mm512_fmsub_ps(dlo, _mm512_cvtepi32_ps(_mm512_cvtepu8_epi32(_mm256_extracti128_si256(lo, 1))), mlo));
            _mm512_storeu_ps(out + 32, _mm512_fmsub_ps(dhi, _mm512_cvtepi32_ps(_mm512_cvtepu8_epi32(_mm256_castsi256_si128(hi))), mhi));
            _mm512_storeu_ps(out + 48, _mm512_fmsub_ps(dhi, _mm512_cvtepi32_ps(_mm512_cvtepu8_epi32(_mm256_extracti128_si256(hi, 1))), mhi));
        }
    }
}

AVX512_TARGET void avx_q6_k(const void* src, float* y, int64_t k) {
    const BlockQ6K* b = (const BlockQ6K*)src;
    const __m256i m4 = _mm256_set1_epi8(0xF), m2 = _mm256_set1_epi8(3), c32 = _mm256_set1_epi8(32);
    for (int64_t i = 0; i < k / 256; i++) {
        const float d = h2f(b[i].d);
        for (int n = 0; n < 2; n++) {
            const __m256i l0 = _mm256_loadu_si256((const __m256i*)(b[i].ql + 64 * n));
            const __m256i l1 = _mm256_loadu_si256((const __m256i*)(b[i].ql + 64 * n + 32));
            const __m256i h = _mm256_loadu_si256((const __m256i*)(b[i].qh + 32 * n));
            __m256i q[4];  // mask bytes before shifting so 16-bit shifts never pull in the neighbour
            q[0] = _mm256_or_si256(_mm256_and_si256(l0, m4), _mm256_slli_epi16(_mm256_and_si256(h, m2), 4));
            q[1] = _mm256_or_si256(_mm256_and_si256(l1, m4), _mm256_slli_epi16(_mm256_and_si256(_mm256_srli_epi16(h, 2), m2), 4));
            q[2] = _mm256_or_si256(_mm256_and_si256(_mm256_srli_epi16(l0, 4), m4), _mm256_slli_epi16(_mm256_and_si256(_mm256_srli_epi16(h, 4), m2), 4));
            q[3] = _mm256_or_si256(_mm256_and_si256(_mm256_srli_epi16(l1, 4), m4), _mm256_slli_epi16(_mm256_and_si256(_mm256_srli_epi16(h, 6), m2), 4));
            const int8_t* sc = b[i].scales + 8 * n;
            float* out = y + i * 256 + 128 * n;
            for (int s = 0; s < 4; s++) {
                const __m256i qs = _mm256_sub_epi8(q[s], c32);
                _mm512_storeu_ps(out + 32 * s, _mm512_mul_ps(_mm512_cvtepi32_ps(_mm512_cvtepi8_epi32(_mm256_castsi256_si128(qs))), _mm512_set1_ps(d * (float)sc[2 * s])));
                _mm512_storeu_ps(out + 32 * s + 16, _mm512_mul_ps(_mm512_cvtepi32_ps(_mm512_cvtepi8_epi32(_mm256_extracti128_si256(qs, 1))), _mm512_set1_ps(d * (float)sc[2 * s + 1])));
            }
        }
    }
}

bool g_avx512 = false;
bool g_avx512_probed = false;
bool has_avx512() {
    if (!g_avx512_probed) {
        __builtin_cpu_init();
        g_avx512 = __builtin_cpu_supports("avx512f") && __builtin_cpu_supports("avx512bw") &&
                   __builtin_cpu_supports("avx512dq") && __builtin_cpu_supports("avx512vl") &&
                   __builtin_cpu_supports("fma") && __builtin_cpu_supports("f16c");
        g_avx512_probed = true;
    }
    return g_avx512;
}

int dequant_fast(uint32_t type, const void* src, float* y, int64_t k) {  // quants.h:193-203 dispatch
    if (has_avx512()) {
        if (type == T_Q4_K) { avx_q4_k(src, y, k); return 0; }
        if (type == T_Q6_K) { avx_q6_k(src, y, k); return 0; }
    }
    return dequant_scalar(type, src, y, k);
}

// ---------------------------------------------------------------- thread pool (pool.h:24-73)
struct Pool {
    int n = 1;
    std::atomic<uint32_t> gen{0};
    std::atomic<int> next{0}, pending{0};
    int items = 0;
    void (*fn)(void*, int, int) = nullptr;
    void* ctx = nullptr;

    void work(int tid) {
        for (;;) {
            const int i = next.fetch_add(1, std::memory_order_relaxed);
            if (i >= items) return;
            fn(ctx, i, tid);
        }
    }
    void worker(int tid) {
        uint32_t seen = 0;
        for (;;) {
            uint32_t g;
            for (int s = 0;; s++) {  // spin first, then sleep on the generation counter
                g = gen.load(std::memory_order_acquire);
                if (g != seen) break;
                if (s < 20000) _mm_pause();
                else gen.wait(seen, std::memory_order_acquire);
            }
            seen = g;
            work(tid);
            pending.fetch_sub(1, std::memory_order_release);
        }
    }
    void start(int threads) {
        n = threads < 1 ? 1 : threads;
        for (int i = 1; i < n; i++) std::thread(&Pool::worker, this, i).detach();
    }
    template <class F> void run(int nitems, F&& f) {
        if (nitems <= 0) return;
        if (n == 1 || nitems == 1) {
            for (int i = 0; i < nitems; i++) f(i, 0);
            return;
        }
        using FT = std::remove_reference_t<F>;
        fn = [](void* c, int i, int tid) { (*(FT*)c)(i, tid); };
        ctx = (void*)&f;
        items = nitems;
        next.store(0, std::memory_order_relaxed);
        pending.store(n - 1, std::memory_order_relaxed);
        gen.fetch_add(1, std::memory_order_release);
        gen.notify_all();
        work(0);
        while (pending.load(std::memory_order_acquire) != 0) _mm_pause();
    }
};

Pool* g_pool = nullptr;
std::vector<float*> g_tbuf;  // per-thread dequant buffers, ROWS x KMAX floats (ops.h:26-30)

// ---------------------------------------------------------------- matmul micro-kernels (ops.h:34-51)
// Lane i of each 16-lane accumulator sums k = i, i+16, ... with fused multiply-adds; the final
// horizontal sum is the tree (a[i]+a[i+8]) -> (+4) -> (+2) -> (+1), the order of
// _mm512_reduce_add_ps, so the scalar and AVX-512 forms give identical bits.
AVX512_TARGET void micro_avx(int nt, const float* const* wr, const float* x, int k, float* y, int ldy) {
    __m512 acc[4][ROWS];
    for (int t = 0; t < nt; t++)
        for (int r = 0; r < ROWS; r++) acc[t][r] = _mm512_setzero_ps();
    for (int i = 0; i < k; i += 16) {
        const __m512 w0 = _mm512_loadu_ps(wr[0] + i), w1 = _mm512_loadu_ps(wr[1] + i);
        const __m512 w2 = _mm512_loadu_ps(wr[2] + i), w3 = _mm512_loadu_ps(wr[3] + i);
        for (int t = 0; t < nt; t++) {
            const __m512 xv = _mm512_loadu_ps(x + (size_t)t * k + i);
            acc[t][0] = _mm512_fmadd_ps(w0, xv, acc[t][0]);
            acc[t][1] = _mm512_fmadd_ps(w1, xv, acc[t][1]);
            acc[t][2] = _mm512_fmadd_ps(w2, xv, acc[t][2]);
            acc[t][3] = _mm512_fmadd_ps(w3, xv, acc[t][3]);
        }
    }
    for (int t = 0; t < nt; t++)
        for (int r = 0; r < ROWS; r++) y[(size_t)t * ldy + r] = _mm512_reduce_add_ps(acc[t][r]);
}

float tree16(const float* a) {
    float b[8], c[4];
    for (int i = 0; i < 8; i++) b[i] = a[8 + i] + a[i];
    for (int i = 0; i < 4; i++) c[i] = b[4 + i] + b[i];
    const float d0 = c[0] + c[2], d1 = c[1] + c[3];
    return d0 + d1;
}

void micro_scalar(int nt, const float* const* wr, const float* x, int k, float* y, int ldy) {
    float acc[4][ROWS][16] = {};
    for (int i = 0; i < k; i += 16)
        for (int t = 0; t < nt; t++)
            for (int r = 0; r < ROWS; r++)
                for (int l = 0; l < 16; l++) acc[t][r][l] = fmaf(wr[r][i + l], x[(size_t)t * k + i + l], acc[t][r][l]);
    for (int t = 0; t < nt; t++)
        for (int r = 0; r < ROWS; r++) y[(size_t)t * ldy + r] = tree16(acc[t][r]);
}

// ---------------------------------------------------------------- splitmix64 streams
constexpr uint64_t GAMMA = 0x9e3779b97f4a7c15ULL;
inline uint64_t mix64(uint64_t z) {  // finaliser of qwen_cpu/qwen.cpp:314-319
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ULL;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebULL;
    return z ^ (z >> 31);
}
// Output number i (0-based) of the splitmix64 generator seeded with `seed`: random access, so the
// GPU fill kernels and this host code produce the same bytes in any order.
inline uint64_t sm_at(uint64_t seed, uint64_t i) { return mix64(seed + (i + 1) * GAMMA); }
inline uint8_t sm_byte(uint64_t r) { return (uint8_t)(r >> 56); }
inline float sm_u24(uint64_t r) { return (float)(r >> 40) * (1.0f / 16777216.0f); }

}  // namespace

extern "C" {

float qko_fp16_to_f32(uint16_t h) { return h2f(h); }
uint16_t qko_f32_to_fp16(float f) { return f2h_rne(f); }
unsigned long long qko_row_bytes(uint32_t type, long long k) { return row_bytes(type, k); }
void qko_scale_min_k4(int j, const uint8_t* q, uint8_t* sc, uint8_t* m) { scale_min_k4(j, q, sc, m); }
int qko_has_avx512(void) { return has_avx512() ? 1 : 0; }

int qko_dequant_row(uint32_t type, const void* src, float* y, long long k) { return dequant_scalar(type, src, y, k); }
int qko_dequant_row_fast(uint32_t type, const void* src, float* y, long long k) { return dequant_fast(type, src, y, k); }

// Starts the worker pool (idempotent; the first call fixes the thread count).
int qko_init(int threads) {
    if (g_pool) return g_pool->n;
    g_pool = new Pool();
    g_pool->start(threads);
    g_tbuf.resize(g_pool->n);
    for (int i = 0; i < g_pool->n; i++) g_tbuf[i] = (float*)aligned_alloc(64, sizeof(float) * ROWS * KMAX);
    return g_pool->n;
}

// y[t][r] = sum_k W[r][k] * x[t][k] over GGUF-layout rows (ops.h:54-76).  force_scalar selects the
// portable form (same bits).  Returns 0, or -1 on an unsupported type/shape.
int qko_matmul(const uint8_t* w, uint32_t type, int k, int n, const float* x, int T, float* y, int force_scalar) {
    const size_t rb = row_bytes(type, k);
    if (!g_pool || rb == 0 || k > KMAX || k % 256 || n % ROWS || T < 1) return -1;
    const bool avx = has_avx512() && !force_scalar;
    g_pool->run(n / ROWS, [&](int item, int tid) {
        const int n0 = item * ROWS;
        const float* wr[ROWS];
        for (int r = 0; r < ROWS; r++) {
            const uint8_t* src = w + (size_t)(n0 + r) * rb;
            if (type == T_F32) { wr[r] = (const float*)src; continue; }
            float* dst = g_tbuf[tid] + (size_t)r * KMAX;
            if (avx) dequant_fast(type, src, dst, k);
            else dequant_scalar(type, src, dst, k);
            wr[r] = dst;
        }
        for (int t = 0; t < T; t += 4) {
            const int nt = T - t < 4 ? T - t : 4;
            if (avx) micro_avx(nt, wr, x + (size_t)t * k, k, y + (size_t)t * n + n0, n);
            else micro_scalar(nt, wr, x + (size_t)t * k, k, y + (size_t)t * n + n0, n);
        }
    });
    return 0;
}

// The CPU baseline's timing loop when the reference build cannot run (same contract as the reference
// wrapper's qkref_time_seq): matmul i of `count` in order, `reps` times over; elapsed nanoseconds.
long long qko_time_seq(int count, const uint8_t* const* w, const uint32_t* types, const int* ks, const int* ns,
                       const float* const* xs, int T, float* const* ys, int reps) {
    const auto t0 = std::chrono::steady_clock::now();
    for (int r = 0; r < reps; r++)
        for (int i = 0; i < count; i++)
            if (qko_matmul(w[i], types[i], ks[i], ns[i], xs[i], T, ys[i], 0)) return -1;
    return (long long)std::chrono::duration_cast<std::chrono::nanoseconds>(std::chrono::steady_clock::now() - t0)
        .count();
}

// Brute force in double over the exactly dequantized rows: ref[t][r] = sum w*x and
// mag[t][r] = sum |w*x| (the yardstick of qwen_cpu/qwen.cpp:889-899, qwen_cuda/qwen.cpp:1346-1353).
int qko_matmul_f64(const uint8_t* w, uint32_t type, int k, int n, const float* x, int T, double* ref, double* mag) {
    const size_t rb = row_bytes(type, k);
    if (rb == 0 || k % 256) return -1;
    std::vector<float> row((size_t)k);
    for (int r = 0; r < n; r++) {
        dequant_scalar(type, w + (size_t)r * rb, row.data(), k);
        for (int t = 0; t < T; t++) {
            double s = 0, a = 0;
            const float* xt = x + (size_t)t * k;
            for (int i = 0; i < k; i++) {
                const double p = (double)row[i] * (double)xt[i];
                s += p;
                a += fabs(p);
            }
            ref[(size_t)t * n + r] = s;
            if (mag) mag[(size_t)t * n + r] = a;
        }
    }
    return 0;
}

// ---------------------------------------------------------------- synthetic inputs
// Q4_K: one stream output per field, fields in struct order: d, dmin, scales[12], qs[128]
// (142 outputs per block).  d, dmin = fp16_rne(u24 * 0.01); bytes = top 8 bits of the output.
void qko_fill_q4k(uint64_t seed, uint64_t block0, uint64_t nblocks, uint8_t* dst) {
    for (uint64_t b = 0; b < nblocks; b++) {
        const uint64_t base = (block0 + b) * 142;
        BlockQ4K blk;
        blk.d = f2h_rne(sm_u24(sm_at(seed, base + 0)) * 0.01f);
        blk.dmin = f2h_rne(sm_u24(sm_at(seed, base + 1)) * 0.01f);
        for (int i = 0; i < 12; i++) blk.scales[i] = sm_byte(sm_at(seed, base + 2 + i));
        for (int i = 0; i < 128; i++) blk.qs[i] = sm_byte(sm_at(seed, base + 14 + i));
        memcpy(dst + b * sizeof(BlockQ4K), &blk, sizeof(BlockQ4K));
    }
}

// Q6_K: fields in struct order ql[128], qh[64], scales[16], d (209 outputs per block);
// scales = (int8)((r % 64) - 32), d = fp16_rne(u24 * 0.005).
void qko_fill_q6k(uint64_t seed, uint64_t block0, uint64_t nblocks, uint8_t* dst) {
    for (uint64_t b = 0; b < nblocks; b++) {
        const uint64_t base = (block0 + b) * 209;
        BlockQ6K blk;
        for (int i = 0; i < 128; i++) blk.ql[i] = sm_byte(sm_at(seed, base + i));
        for (int i = 0; i < 64; i++) blk.qh[i] = sm_byte(sm_at(seed, base + 128 + i));
        for (int i = 0; i < 16; i++) blk.scales[i] = (int8_t)((int)(sm_at(seed, base + 192 + i) % 64) - 32);
        blk.d = f2h_rne(sm_u24(sm_at(seed, base + 208)) * 0.005f);
        memcpy(dst + b * sizeof(BlockQ6K), &blk, sizeof(BlockQ6K));
    }
}

// Q5_K: fields in struct order d, dmin, scales[12], qh[32], qs[128] (174 outputs per block), drawn as
// for Q4_K.
void qko_fill_q5k(uint64_t seed, uint64_t block0, uint64_t nblocks, uint8_t* dst) {
    for (uint64_t b = 0; b < nblocks; b++) {
        const uint64_t base = (block0 + b) * 174;
        BlockQ5K blk;
        blk.d = f2h_rne(sm_u24(sm_at(seed, base + 0)) * 0.01f);
        blk.dmin = f2h_rne(sm_u24(sm_at(seed, base + 1)) * 0.01f);
        for (int i = 0; i < 12; i++) blk.scales[i] = sm_byte(sm_at(seed, base + 2 + i));
        for (int i = 0; i < 32; i++) blk.qh[i] = sm_byte(sm_at(seed, base + 14 + i));
        for (int i = 0; i < 128; i++) blk.qs[i] = sm_byte(sm_at(seed, base + 46 + i));
        memcpy(dst + b * sizeof(BlockQ5K), &blk, sizeof(BlockQ5K));
    }
}

// Q8_0, counted in runs of eight blocks (256 weights): block j of run b is stream block 8b + j with
// 33 outputs, d = fp16_rne(u24 * 0.01) then qs[32] as bytes.
void qko_fill_q8_0(uint64_t seed, uint64_t block0, uint64_t nblocks, uint8_t* dst) {
    for (uint64_t b = 0; b < nblocks * 8; b++) {
        const uint64_t base = (block0 * 8 + b) * 33;
        BlockQ8_0 blk;
        blk.d = f2h_rne(sm_u24(sm_at(seed, base)) * 0.01f);
        for (int i = 0; i < 32; i++) blk.qs[i] = (int8_t)sm_byte(sm_at(seed, base + 1 + i));
        memcpy(dst + b * sizeof(BlockQ8_0), &blk, sizeof(BlockQ8_0));
    }
}

// N(0,1) activations: Box-Muller in double on output pairs (2i, 2i+1), cast to fp32.
void qko_fill_normal(uint64_t seed, uint64_t n, float* dst) {
    const double two_pi = 6.283185307179586476925286766559;
    for (uint64_t i = 0; i < (n + 1) / 2; i++) {
        const uint64_t r1 = sm_at(seed, 2 * i), r2 = sm_at(seed, 2 * i + 1);
        const double u1 = ((double)(r1 >> 11) + 1.0) * (1.0 / 9007199254740992.0);
        const double u2 = (double)(r2 >> 11) * (1.0 / 9007199254740992.0);
        const double rad = sqrt(-2.0 * log(u1));
        dst[2 * i] = (float)(rad * cos(two_pi * u2));
        if (2 * i + 1 < n) dst[2 * i + 1] = (float)(rad * sin(two_pi * u2));
    }
}

}  // extern "C"
