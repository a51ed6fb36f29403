// Host-side launch interface between the C ABI (qk_abi.cpp) and the kernel translation units.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace qk {

constexpr int GEMV_MAX_M = 8;      // tokens per GEMV launch (the ABI splits larger m)
constexpr int GEMV_MAX_CNT = 4;    // matrices per group (qwen_cuda/kernels.cu:403-408)
constexpr int GEMV_ROWS_PER_WG = 64;

// One GEMV launch over a group of weights that share x.  Tiles of 16 rows of all matrices are
// concatenated: matrix i owns tiles [tile0[i], tile0[i+1]).  With glu, the group is the pair
// gate/up and the tiles index gate rows; each wave streams both matrices.
struct GemvParams {
    const uint8_t* w[GEMV_MAX_CNT];
    float* y[GEMV_MAX_CNT];
    int n[GEMV_MAX_CNT];
    int tile0[GEMV_MAX_CNT + 1];
    int cnt;
    int glu;
    const float* x;  // [m][k] fp32, tokens tok0.. of the caller's x
    int ldx;         // elements between consecutive tokens of x (= k)
    int ldy_tok0;    // first token index written (outputs are [m_total][n]; y already offset)
    int k, nsb, m;
    int ks, sb_per;  // split of the super-block columns over gridDim.y
    float* part;     // split-K partials, [ks][ntiles][NA][m][16]
    int* counters;   // one self-resetting arrival counter per 64-row group
};

size_t gemv_lds_bytes(int type, int m, int sb_per);
int launch_gemv(int type, const GemvParams& p, hipStream_t s);

int launch_repack(const uint8_t* src, uint8_t* dst, int type, int k, int n, uint64_t rb, int dir, hipStream_t s);
int launch_dequant(const uint8_t* w, int type, int layout, int k, uint64_t rb, const int32_t* rows, int nrows,
                   float* out, hipStream_t s);
int launch_synth(uint8_t* dst, int type, uint64_t seed, uint64_t block0, uint64_t nblocks, hipStream_t s);

}  // namespace qk
