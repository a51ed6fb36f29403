// Host-side launch interface between the C ABI (qk_abi.cpp) and the kernel translation units.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace qk {

constexpr int GEMV_MAX_M = 8;    // tokens per GEMV launch (the ABI splits larger m)
constexpr int GEMV_MAX_CNT = 4;  // matrices per group (qwen_cuda/kernels.cu:403-408)

// One GEMV launch over a group of weights that share x.  Tiles of 16 rows of all matrices are
// concatenated: matrix i owns tiles [tile0[i], tile0[i+1]).  With glu the group is the pair
// gate/up, the tiles index gate rows and each wave streams both matrices.
//
// Work is the list of units (tile, super-block) in tile-major order, units = ntiles * nsb; wave w of
// `waves` owns units [w*units/waves, (w+1)*units/waves).
struct GemvParams {
    const uint8_t* w[GEMV_MAX_CNT];
    void* y[GEMV_MAX_CNT];  // fp32 [m][n], or the GLU output in yfmt
    int n[GEMV_MAX_CNT];
    int tile0[GEMV_MAX_CNT + 1];
    int cnt;
    int glu;
    const void* x;        // [m][k] in xfmt
    int ldx;              // elements between consecutive tokens of x (= k)
    int xfmt;             // ACT_F32, ACT_F16 or ACT_F16_XPERM (qk_device.h)
    int yfmt;             // GLU output format (ACT_*); other outputs are fp32
    const uint8_t* ximg;  // B-operand image of x for this type (written by launch_gemv's prepass)
    int k, nsb, m;
    int units, waves;
    float* part;     // tile pieces of split tiles: [waves][2][na][mt][16]
    size_t part_cap;  // floats available at part
    int* counters;   // per tile: units accumulated so far; the finishing wave resets it to 0
    // single-token kernel: combine slots, [tile][xnodes][16 rows] of (stream 0, stream 1) fp32 pairs;
    // all-ones bits mark an empty slot, and every combine leaves its slot empty again
    uint64_t* xslot;
    size_t xslot_cap;  // slots available at xslot
    int xnodes;        // slots per row of a tile: slices * (levels of the slice tree + 1)
    // single-token kernel only: units in slice-major order (k cut into `slices` runs of cs
    // super-blocks), tiles of all matrices, LDS offsets of the unit sums, the hand-out counter, the
    // unit table and the rings
    int slices, cs, ntiles;
    int wpg;         // waves per work-group (blockDim.x / 64, here so the prologue needs no other argument)
    int xm;          // super-blocks of x each wave converts (a kernel instantiation: 2, 4, 6 or 12)
    int rq, rrem;    // range split: work-group b owns units [b*rq + min(b, rrem), ...) (no division)
    int dshift;      // about nu >> dshift of a range's units are handed out dynamically (the rest static)
    int lds_part, lds_cnt, lds_tab, lds_ring;
};

// Device memory a matmul call works in beyond its inputs and outputs.  The C ABI keeps one per
// (device, stream), allocated on first use; the allocation-free entry point carves one out of a
// static device array (qk_noalloc.hip).
struct Workspace {
    float* part = nullptr;       // general GEMV: pieces of split tiles
    size_t part_bytes = 0;
    int* counters = nullptr;     // general GEMV: per-tile arrival counters, zero between launches
    int ncounters = 0;
    uint8_t* img = nullptr;      // general GEMV: B-operand image of x
    size_t img_bytes = 0;
    uint8_t* gimg = nullptr;     // GEMM: fp16 image of a token chunk of x
    size_t gimg_bytes = 0;
    uint64_t* xslot = nullptr;   // int8 GEMV: combine slots, zero (empty) between launches
    size_t nxslot = 0;
    float* kpart = nullptr;      // GEMM: split-K partials
    size_t kpart_bytes = 0;
};
// The static workspace of the current device for the allocation-free entry point, set up (symbol
// address, slots emptied and counters cleared by a fill kernel on `s`) on the first call per device.
// Returns 0 or -1 when a HIP call failed.
int noalloc_workspace(hipStream_t s, Workspace* out);
size_t noalloc_scratch_bytes();

// Compute units of the current device (cached per device; 256 when no device is visible, so that
// planning queries also run without a GPU).
int current_cus();
int current_device();  // the current device index (0 when none is visible)
constexpr int MAX_DEVICES = 64;

// Launch plan: waves to use for a GEMV of the given shape (bounded by what is resident at once).
int gemv_plan_waves(int type, int na, int m, int units);
void gemv_set_waves(int waves);  // tuning override of the plan (0 = occupancy-derived)
void gemv_set_fused(bool on);    // m == 1 through the single-token kernel (default on)
void gemv_set_wpg(int w);        // single-token kernel: cap on waves per work-group (0 = LDS-limited)
void gemv_set_img_kib(int kib);  // int8 kernel: activation image per range before more K-slices (0 = 32)
void gemv_set_dshift(int sh);    // int8 kernel: about nu >> sh of a range's units handed out dynamically
void gemv_set_min_waves(int w);  // int8 kernel at m >= 2: fewest waves per work-group (else the general kernel)
void gemv_set_max_slots(int t);  // int8 GEMV: the most token slots per launch (4 or 8)
// What a GEMV launch runs (the plan query of the C ABI, qk_gemv_plan).
enum { GEMV_KERNEL_INT8 = 1, GEMV_KERNEL_GENERAL = 2, GEMV_KERNEL_F32 = 3, GEMV_KERNEL_GEMM = 4 };
struct GemvPlan {
    int kernel, work_groups, waves_per_group, ring_depth, slices, token_slots, lds_bytes;
};
// Runs the GEMV of p (the general kernel converts x into its image at p.ximg first).  info != nullptr:
// fills the plan and launches nothing.  Returns 0, 1 when no kernel has a plan for the shape, -1 when a
// launch failed.
int launch_gemv(int type, const GemvParams& p, hipStream_t s, GemvPlan* info = nullptr);
size_t gemv_part_floats(int waves, int na, int m);
size_t gemv_image_bytes(int type, int m, int nsb);  // workspace bytes of the B-operand image

// Prefill GEMM (m >= 5 through qk_matmul): the LDS-dequant MFMA GEMM on fp16 x [m][k] (fp32 x is first
// rounded into ximg, gemm_image_bytes(m, k) workspace bytes; fp16 x, plain or xperm, is read where it
// lies).  y is fp32 [m][n].
constexpr int GEMM_BM = 128;  // tokens per work-group
size_t gemm_image_bytes(int m, int k);
// part: part_cap floats of split-K partials ([parts][m][n]; the plan splits K only where they fit).
// x in xfmt: ACT_F32 (rounded to fp16 by k_gemm_cvt_x), ACT_F16 or ACT_F16_XPERM (k % 1024 == 0);
// any other format returns -1.
int launch_gemm(int type, const uint8_t* w, int k, int n, const void* x, int xfmt, int m, uint8_t* ximg, float* y,
                float* part, size_t part_cap, hipStream_t s);
// cnt (1..4) matrices of one type and k sharing x in one launch: ws[i] with ns[i] rows into fp32
// ys[i][m][ns[i]] (split-K partials of all of them must fit part; the planner splits K only as far).
int launch_gemm_group(int type, const uint8_t* const* ws, const int* ns, float* const* ys, int cnt, int k, const void* x,
                      int xfmt, int m, uint8_t* ximg, float* part, size_t part_cap, hipStream_t s);
// The gate/up pair wg / wu (same type and shape) in one launch, y = silu(gate x) (up x) in yfmt (ACT_F32,
// ACT_F16 or ACT_F16_XPERM, n % 1024 == 0 for the last): the partials of both, [2][parts][m][n], go to
// part (at least 2 m n floats), then k_glu_sum adds the parts and stores.  -1 when part is too small.
int launch_gemm_glu(int type, const uint8_t* wg, const uint8_t* wu, int k, int n, const void* x, int xfmt, int m,
                    uint8_t* ximg, void* y, int yfmt, float* part, size_t part_cap, hipStream_t s);
void gemm_set_map(int map);  // tuning: 1 = one token block per XCD (default), 0 = a unit's token blocks on one XCD
bool gemm_set_pairs(int p);  // tuning override of the tile pairs per work-group (0 = planned)
bool gemm_set_ksplit(int ks);  // tuning override of the K-parts (0 = planned, 1..16)

// F32 weights, row-major [n][k] (GGUF layout): y[m][n] = x[m][k] W^T, fp32 accumulate, any m; x in
// xfmt (ACT_*).
int launch_f32(const float* w, int k, int n, const void* x, int xfmt, int m, float* y, hipStream_t s);

int launch_repack(const uint8_t* src, uint8_t* dst, int type, int k, int n, uint64_t rb, int dir, hipStream_t s);
int launch_dequant(const uint8_t* w, int type, int layout, int k, int n, uint64_t rb, const int32_t* rows, int nrows,
                   float* out, hipStream_t s);
int launch_embed(const uint8_t* w, int type, int layout, int k, int n, uint64_t rb, const int32_t* tokens,
                 const uint8_t* mask, const float* embd, int m, float* x, hipStream_t s);
int launch_synth(uint8_t* dst, int type, uint64_t seed, uint64_t block0, uint64_t nblocks, hipStream_t s);

}  // namespace qk
