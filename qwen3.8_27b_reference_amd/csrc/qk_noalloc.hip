// Static workspace of the allocation-free matmul entry point (qk_matmul_noalloc in include/qk.h).
//
// Callers that cannot allocate device memory on their call path (code under HIP graph capture, tight
// serving loops, harnesses that forbid hipMalloc) get their workspace from one file-scope device array
// instead of the per-stream buffers the other entry points allocate on first use.  Every GPU the
// library runs on holds its own copy of the array, at its own address, until the process ends.  The
// address is looked up once per device with hipGetSymbolAddress (the array's name in host code is only
// a host-side stand-in) and that pointer is what the kernels receive.  All calls on one GPU share the
// array, so calls that overlap on one GPU race; the array keeps the last call's contents.
#include <hip/hip_runtime.h>

#include <mutex>

#include "qk_internal.h"

namespace qk {
namespace {

// Carve-up of the array (byte offsets, each a multiple of 256).
constexpr size_t XSLOT_BYTES = 32ull << 20;     // 4 Mi combine slots of the int8 GEMV
constexpr size_t COUNTER_BYTES = 256ull << 10;  // 64 Ki tile counters of the general GEMV
constexpr size_t PART_BYTES = 4ull << 20;       // split-tile pieces of the general GEMV
constexpr size_t IMG_BYTES = 4ull << 20;        // x image of the general GEMV
constexpr size_t GIMG_BYTES = 16ull << 20;      // fp16 x image of a GEMM token chunk
constexpr size_t KPART_BYTES = 16ull << 20;     // GEMM split-K partials
constexpr size_t OFF_XSLOT = 0;
constexpr size_t OFF_COUNTERS = OFF_XSLOT + XSLOT_BYTES;
constexpr size_t OFF_PART = OFF_COUNTERS + COUNTER_BYTES;
constexpr size_t OFF_IMG = OFF_PART + PART_BYTES;
constexpr size_t OFF_GIMG = OFF_IMG + IMG_BYTES;
constexpr size_t OFF_KPART = OFF_GIMG + GIMG_BYTES;
constexpr size_t SCRATCH_BYTES = OFF_KPART + KPART_BYTES;  // 72.25 MiB
static_assert(OFF_COUNTERS % 256 == 0 && OFF_PART % 256 == 0 && OFF_IMG % 256 == 0 && OFF_GIMG % 256 == 0 &&
                  OFF_KPART % 256 == 0,
              "256-byte aligned pieces");

// Static storage is zero-initialised, and zero is the state every launch leaves the combine slots
// (empty) and the tile counters in, so the array needs no set-up kernel: a first call may come under
// graph capture and record nothing but its own kernels.
static __device__ __align__(256) uint8_t scratch[SCRATCH_BYTES];

std::mutex g_mu;
uint8_t* g_ptr[MAX_DEVICES];  // device address of `scratch` on each device, once looked up

}  // namespace

size_t noalloc_scratch_bytes() { return SCRATCH_BYTES; }

int noalloc_workspace(hipStream_t s, Workspace* out) {
    (void)s;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEVICES) return -1;
    uint8_t* base = nullptr;
    {
        std::lock_guard<std::mutex> lock(g_mu);
        if (!g_ptr[dev]) {
            // first use on this device (which is current): its copy's address
            void* p = nullptr;
            if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return -1;
            g_ptr[dev] = (uint8_t*)p;
        }
        base = g_ptr[dev];
    }
    Workspace w;
    w.xslot = (uint64_t*)(base + OFF_XSLOT);
    w.nxslot = XSLOT_BYTES / sizeof(uint64_t);
    w.counters = (int*)(base + OFF_COUNTERS);
    w.ncounters = (int)(COUNTER_BYTES / sizeof(int));
    w.part = (float*)(base + OFF_PART);
    w.part_bytes = PART_BYTES;
    w.img = base + OFF_IMG;
    w.img_bytes = IMG_BYTES;
    w.gimg = base + OFF_GIMG;
    w.gimg_bytes = GIMG_BYTES;
    w.kpart = (float*)(base + OFF_KPART);
    w.kpart_bytes = KPART_BYTES;
    *out = w;
    return 0;
}

}  // namespace qk
