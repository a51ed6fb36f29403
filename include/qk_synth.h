/* qk_synth.h — on-GPU synthetic GGUF block generator used by the benchmark and the large parity
 * tests (no counterpart in the reference: its inputs come from a real GGUF file).
 *
 * Fills `nblocks` GGUF-layout super-blocks (for Q8_0: runs of eight 34-byte blocks, 256 weights)
 * starting at global block index `block0` of the counter-based splitmix64 stream seeded with
 * `seed` (mixing constants of qwen_cpu/qwen.cpp:314-319; output i = mix(seed + (i+1)*0x9e3779b97f4a7c15)):
 *   Q4_K: 142 outputs per block in struct order d, dmin, scales[12], qs[128];
 *         d, dmin = fp16_rne(u24 * 0.01f) with u24 = (r >> 40) * 2^-24; bytes = r >> 56.
 *   Q5_K: 174 outputs per block in struct order d, dmin, scales[12], qh[32], qs[128]; as Q4_K.
 *   Q6_K: 209 outputs per block in struct order ql[128], qh[64], scales[16], d;
 *         scales = (int8)((r % 64) - 32); d = fp16_rne(u24 * 0.005f).
 *   Q8_0: 33 outputs per 34-byte block (block j of run b is stream block 8b + j): d = fp16_rne(u24 *
 *         0.01f), then qs[32] as bytes.
 * Byte-identical to the host generator in the test oracle. */
#ifndef QK_SYNTH_H
#define QK_SYNTH_H

#include <stdint.h>
#include "qk.h"

#ifdef __cplusplus
extern "C" {
#endif

int qk_synth_fill(uint32_t type, uint64_t seed, uint64_t block0, uint64_t nblocks, void* dst, qk_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* QK_SYNTH_H */
