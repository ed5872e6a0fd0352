/* midge_hip_synth.h — seeded synthetic inputs generated on the device.
 *
 * No counterpart in the reference's hot path: the nearest is run_bench's
 * fixed synthetic fill (engine/midge.c:698-700). These exist so a benchmark
 * can build a full gpt-oss-120b expert table (36 layers x 128 experts,
 * ~60 GiB) in HBM without a host copy. Every value is a pure function of
 * (key, index), computed with integer arithmetic plus at most one IEEE f32
 * multiply, so a CPU can regenerate any slice bit for bit:
 *   hash(key, i)  = SplitMix64 finaliser of key + (i+1) * 0x9e3779b97f4a7c15
 *   bytes         : byte i = byte (i % 8) of hash(key, i / 8), little endian
 *   f16 scales    : 2^e, e = emin + (hash(key, i) >> 32) % (emax - emin + 1)
 *   int8          : (16-bit field i % 4 of hash(key, i / 4)) % 255 - 127
 *   normal-ish f32: (f32)(sum of the four 16-bit fields of hash(key, i) - 131070) * c
 *                   with c = std / 37837.23 (an Irwin-Hall(4) approximation
 *                   of N(0, std^2)); c is passed as the f32 `c`.
 *   uniform f32   : lo + (f32)(hash(key,i) >> 40) * c  with c = (hi-lo) / 2^24
 * Asynchronous on the library stream; dst is device memory.
 */
#ifndef MIDGE_HIP_SYNTH_H
#define MIDGE_HIP_SYNTH_H
#include <stdint.h>
#include "midge_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

int mh_synth_bytes_dev(void *dst, uint64_t n, uint64_t key);
int mh_synth_scales_dev(uint16_t *dst, uint64_t n, uint64_t key, int emin, int emax);
int mh_synth_i8_dev(int8_t *dst, uint64_t n, uint64_t key);
int mh_synth_normal_dev(float *dst, uint64_t n, uint64_t key, float c);
int mh_synth_uniform_dev(float *dst, uint64_t n, uint64_t key, float lo, float c);

/* Fill a whole expert table: for layer l < n_layers, expert e < n_experts,
 * matrix m < 3 the data blob gets bytes with key k(l,e,m,0), the scales blob
 * f16 scales with key k(l,e,m,1) in [emin, emax], and the bias blob
 * normal-ish floats with key k(l,e,m,2) and factor bias_c, where
 * k(l,e,m,p) = hash(key, ((l * n_experts + e) * 3 + m) * 3 + p).
 * Offsets and strides as mh_moe_layer (expert_dt must be MXFP4 or Q4G32);
 * layer l starts at base + l * n_experts * expert_stride. */
int mh_synth_expert_table_dev(void *base, const mh_moe_layer *shape, int n_layers,
                              uint64_t key, int emin, int emax, float bias_c);

#ifdef __cplusplus
}
#endif
#endif /* MIDGE_HIP_SYNTH_H */
