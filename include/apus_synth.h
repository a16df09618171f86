/*
 * include/apus_synth.h — deterministic synthetic inputs for the FP8-block
 * MoE hot path (host side, C ABI). The reference has no counterpart: its
 * fixtures come from tests/m3g/gen_golden.py and the splitmix64 streams of
 * tests/m7b/test_gkernels.c:60-73. This generator is the one spec shared by
 * the GPU path (bench, device fill kernels) and the CPU checker (tests), so
 * both sides see identical inputs. Exported by libapus_ghip.so.
 *
 * Draw i of stream s under seed: mix64(key + (i+1)*0x9E3779B97F4A7C15),
 * key = mix64(seed + (s+1)*0x632BE59BD9B4E019), mix64 = splitmix64's
 * finalizer.
 */
#ifndef APUS_SYNTH_H
#define APUS_SYNTH_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

uint64_t apus_synth_mix64(uint64_t z);
uint64_t apus_synth_key(uint64_t seed, uint64_t stream);
uint64_t apus_synth_u64(uint64_t key, uint64_t i);

/* FP8-E4M3 codes uniform over the 254 finite codes (0x7F/0xFF excluded):
 * out[i] = code of draw (offset + i). */
void apus_synth_fp8_codes(uint8_t *out, size_t n, uint64_t seed,
                          uint64_t stream, uint64_t offset);
/* F32 scales log-uniform in [lo, hi] (draws 0..n-1). */
void apus_synth_scales(float *out, size_t n, uint64_t seed, uint64_t stream,
                       float lo, float hi);
/* The 65536-entry bf16 N(0,1) quantile table: bf16(Phi^-1((i+0.5)/65536)). */
void apus_synth_normal_table(uint16_t *tab);
const uint16_t *apus_synth_normal_table_ptr(void);
/* BF16 N(0,1): out[i] = table[draw(offset + i) >> 48]. */
void apus_synth_bf16_normal(uint16_t *out, size_t n, uint64_t seed,
                            uint64_t stream, uint64_t offset);
/* F32 N(0,1), Box-Muller in double over draws 2(offset+i), 2(offset+i)+1. */
void apus_synth_f32_normal(float *out, size_t n, uint64_t seed,
                           uint64_t stream, uint64_t offset);
/* Routing for T tokens: k distinct experts of E per token, Zipf(zipf_s)
 * over ranks (zipf_s <= 0: uniform), ranks -> ids by a seeded permutation;
 * w = softmax over k iid N(0,1) slot logits. idx/w: [T, k]. 0 on success. */
int apus_synth_route(int32_t *idx, float *w, size_t T, int E, int k,
                     double zipf_s, uint64_t seed);
/* Stream id of member j (0 gate codes, 1 gate scales, 2 up codes,
 * 3 up scales, 4 down codes, 5 down scales) of expert e in bank b. */
uint64_t apus_synth_expert_stream(int bank, int expert, int member);

/* Device fills (libapus_ghip.so, asynchronous on `stream`, a hipStream_t):
 * the same bytes as apus_synth_fp8_codes / apus_synth_bf16_normal, written
 * to device memory. 0 on success. */
int apus_synth_fp8_codes_dev(uint8_t *out, size_t n, uint64_t seed,
                             uint64_t stream_id, uint64_t offset, void *stream);
int apus_synth_bf16_normal_dev(uint16_t *out, size_t n, uint64_t seed,
                               uint64_t stream_id, uint64_t offset,
                               void *stream);

#ifdef __cplusplus
}
#endif
#endif /* APUS_SYNTH_H */
