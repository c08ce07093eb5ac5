/* fa_synth.h — seeded synthetic inputs for the EmbeddingGemma path.
 *
 * No counterpart in the reference: fiber/ai loads real checkpoints
 * (safetensors) and tokenises text. The benchmark configurations instead
 * specify random-init weights (N(0, 0.02) rounded to bf16; norm weights
 * N(0, 0.1)) and token ids drawn uniformly or from a Zipf law. These
 * generators produce them deterministically from (seed, tensor name), so the
 * GPU path and the CPU oracle consume bit-identical inputs without writing
 * gigabyte fixture files. Host-only; no GPU needed.
 *
 * Streams: every tensor name selects an independent stream, split into
 * chunks of 2^20 values that are generated in parallel; the output does not
 * depend on the thread count.
 */
#ifndef FA_SYNTH_H
#define FA_SYNTH_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* N(0, std) in float64 (Box-Muller over xoshiro256**), rounded to float32
 * then to bfloat16 with round-to-nearest-even. */
void fa_synth_normal_bf16(uint64_t seed, const char* name, double std, int64_t n, uint16_t* out);

/* N(0, std) rounded to float32. */
void fa_synth_normal_f32(uint64_t seed, const char* name, double std, int64_t n, float* out);

/* Widen bfloat16 to float32 (exact). */
void fa_bf16_to_f32(const uint16_t* in, int64_t n, float* out);

/* Round float32 to bfloat16, round-to-nearest-even (NaN kept quiet). */
void fa_f32_to_bf16(const float* in, int64_t n, uint16_t* out);

/* Uniform integers in [lo, hi). */
void fa_synth_uniform_i32(uint64_t seed, const char* name, int32_t lo, int32_t hi, int64_t n, int32_t* out);

/* Zipf(s) over ranks 1..n_ranks (P(r) proportional to r^-s), written as
 * rank + offset. */
int fa_synth_zipf_i32(uint64_t seed, const char* name, double s, int32_t n_ranks, int32_t offset, int64_t n,
                      int32_t* out);

/* n rows of d float32 values: N(0, 1) rows scaled to unit L2 norm
 * (normalised in float64, then rounded). */
void fa_synth_unit_rows(uint64_t seed, const char* name, int64_t n, int32_t d, float* out);

#ifdef __cplusplus
}
#endif
#endif
