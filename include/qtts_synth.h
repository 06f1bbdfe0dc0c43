/*
 * qtts_synth.h — seeded synthetic checkpoints for benchmarks and tests.
 *
 * The reference loads real weights from a `.qora-tts` file (src/save.rs:262)
 * that quantizes with quantize_f32_to_q4 (src/gemv.rs:92-130).  No weights
 * ship with the reference, so benchmarks and parity tests run on random-init
 * weights drawn here, in the reference's Q4 layout, from a counter-based
 * generator: every value is a pure function of (seed, stream, index), so any
 * process on any host reproduces the same bytes.
 *
 *   nibbles   uniform on 0..15 (q = nibble - 8 uniform on -8..7)
 *   scales    binary16(|N(0, scale_std)|), rounded once to nearest-even
 *   vectors   N(mean, std) as float32, or rounded to binary16
 */
#ifndef QTTS_SYNTH_H
#define QTTS_SYNTH_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* 64-bit hash of (seed, stream, index) (splitmix64 finaliser, twice). */
uint64_t qtts_synth_u64(uint64_t seed, uint64_t stream, uint64_t index);

/* Fills a Q4 weight [k][n] in the reference layout. */
void qtts_synth_q4(uint64_t seed, uint64_t stream, int32_t k, int32_t n, float scale_std, uint8_t *packed,
                   uint16_t *scales);

/* count float32 draws of N(mean, std) (Box-Muller in double). */
void qtts_synth_normal_f32(uint64_t seed, uint64_t stream, int64_t count, float mean, float std, float *out);

/* count binary16 draws of N(mean, std) (rounded from the float32 draw). */
void qtts_synth_normal_f16(uint64_t seed, uint64_t stream, int64_t count, float mean, float std,
                           uint16_t *out);

/* IEEE-754 binary16 conversions: to-nearest-even including subnormals; the
 * widening conversion is exact (the `half` 2.7.1 crate's from_f32/to_f32). */
uint16_t qtts_f32_to_f16(float x);
float qtts_f16_to_f32(uint16_t h);

/* quantize_f32_to_q4(data, k, n), src/gemv.rs:92-130: per (row, 32-column
 * group) scale = absmax/7 stored as binary16, q = clamp(round(v/scale), -8, 7)
 * with round half away from zero, nibble = q + 8. */
void qtts_quantize_f32_to_q4(const float *data, int32_t k, int32_t n, uint8_t *packed, uint16_t *scales);

/* Reads every 16-byte word of a device buffer once, in one launch, on
 * `stream` (a hipStream_t; null for the default stream): the single-launch
 * time of streaming `bytes` from HBM with nothing else to do, the floor the Q4
 * GEMV timings are compared against.  A grid of a few blocks per CU walks the
 * buffer with several 16-byte loads in flight per thread (the fastest shape
 * measured).  bytes must be a positive multiple of 16 and d_buf 16-byte
 * aligned.  Returns 0, or -1 for bad arguments or a failed launch.  No
 * counterpart in the reference (a measurement aid, like the synthetic weights
 * above). */
int32_t qtts_stream_read_device(const void *d_buf, uint64_t bytes, void *stream);

/* The same with the launch shape given: `blocks` 256-thread blocks, each
 * thread keeping `unroll` (1, 2, 4 or 8) loads in flight per grid-wide
 * stride; blocks == 0 launches one block per 256 words, one word per thread. */
int32_t qtts_stream_read_device_ex(const void *d_buf, uint64_t bytes, int32_t blocks, int32_t unroll, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* QTTS_SYNTH_H */
