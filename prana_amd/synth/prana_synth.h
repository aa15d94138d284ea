/*
 * prana_synth.h — fixture encoders for synthetic models (libprana_synth.so).
 *
 * Test and benchmark plumbing, not part of the drop-in boundary: the product
 * library (libprana_hip.so, include/prana_hip.h) only uploads tensor bytes.
 * Block layouts are ggml's; Q4_K/Q6_K follow the reference's converter
 * (scripts/convert-to-gguf.py:29-89). Host code only, no GPU.
 *
 * Every function returns 0 on success or a negative code, with the message in
 * prana_synth_last_error() (thread-local).
 */
#ifndef PRANA_SYNTH_H
#define PRANA_SYNTH_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

const char *prana_synth_last_error(void);
/* Encode a rows x cols f32 tensor into ggml block bytes of ggml_type. */
int prana_quantize_tensor(int ggml_type, const float *src, size_t rows, size_t cols, void *out, size_t nbytes);
/* Seeded N(0, sigma) values (xorshift64* streams + Box-Muller), n floats. */
int prana_synth_normal(uint64_t seed, float sigma, float *out, size_t n);
/* prana_synth_normal values for a rows x cols tensor, encoded straight into
 * ggml bytes (no f32 copy of the whole tensor is materialised). */
int prana_synth_tensor(int ggml_type, size_t rows, size_t cols, uint64_t seed, float sigma, void *out, size_t nbytes);

#ifdef __cplusplus
}
#endif
#endif /* PRANA_SYNTH_H */
