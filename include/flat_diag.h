/* Measurement aids of the gfx950 backend (no counterpart in the reference): the practical
 * ceilings the rooflines of the attention kernels are read against. Built as a separate shared
 * object (flat_attention_amd/libflat_diag.so) that only bench.py --ceilings and its GPU test
 * load; the attention library (libflat_hip.so) carries none of this.
 *
 * Status codes are the attention library's (flat_hip.h): 0 ok, FA_ERR_UNAVAILABLE (20) for a
 * missing device or an unsupported argument, FA_ERR_UNSUPPORTED_DTYPE (29), FA_ERR_NULL_ARGUMENT
 * (50), FA_ERR_HIP (60). */
#ifndef FLAT_DIAG_H
#define FLAT_DIAG_H
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif

/* Back-to-back v_mfma_f32_32x32x16_bf16 (dtype 2 = bf16) or v_mfma_f32_32x32x2_f32 (dtype 0 =
 * f32) on register operands (random attention-like values, or a constant 0.5 when
 * constant_operands != 0) for ~1.5 s on `device` (1 s untimed, so the clock settles); returns
 * TFLOP/s. Uses its own stream, allocates and frees its own buffer, synchronizes. */
int fad_mfma_ceiling(int32_t device, int32_t dtype, int32_t constant_operands, double* tflops);

/* Streams a 4 GiB buffer with non-temporal 16-byte loads, loads_in_flight (4, 8 or 16) per
 * lane, one 8-wave workgroup per CU; returns TB/s. Own stream and buffers, synchronizes. */
int fad_stream_read(int32_t device, int32_t loads_in_flight, double* tbps);

#ifdef __cplusplus
}
#endif
#endif
