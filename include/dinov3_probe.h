/* Machine-ceiling probes: a measurement library for bench.py and the tests
 * (dinov3-loom_amd/lib/libdinov3_probe.so, built from
 * csrc/kernels/probe.hip), separate from the forward pass's
 * libdinov3_hrx.so. No reference counterpart. */
#ifndef DINOV3_PROBE_H
#define DINOV3_PROBE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Machine-ceiling probes on `device`, one workgroup of four waves per CU
 * (one wave per SIMD), 256 workgroups, 32x32x16 f16 MFMAs on 8 independent
 * accumulators.
 * results[0] = s_memtime cycles per 8 MFMAs of one wave, results[1] = TFLOP/s
 * over the GPU, results[2] = the clock those two imply (GHz). kind: 0 MFMAs on
 * random operands (param 0), 1 on zeros (param 0), 2 with param VALU FMAs per
 * MFMA (0, 2, 4, 6, 8), 3 with param exp2 per MFMA (1, 2), 4 / 5 / 6 with param
 * 16-byte buffer loads per 8 MFMAs (0, 2, 3, 4, 6) from an 8 KB (L1) / 16 KB
 * (L2) / 512 KB (HBM) footprint per wave, 7 with the MFMAs on param (1, 2, 4,
 * 8) independent accumulators (MFMA j adds into accumulator j % param).
 * Returns 0, 2 for an unsupported (kind, param), 1 on a HIP error. Allocates
 * its own buffers. */
int dhx_probe(int32_t device, int32_t kind, int32_t param, double *results);

#ifdef __cplusplus
}
#endif
#endif
