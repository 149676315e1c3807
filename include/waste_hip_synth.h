/* SPDX-License-Identifier: Apache-2.0 */
/*
 * waste_hip_synth.h — seeded synthetic MoE layers in WARP's container
 * format, for tests and benchmarks.
 *
 * No counterpart in the engine's kernel interface: this is the device-side
 * equivalent of the reference's converter path for expert weights
 * (tools/convert.py:745-851 residual k-means codebooks and row-scaled VQ
 * encode; src/vq.c:50-107 nearest-centroid assignment; tools/convert.py:
 * 942-977 record layout), run on generated weights instead of a
 * checkpoint, because a DeepSeek-V3-sized layer holds 11.3 G weights.
 *
 * Built into libwaste_hip_synth.so, not into the product library: the
 * engine never calls these.
 */
#ifndef WASTE_HIP_SYNTH_H
#define WASTE_HIP_SYNTH_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Bytes of one expert record for a layer of this shape (4 KiB padded). */
size_t waste_hip_record_bytes(int hidden, int moe_inter);

/* Nine fp16 books [kind gate|up|down][stage 0..2][256][8]: residual k-means
 * per kind on row-absmax-normalised Gaussian rows of that kind's width,
 * seeded.  Host only. */
int waste_hip_synth_codebooks(uint64_t seed, int hidden, int moe_inter,
                              uint16_t *books_f16);

/* Records for experts [e0, e0 + n) of `layer`: each matrix's weights are
 * N(0, std) from a counter-based generator keyed by (seed, expert, kind,
 * row, column), scaled per row by max|w| (clamped to 1e-8, stored as f16),
 * and encoded stage by stage to the nearest entry (squared L2, first
 * minimum) of the books as the engine decodes them.  Written to device
 * memory dst, n * rec_bytes.  The header's crc32 is left 0.  raw, when
 * not NULL, receives expert e0's normalised gate rows (fp32 [I][H]). */
int waste_hip_synth_records(uint64_t seed, int layer, int hidden,
                            int moe_inter, int cb_base,
                            const uint16_t *books_f16, int e0, int n,
                            void *dst, float std, float *raw, void *stream);

#ifdef __cplusplus
}
#endif
#endif
