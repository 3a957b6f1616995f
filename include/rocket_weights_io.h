/*
 * rocket_weights_io.h — a serialised form of the resident int8 / int4 weights (MI355X
 * addition; the reference library keeps packed weights only in live NPU buffer objects and
 * has no file form). A model loader packs each quantised weight once, saves it, and later
 * loads it straight into HBM with no re-pack: the file holds the codes in the device layout
 * (int8 rows [N][K]; int4 nibble-packed [N][K/2], the layout rocket_i4_weights_device
 * documents) and, optionally, the fp32 group scales b_scale[N][K/group].
 *
 * Callers: model loaders for GGUF-style quantised checkpoints (Q8_0 / Q4 blocks mapped onto
 * the group-wise resident entries), and anything that wants to cache packed weights on disk.
 *
 * Layout (little-endian; 64-byte header, then the codes, then the scales):
 *   0  char[4]  "RKTW"           32 u64 code_bytes
 *   4  u32      version (1)      40 u64 scale_bytes (0, or 4 * N * K / group)
 *   8  u32      kind (1 int8,    48 u64 XXH64 (seed 0) of the codes followed by the scales
 *               2 int4 packed)   56 u64 XXH64 (seed 0) of header bytes 0..55
 *   12 u32      flags (bit 0: scales present)
 *   16 u32 N    20 u32 K    24 u32 group (0: per-channel)    28 u32 M it was packed for
 * A reader rejects any other magic, version or kind, a size that disagrees with N, K and
 * group, a short buffer, and either checksum mismatch.
 */
#ifndef ROCKET_WEIGHTS_IO_H
#define ROCKET_WEIGHTS_IO_H

#include <stddef.h>
#include <stdint.h>

#include "rocket_matmul.h"

#ifdef __cplusplus
extern "C" {
#endif

#define ROCKET_WEIGHTS_KIND_INT8 1u
#define ROCKET_WEIGHTS_KIND_INT4 2u

typedef struct rocket_weights_info {
    uint32_t kind, flags, N, K, group, M;
    uint64_t code_bytes, scale_bytes;
} rocket_weights_info;

/* XXH64 (seed 0) of buf[len], the checksum the format uses. */
uint64_t rocket_weights_xxh64(const void *buf, size_t len);

/* Validates a serialised weight (header, sizes, both checksums) and fills *info. Needs no
 * device. Returns 0, or -1 for anything malformed. */
int rocket_weights_info_read(const void *buf, size_t len, rocket_weights_info *info);

/* Bytes the serialised form of w takes (with the N * K/group fp32 scales if with_scales and
 * the weight is group-wise). 0 for a NULL weight. */
size_t rocket_i8_weights_serialized_bytes(const rocket_i8_weights *w, int with_scales);
size_t rocket_i4_weights_serialized_bytes(const rocket_i4_weights *w, int with_scales);

/* Writes w (and b_scale[N][K/group] when non-NULL; group-wise weights only) into buf[cap].
 * Returns the bytes written, or -1 (bad argument, cap too small), ROCKET_E_DEVICE. */
long rocket_i8_weights_serialize(rocket_i8_ctx *ctx, const rocket_i8_weights *w, const float *b_scale,
                                 void *buf, size_t cap);
long rocket_i4_weights_serialize(rocket_i4_ctx *ctx, const rocket_i4_weights *w, const float *b_scale,
                                 void *buf, size_t cap);

/* A new resident weight on ctx from a serialised one (the codes are copied to HBM as they
 * are). When the buffer carries scales and b_scale_out is non-NULL, they are copied there
 * (N * K/group floats). NULL on any validation failure or of the wrong kind. Free with
 * rocket_i{8,4}_weights_free. */
rocket_i8_weights *rocket_i8_weights_deserialize(rocket_i8_ctx *ctx, const void *buf, size_t len,
                                                 float *b_scale_out);
rocket_i4_weights *rocket_i4_weights_deserialize(rocket_i4_ctx *ctx, const void *buf, size_t len,
                                                 float *b_scale_out);

/* The same through a file. save returns 0, -1 (argument / I/O), ROCKET_E_DEVICE. */
int rocket_i8_weights_save(rocket_i8_ctx *ctx, const rocket_i8_weights *w, const float *b_scale,
                           const char *path);
int rocket_i4_weights_save(rocket_i4_ctx *ctx, const rocket_i4_weights *w, const float *b_scale,
                           const char *path);
rocket_i8_weights *rocket_i8_weights_load(rocket_i8_ctx *ctx, const char *path, float *b_scale_out);
rocket_i4_weights *rocket_i4_weights_load(rocket_i4_ctx *ctx, const char *path, float *b_scale_out);

#ifdef __cplusplus
}
#endif
#endif /* ROCKET_WEIGHTS_IO_H */
