/* chpe_pack.h -- seeded synthetic .chpe archive writer (libchpe_pack.so).
 *
 * The reference ships only offline converters between existing archives
 * (src/weight_archive.zig:516-776: createArchive, convertToDense/RawContiguous/
 * RawFp16Contiguous) and fetches real weights from the network.  This library writes
 * complete archives in the same on-disk format from a deterministic generator, so the
 * engine and the oracle can be run on identical bytes without any download.
 *
 * Generator: element e of tensor `tid` is N(0,1) * 0.02 from Box-Muller over
 * splitmix64(key(seed, tid) + e/2) (e even -> cosine branch, odd -> sine branch),
 * computed in double, rounded to f32 and then to fp16 (the "FP16 weights").  Quantized
 * archives quantize those fp16 values: group-128 absmax scales rounded to fp16,
 * 8 outlier columns per 16-row cell and 64 outlier weights per flat tile stored as fp16
 * with their code set to zero.  Norm gains are 1.0 f32, q/k/v biases N(0,0.02) f32.
 */
#ifndef CHPE_PACK_H
#define CHPE_PACK_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum chpe_pack_kind {
  CHPE_PACK_3B_FP16_RAW = 0, /* raw 16384 B tiles, RAW_FP16 flag (Bf16LayerOffsets map) */
  CHPE_PACK_3B_BF16_RAW = 1, /* raw tiles, bf16 */
  CHPE_PACK_3B_W4 = 2,       /* dense 17408 B cells, 4-bit GROUP128 (qwen3b_tensor_map) */
  CHPE_PACK_3B_W2 = 3,       /* dense cells, 2-bit GROUP128 */
  CHPE_PACK_3B_W4_STD = 4,   /* standard 20480 B records (prefetch label + cell), 4-bit */
  CHPE_PACK_72B_W4 = 5,      /* dense cells, 4-bit flat tiles (qwen72b_tensor_map) */
  CHPE_PACK_72B_W2 = 6       /* dense cells, 2-bit flat tiles */
};

/* Bytes of the archive `kind` (header included). */
uint64_t chpe_pack_size(int kind);

/* Write archive `kind` to `path`.  threads <= 0: all cores.  Returns 0 on success,
 * -1 bad kind, -2 cannot create/size/map the file. */
int chpe_pack_write(const char *path, int kind, uint64_t seed, int threads);

/* n generator values (std * N(0,1), f32, before any fp16 rounding) of tensor `tid`
 * starting at element `first`. */
void chpe_pack_normals(uint64_t seed, uint64_t tid, uint64_t first, uint64_t n, float std_dev,
                       float *out);

/* Quantize one 16-row cell: w is rows x cols f32 row-major; bits 2/4; n_outlier_cols 0 or 8
 * (GROUP128 flag set either way).  Writes the full 17408-byte cell. Returns 0 or -1. */
int chpe_pack_cell16(const float *w, int rows, int cols, int bits, int n_outlier_cols,
                     uint32_t layer, uint8_t *cell);

/* Quantize one flat tile of 32768 weights (bits 2/4, GROUP128) with up to 64 outliers. */
int chpe_pack_flat(const float *w, int bits, int n_outliers, uint32_t layer, uint8_t *cell);

#ifdef __cplusplus
}
#endif
#endif
