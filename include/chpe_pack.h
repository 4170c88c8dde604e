/* chpe_pack.h -- seeded synthetic .chpe archive writer (libchpe_pack.so).
 *
 * The reference ships only offline converters between existing archives
 * (src/weight_archive.zig:516-776: createArchive, convertToDense/RawContiguous/
 * RawFp16Contiguous) and fetches real weights from the network.  This library writes
 * complete archives in the same on-disk format from a deterministic generator, so the
 * engine and the oracle can be run on identical bytes without any download.
 *
 * Generator: element e of tensor `tid` is N(0,1) * 0.02 from Box-Muller over
 * splitmix64(key(seed, tid) + e/2) (e even -> cosine branch, odd -> sine branch; u1 and u2
 * are the high and low 24 bits, r = sqrt(-2 ln u1)), computed in single precision from
 * correctly rounded operations only (ln by 2 atanh((m-1)/(m+1)) to t^11 after reducing u1
 * to m in [0.75, 1.5); sin / cos of 2 pi u2 by Taylor polynomials on the nearest quarter
 * turn; pack.cpp), then rounded to fp16 (the "FP16 weights").
 * Quantized archives quantize those fp16 values: group-128 absmax scales rounded to fp16
 * (absmax / 7 for 4-bit, / 2 for 2-bit), q = clamp(rint(w / s)), 8 outlier columns per
 * 16-row cell and 64 outlier weights per flat tile (largest |w|, ties to the lower index)
 * stored as fp16 with their code set to the zero code.  Norm gains are 1.0 f32, q/k/v
 * biases N(0,0.02) f32.
 *
 * Layout where the reference reads past a record (its readers, src/chpe_engine.zig):
 *  - a vector longer than a code area's 4096 floats (the 8192-wide q_proj bias of
 *    Qwen2.5-72B, read by unpackBias :1172-1192 as one array from the code area) continues
 *    through its record's payload (240 floats), the next record's 64-byte header (16
 *    floats) and the next record's code area; those bytes are the next tile's leading codes,
 *    and that tile's outliers are chosen among the weights after them.  Gains of 1.0 that
 *    wide (the 72B norms, read by unpackNorm :1144-1170) hold 1.0 in the code area and a NaN
 *    first in the payload: the reader's non-finite rule sets every gain to 1.0;
 *  - embeddings of archives with D >= 4096 (read as 16-row cells, :1540-1546, whose rows and
 *    group scales run past the cell) are written in the per-tile scale form (quant_bits 0,
 *    no group-128 flag: (nibble - 8) * scale + bias, :1384-1394): the code area holds the
 *    flat tile's 32768 weights quantized with one f32 scale (absmax / 7), and the header
 *    and the payload after its metadata and dims hold 4-bit codes of 1952 more generated
 *    weights, so that every byte a row reaches is a code.
 * Qwen3.5-9B (kind CHPE_PACK_9B_W4) holds the real tensors at the front of each INT8-map
 * span (4-bit flat tiles; the span's other records are zero); its linear-attention small
 * tensors are bf16, 8192 values per record: conv1d [8192][4] N(0,0.02), a_log and dt_bias
 * N(0,0.1), linear / q / k norms 1.0.
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
  CHPE_PACK_72B_W2 = 6,      /* dense cells, 2-bit flat tiles */
  CHPE_PACK_9B_W4 = 7        /* dense cells, 4-bit flat tiles at the INT8 map's indices
                                (qwen35_tensor_map), the real Qwen3.5 shapes */
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

/* Records [first, first + count) of archive `kind` into `out` (count * record bytes, as
 * they lie in the file after the 4096-byte header).  Returns 0, or -1 for a bad kind or
 * range. */
int chpe_pack_records(int kind, uint64_t seed, uint64_t first, uint64_t count, int threads,
                      uint8_t *out);

/* The 4096-byte header of archive `kind` into `out`.  Returns 0 or -1. */
int chpe_pack_header(int kind, uint8_t *out);

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
