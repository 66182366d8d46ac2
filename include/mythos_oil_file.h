/*
 * mythos_oil_file.h — reading MYTHOS.cpp `.oil` model files into the layouts
 * the gfx950 kernels of libmythos_oil.so consume (libmythos_host.so).
 *
 * Replaces the read side of the reference container, src/oil_format.cpp
 * (OILReader, :287-462; format in include/oil/oil_format.h:14-40) and the
 * codebook deserialisers of src/codebook.cpp:196-212 / :348-364:
 *
 *   header   "OIL1", u32 version, u32 flags, u32 config_size, config bytes
 *   formats  u32 n, then n x {u32 block_id, u8 format, u32 cb_bytes}
 *   tensors  u32 n, then n x {u16 name_len, name, u32 block_start, u32 num_blocks}
 *   blocks   in file order: u32 num_weights, u32 cb_bytes, codebook,
 *            u32 idx_bytes, indices
 *
 * Codebooks: OIL8 = u32 magic 0x4F494C38 + 256 f32; OIL4 = u32 magic
 * 0x4F494C34 + 16 FP16.  A tensor's blocks hold consecutive runs of its
 * row-major weights, each run with its own codebook.
 *
 * Instead of the reference's dequantisation to FP32 (OILReader::read_tensor),
 * a tensor is repacked into the structure-of-arrays layout of the kernels and
 * kept quantised:
 *   OIL4:    packed nibbles [rows][cols/2] (even element in the low nibble)
 *            and FP16 codebooks [rows*cols/B][16]; cb_block = B, the block
 *            length (0: one block for the whole tensor); B must divide cols
 *   OIL8:    indices [rows][cols] and one 256-entry FP32 codebook (every
 *            block of the tensor must carry the same codebook)
 *   TERNARY: 2-bit codes [rows][cols/4], element i in bits 2(i%4) of byte
 *            i/4 (the I2_S layout); codebooks: the 3 FP32 values
 *   FP32:    the floats
 * OIL4 codebook entries are kept as FP16 bits: the kernels decode them
 * exactly (as src/kernel_oil4.cpp:15-29 does); the reference's read_tensor
 * decodes subnormal entries with CodebookOIL4::half_to_float, which differs.
 *
 * Functions return MTH_FILE_OK (0) or a negative code; the message of the
 * last failure of the calling thread is mth_oil_error().  Every offset read
 * from the file is bounds-checked: a truncated or corrupt file is an error,
 * never an out-of-bounds read.
 */
#ifndef MYTHOS_OIL_FILE_H
#define MYTHOS_OIL_FILE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MTH_FILE_OK 0
#define MTH_FILE_EINVAL (-1)       /* bad argument, unknown tensor, size mismatch */
#define MTH_FILE_EFORMAT (-2)      /* not an OIL1 file, truncated or inconsistent */
#define MTH_FILE_EUNSUPPORTED (-3) /* a valid tensor this layout cannot express */
#define MTH_FILE_EDEVICE (-4)      /* HIP error while uploading */

/* .oil format byte of a block (include/oil/types.h:17-24) */
#define MTH_OIL_BINARY 0
#define MTH_OIL_TERNARY 1
#define MTH_OIL_OIL4 2
#define MTH_OIL_OIL8 3
#define MTH_OIL_FP32 5 /* any other byte, as OILReader::read_block treats it */

typedef struct mth_oil_file mth_oil_file;

/* Maps and indexes the file (one pass over the blocks).  OILReader::OILReader */
mth_oil_file* mth_oil_open(const char* path);
void mth_oil_close(mth_oil_file* f);
const char* mth_oil_error(void);

/* OILReader::tensor_names */
int64_t mth_oil_num_tensors(const mth_oil_file* f);
const char* mth_oil_tensor_name(const mth_oil_file* f, int64_t i);

/* Format of the tensor's blocks (all must agree), total weights, block count
 * and the common block length (-1 if the blocks differ in length). */
int mth_oil_tensor_info(const mth_oil_file* f, const char* name, int* format, int64_t* num_weights,
                        int64_t* num_blocks, int64_t* block_weights);

/* Repack into host buffers (sizes in bytes; see the layouts above) as a
 * rows x cols matrix, row = output feature (the kernels' [M][K]).
 * in_major = 0: the file holds the weights row-major as [rows][cols] (the
 *   converter's order, tools/convert.cpp:502-509).
 * in_major = 1: the file holds them as the reference's Linear layer keeps its
 *   weight in memory, input-major: element (m, k) at k*rows + m (Linear::forward
 *   multiplies with scalar_gemm, which reads B[k*N + n], src/transformer.cpp:62-70,
 *   src/kernel_i2s.cpp:91-102); the repack transposes.  An input-major OIL4
 *   tensor needs one codebook for all its blocks.
 * *cb_block receives the OIL4 block length (0 = one codebook). */
int mth_oil_repack(const mth_oil_file* f, const char* name, int64_t rows, int64_t cols, int in_major,
                   void* indices, int64_t indices_bytes, void* codebooks, int64_t codebooks_bytes,
                   int64_t* cb_block);

/* Repack and copy into device buffers on `stream` (hipStream_t); returns when
 * the copies are complete. */
int mth_oil_upload(const mth_oil_file* f, const char* name, int64_t rows, int64_t cols, int in_major,
                   void* d_indices, int64_t indices_bytes, void* d_codebooks, int64_t codebooks_bytes,
                   int64_t* cb_block, void* stream);

#ifdef __cplusplus
}
#endif
#endif
