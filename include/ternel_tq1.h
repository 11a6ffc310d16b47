/*
 * ternel_tq1.h -- C ABI of the MI355X (gfx950) TQ1_G128 packed-weight engine.
 *
 * Every entry point:
 *   - takes device pointers owned by the caller (nothing is allocated inside),
 *   - is asynchronous on the caller's hipStream_t (passed as void*),
 *   - returns 0 on success, TERNEL_TQ1_EINVAL for a rejected argument, or
 *     TERNEL_TQ1_EHIP when a HIP call failed; ternel_tq1_last_error() then holds
 *     the message (thread-local). Nothing throws across this boundary.
 *
 * Weight layout ("canonical blocks"): a weight of `rows` x `columns` is
 * rows * (columns / 128) consecutive 28-byte TQ1_G128 blocks, row-major
 * (row r, group g at byte offset (r * G + g) * 28), each block being
 *   bytes 0-1   raw little-endian fp16 scale bits,
 *   bytes 2-26  25 code bytes, byte 2+j = sum_{i<5} t[5j+i] * 3^i  (legal 0..242),
 *   byte  27    tail byte     = sum_{i<3} t[125+i] * 3^i           (legal 0..26),
 * with weight (t - 1) * scale. This is exactly the byte stream that
 * src/bonsai_tq1/format.py:66-122 encodes/decodes and that
 * cuda/tq1_g128.cuh:14-18 (block_tq1_g128) declares. `blocks` must be 4-byte
 * aligned. Kernels other than validate/decode assume validated bytes; they stay
 * memory-safe on illegal bytes but their arithmetic is then undefined.
 *
 * Activations x are [M][columns] row-major, outputs y are [M][rows] row-major,
 * both of `dtype` (TERNEL_TQ1_F16 is the graded type; BF16/F32 also accepted by
 * the LUT path), fp32 accumulation throughout.
 */
#ifndef TERNEL_TQ1_H
#define TERNEL_TQ1_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TERNEL_TQ1_OK 0
#define TERNEL_TQ1_EINVAL (-1)
#define TERNEL_TQ1_EHIP (-2)

#define TERNEL_TQ1_F16 0
#define TERNEL_TQ1_BF16 1
#define TERNEL_TQ1_F32 2

/* Message of the last failed call on this thread ("" if none). */
const char *ternel_tq1_last_error(void);

/* Library version string. */
const char *ternel_tq1_version(void);

/*
 * Fail-closed byte scan. Writes counters[0] = regular code bytes > 242 and
 * counters[1] = tail bytes > 26 over nblocks canonical blocks (counters is a
 * device array of two uint64, overwritten). Replaces the validation of
 * src/bonsai_tq1/format.py:104-110 and
 * src/ternel_mlx/packing.py:29-48 (validate_packed_codes); the host wrapper
 * raises FormatError with the reference's message when either is nonzero.
 */
int ternel_tq1_validate(const uint8_t *blocks, int64_t nblocks, uint64_t *counters,
                        void *stream);

/*
 * Bit-exact decode (test/inspection entry; never used on the hot path):
 * scales_out[n*2 + b] = block n byte b, codes_out[n*128 + c] = trit c in {0,1,2}
 * computed as (byte // 3^i) % 3 for every byte value, legal or not. Replaces
 * decode_tq1_blocks(validate=False) of src/bonsai_tq1/format.py:94-122; the
 * validate=True form is ternel_tq1_validate followed by this call.
 */
int ternel_tq1_decode(const uint8_t *blocks, int64_t nblocks, uint8_t *scales_out,
                      uint8_t *codes_out, void *stream);

/*
 * LUT23 product y = x @ W^T for small M (decode GEMV at M=1, small batches).
 * Replaces tq1_matmul of src/ternel_mlx/kernels.py:1215-1271 (and the CUDA
 * launchers launch_tq1_g128_gemv_v1, cuda/tq1_g128_gemv.cu:169-180, and
 * launch_tq1_lut23_smem_streamk, cuda/tq1_lut23_streamk.cu:336-367).
 * batch_tile in {1,2,4} (0 = auto); k_split divides columns/128 (0 = auto).
 * ws: fp32 split-K partials, at least
 * ternel_tq1_matmul_workspace_bytes(M, rows, columns, batch_tile, k_split) bytes
 * (0 when the split resolves to 1; ws may then be NULL).
 */
int ternel_tq1_matmul(const uint8_t *blocks, const void *x, void *y, int64_t M, int64_t rows,
                      int64_t columns, int dtype, int batch_tile, int k_split, void *ws,
                      size_t ws_bytes, void *stream);
size_t ternel_tq1_matmul_workspace_bytes(int64_t M, int64_t rows, int64_t columns,
                                         int batch_tile, int k_split);

/*
 * MFMA product y = x @ W^T (prefill, and small batches through split-K): trits
 * decoded to fp16 (t-1)*scale tiles in LDS, v_mfma_f32_32x32x16_f16, fp32
 * accumulation. fp16 activations only. Replaces tq1_gemm of
 * src/ternel_mlx/kernels.py:1287-1357 (prefill path). k_split divides
 * columns/128 (0 = auto); ws as for ternel_tq1_matmul, sized by
 * ternel_tq1_gemm_workspace_bytes.
 */
int ternel_tq1_gemm(const uint8_t *blocks, const void *x, void *y, int64_t M, int64_t rows,
                    int64_t columns, int dtype, int k_split, void *ws, size_t ws_bytes,
                    void *stream);
size_t ternel_tq1_gemm_workspace_bytes(int64_t M, int64_t rows, int64_t columns, int k_split);

/*
 * Packed embedding gather: out[t][c] = (trit(ids[t], c) - 1) * scale for
 * 0 <= ids[t] < rows, zeros otherwise (any id outside the table). ids are
 * int64. Replaces tq1_get_rows of src/ternel_mlx/kernels.py:1360-1398 and
 * k_get_rows_tq1_g128 of patches/prism-tq1-g128-distribution.patch:132-190.
 */
int ternel_tq1_get_rows(const uint8_t *blocks, int64_t rows, int64_t columns,
                        const int64_t *ids, int64_t n_ids, void *out, int dtype, void *stream);

/*
 * packed_matmul dispatch (src/ternel_mlx/modules.py:425-457): picks the LUT
 * path or the MFMA path and its split from (M, rows, columns) on MI355X
 * measurements. ws sized by ternel_tq1_linear_workspace_bytes.
 */
int ternel_tq1_linear(const uint8_t *blocks, const void *x, void *y, int64_t M, int64_t rows,
                      int64_t columns, int dtype, void *ws, size_t ws_bytes, void *stream);
size_t ternel_tq1_linear_workspace_bytes(int64_t M, int64_t rows, int64_t columns, int dtype);

#ifdef __cplusplus
}
#endif

#endif /* TERNEL_TQ1_H */
