/*
 * ternel_tq1.h -- C ABI of the MI355X (gfx950) TQ1_G128 packed-weight engine.
 *
 * Every entry point:
 *   - takes device pointers owned by the caller (nothing is allocated inside),
 *   - is asynchronous on the caller's hipStream_t (passed as void*),
 *   - returns 0 on success, TERNEL_TQ1_EINVAL for a rejected argument (checked
 *     on the host before anything is launched), or TERNEL_TQ1_EHIP when a HIP
 *     call failed; ternel_tq1_last_error() then holds the message
 *     (thread-local). Nothing throws across this boundary.
 *
 * Canonical blocks: a weight of `rows` x `columns` is rows * G consecutive
 * 28-byte TQ1_G128 blocks (G = columns / 128), row-major (row r, group g at
 * byte offset (r * G + g) * 28), each block being
 *   bytes 0-1   raw little-endian fp16 scale bits,
 *   bytes 2-26  25 code bytes, byte 2+j = sum_{i<5} t[5j+i] * 3^i  (legal 0..242),
 *   byte  27    tail byte     = sum_{i<3} t[125+i] * 3^i           (legal 0..26),
 * with weight (t - 1) * scale -- exactly the byte stream that
 * src/bonsai_tq1/format.py:66-122 encodes/decodes and that
 * cuda/tq1_g128.cuh:14-18 (block_tq1_g128) declares.
 *
 * Packed layout (what the compute kernels read): the same blocks permuted at
 * 4-byte granularity into 64-row tiles -- word j (bytes 4j..4j+3) of block
 * (r, g) is packed[((r / 64) * G + g) * 7 + j][r % 64] (uint32). Rows past
 * `rows` in the last tile are zero. ternel_tq1_packed_words() gives the size;
 * ternel_tq1_interleave / ternel_tq1_deinterleave convert exactly. This is an
 * upload-time permutation of the same bytes, like the code-position-major
 * reorder the reference applies before its fast kernels
 * (src/bonsai_tq1/lut23_reorder.py:126-165, src/ternel_mlx/packing.py:51-83).
 * Compute kernels assume validated bytes; on illegal bytes they stay
 * memory-safe (every byte value's table entries and digits stay in range,
 * checked exhaustively by tests/test_byte_bounds.py) but their arithmetic is
 * undefined.
 *
 * Activations x are [M][columns] row-major, outputs y are [M][rows] row-major,
 * both of `dtype` (TERNEL_TQ1_F16 is the graded type; BF16 also runs the wide
 * MFMA form, F32 the LUT path only), fp32 accumulation throughout.
 *
 * Workspaces: a split workspace starts with a fixed 64 KiB region of
 * arrival counters whose last 32-bit word is the workspace's error word,
 * followed by fp32 partials. The counter region must be zero the first time
 * the workspace is used; every successful call leaves it zero again, so one
 * zero-filled workspace can serve calls of any shape (the reference's
 * stream-K contract, cuda/tq1_lut23_streamk.cu:320-334). Calls sharing one
 * workspace must not overlap in time (one workspace per stream). A kernel
 * whose bounded wait for another workgroup's published partial gives up
 * writes its tile as NaN (it sums nothing), sets the error word
 * (ternel_tq1_workspace_error) and may leave counters set; a later launch of
 * the wide form that finds the word set writes every tile needing the
 * counters as NaN without touching them. The LUT23, direct-form and strip
 * kernels do not read the word, and their results on a workspace whose
 * counters were left set are not defined. Zero the workspace again before
 * any further call on it.
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

/* uint32 words of the packed layout of a rows x columns weight (0 if invalid). */
int64_t ternel_tq1_packed_words(int64_t rows, int64_t columns);

/*
 * Fail-closed byte scan of canonical blocks. Writes counters[0] = regular code
 * bytes > 242 and counters[1] = tail bytes > 26 (counters: device array of two
 * uint64, overwritten). Replaces the validation of
 * src/bonsai_tq1/format.py:104-110 and validate_packed_codes,
 * src/ternel_mlx/packing.py:29-48; the host wrapper raises FormatError with the
 * reference's message when either is nonzero.
 */
int ternel_tq1_validate(const uint8_t *blocks, int64_t nblocks, uint64_t *counters, void *stream);

/*
 * Bit-exact decode of canonical blocks (test/inspection entry, never on the
 * hot path): scales_out[n*2 + b] = block n byte b, codes_out[n*128 + c] = trit
 * c in {0,1,2}, computed as (byte // 3^i) % 3 for every byte value, legal or
 * not. Replaces decode_tq1_blocks(validate=False), src/bonsai_tq1/format.py
 * :94-122; validate=True is ternel_tq1_validate followed by this call.
 */
int ternel_tq1_decode(const uint8_t *blocks, int64_t nblocks, uint8_t *scales_out, uint8_t *codes_out,
                      void *stream);

/*
 * Q2_0/g128 source blocks (34 bytes each, as the GGUF payload stores them)
 * re-encoded as canonical TQ1_G128 blocks on the device: the scale copied,
 * every 2-bit code c in {0,1,2} packed base 3. Replaces decode_q2_blocks +
 * encode_tq1_blocks (src/bonsai_tq1/format.py:51-91, run per tensor by
 * src/bonsai_tq1/pack_model.py:72-80). *bad_codes (device u64, set by the
 * call) receives the number of codes equal to 3, which have no ternary
 * meaning: the reference raises "source contains N non-ternary code(s)" when
 * it is nonzero, and the output blocks are then not to be used. No alignment
 * is required of either buffer.
 */
int ternel_tq1_from_q2(const uint8_t *q2_blocks, int64_t nblocks, uint8_t *blocks, uint64_t *bad_codes,
                       void *stream);

/*
 * Canonical blocks -> packed words and back (exact permutations). Replace the
 * upload-time reorder of the reference (reorder_tensor_arrays /
 * restore_tensor_arrays, src/bonsai_tq1/lut23_reorder.py:126-165; the
 * llama.cpp set_tensor transpose, patches/prism-tq1-g128-distribution.patch
 * :287-340).
 */
int ternel_tq1_interleave(const uint8_t *blocks, int64_t rows, int64_t columns, uint32_t *packed,
                          void *stream);
int ternel_tq1_deinterleave(const uint32_t *packed, int64_t rows, int64_t columns, uint8_t *blocks,
                            void *stream);

/*
 * The reference's tiled pair -> packed words, on the device, with the
 * fail-closed scan folded in: codes is uint8 [rows/tile][G][26][tile], scales
 * uint16 (raw fp16 bits) [rows/tile][G][tile] (src/ternel_mlx/layout.py:100-108),
 * tile divides rows; packed receives ternel_tq1_packed_words(rows, columns)
 * words. counters (two uint64, overwritten) receive the code bytes above 242 in
 * slots 0..24 and above 26 in slot 25, as validate_packed_codes counts them
 * (src/ternel_mlx/packing.py:29-48); the caller rejects the weight when either
 * is nonzero. Replaces unpack_blocks + the upload of
 * src/ternel_mlx/packing.py:67-83.
 */
int ternel_tq1_words_from_tiled(const uint8_t *codes, const uint16_t *scales, int64_t rows, int64_t columns,
                                int64_t tile, uint32_t *packed, uint64_t *counters, void *stream);

/* Packed words -> the tiled pair (the exact inverse); replaces pack_blocks,
 * src/ternel_mlx/packing.py:51-65, for a module's codes/scales state. */
int ternel_tq1_tiled_from_words(const uint32_t *packed, int64_t rows, int64_t columns, int64_t tile, uint8_t *codes,
                                uint16_t *scales, void *stream);

/*
 * LUT23 product y = x @ W^T for small M (decode GEMV at M=1, small batches).
 * Replaces tq1_matmul, src/ternel_mlx/kernels.py:1215-1271 (and the CUDA
 * launchers launch_tq1_g128_gemv_v1, cuda/tq1_g128_gemv.cu:169-180, and
 * launch_tq1_lut23_smem_streamk, cuda/tq1_lut23_streamk.cu:336-367).
 * batch_tile in {1,2,4} (0 = auto); k_split divides columns/128 (0 = auto).
 * A split is reduced inside the same launch, in chunk order (deterministic).
 * With M = 1 and both left automatic, a matrix of at most 40 groups per row
 * whose rows give each CU a strip of at most 96 rows (QKV 8192 x 5120 and
 * gate/up 17408 x 5120 on 256 CUs)
 * runs a form that reduces every row inside one workgroup: no split, no
 * workspace, bit-identical from run to run, equal to the split result to
 * within fp32 reassociation of the per-group terms. A matrix of 41 to 160
 * groups per row whose strips (over CUs / Z) stay within 96 rows, with at
 * most 16368 rows x (Z - 1) (down 17408 -> 5120, O 8192 -> 5120), runs the
 * same form in Z = ceil(groups / 40) K chunks per strip, whose row partials
 * meet in exchange slots in the 64 KiB counter region: its workspace is that
 * region alone, left empty by every call.
 * ws: at least ternel_tq1_matmul_workspace_bytes(...) bytes (0 when the split
 * resolves to 1 or the unsplit form above runs; ws may then be NULL); see the
 * workspace contract above.
 * A split batch whose (row block, batch tile) counters exceed the counter
 * region runs as several launches of as many rows as it holds, in order.
 */
int ternel_tq1_matmul(const uint32_t *packed, const void *x, void *y, int64_t M, int64_t rows,
                      int64_t columns, int dtype, int batch_tile, int k_split, void *ws, size_t ws_bytes,
                      void *stream);
size_t ternel_tq1_matmul_workspace_bytes(int64_t M, int64_t rows, int64_t columns, int batch_tile,
                                         int k_split);

/*
 * ternel_tq1_matmul without a workspace argument, for callers that cannot
 * allocate (code under HIP graph capture, serving loops, harnesses that forbid
 * hipMalloc); no counterpart in the reference. Same arguments, kernels and
 * results as ternel_tq1_matmul; its split-K counters and partials live in a
 * static device array of 64 KiB + 16 MiB that each device the library runs on
 * holds until the process ends. Allocates nothing. A batch whose partials
 * exceed 16 MiB runs as several launches; a requested k_split whose single
 * batch tile needs more (k_split * batch_tile * rows * 4 bytes > 16 MiB) is
 * rejected with TERNEL_TQ1_EINVAL, and an automatic split falls back to none.
 * All calls on one device share the array: calls that overlap in time on a
 * device (two streams, two threads) race. The first call on each device sets
 * the array up (resolves its address, zeroes its counters on `stream`) and
 * must not be under stream capture.
 */
int ternel_tq1_matmul_noalloc(const uint32_t *packed, const void *x, void *y, int64_t M, int64_t rows,
                              int64_t columns, int dtype, int batch_tile, int k_split, void *stream);

/*
 * MFMA product y = x @ W^T, fp16 or bf16 activations, v_mfma_f32_32x32x16_f16
 * with fp32 accumulation, in one of three forms (the reference's GemmConfig forms,
 * src/ternel_mlx/kernels.py:1043-1188, re-chosen for CDNA4):
 *   TERNEL_TQ1_GEMM_TILE   (prefill) 128x128 output tiles, weights decoded to
 *                          fp16 (t-1)*scale tiles in LDS;
 *   TERNEL_TQ1_GEMM_DIRECT (M <= 64) weights decoded straight into MFMA
 *                          operand registers, activations staged in LDS,
 *                          split-K reduced in the same launch in chunk order;
 *   TERNEL_TQ1_GEMM_WIDE   (M > 32, prefill) weights decoded into operand
 *                          registers of 8 waves of 32 rows, 256-row output
 *                          tiles 32, 64, 128 or 256 activation rows wide (the
 *                          narrowest that holds M), both operands DMA'd to
 *                          LDS, K split stream-K over one workgroup per CU
 *                          with an ordered in-launch reduction (k_split must
 *                          be 0/1; columns < 2^22);
 *   TERNEL_TQ1_GEMM_AUTO   DIRECT for M <= 32 (M <= 48 for matrices under
 *                          16 MiB of packed weights); WIDE up to M = 64;
 *                          above, WIDE when it has at least CUs/4 output
 *                          tiles or 15 (tile, group) steps per CU, TILE
 *                          otherwise (and for a fixed k_split > 1).
 * bf16 activations (dtype TERNEL_TQ1_BF16) run the WIDE form only (form AUTO
 * or WIDE, no fixed k_split; size the workspace with form WIDE): a pre-pass
 * scales each row by a power of two into fp16's range and converts it (exact:
 * bf16's 8-bit significand fits fp16's 11 bits; values more than 2^28 below
 * the row's largest lose bits), and the fp32 sums are scaled back and rounded
 * once to bf16; inf and NaN propagate as in the reference. F32 is refused.
 * Replaces tq1_gemm, src/ternel_mlx/kernels.py:1287-1357. x is 16-byte
 * aligned in every form. k_split divides columns/128 (0 = auto). ws: ternel_tq1_gemm_workspace_bytes(...) bytes, the
 * same 64 KiB counter region + fp32 partials contract as ternel_tq1_matmul.
 */
#define TERNEL_TQ1_GEMM_AUTO 0
#define TERNEL_TQ1_GEMM_TILE 1
#define TERNEL_TQ1_GEMM_DIRECT 2
#define TERNEL_TQ1_GEMM_WIDE 3
int ternel_tq1_gemm(const uint32_t *packed, const void *x, void *y, int64_t M, int64_t rows,
                    int64_t columns, int dtype, int form, int k_split, void *ws, size_t ws_bytes,
                    void *stream);
size_t ternel_tq1_gemm_workspace_bytes(int64_t M, int64_t rows, int64_t columns, int form, int k_split);

/*
 * Packed embedding gather: out[t][c] = (trit(ids[t], c) - 1) * scale for
 * 0 <= ids[t] < rows, zeros for any id outside the table. ids are int64.
 * Replaces tq1_get_rows, src/ternel_mlx/kernels.py:1360-1398, and
 * k_get_rows_tq1_g128, patches/prism-tq1-g128-distribution.patch:132-190.
 */
int ternel_tq1_get_rows(const uint32_t *packed, int64_t rows, int64_t columns, const int64_t *ids,
                        int64_t n_ids, void *out, int dtype, void *stream);

/*
 * The same gather over canonical block rows (rows x columns/128 blocks of 28
 * bytes, row-major, as the reference's sidecar stores them,
 * src/bonsai_tq1/format.py:94-122), 4-byte aligned: a token's blocks are one
 * contiguous run, where the packed layout spreads a row over a 256-byte
 * segment per word. Serves tq1_get_rows, src/ternel_mlx/kernels.py:1360-1398,
 * for tables that are only gathered from (an untied embedding).
 */
int ternel_tq1_get_rows_canonical(const uint8_t *blocks, int64_t rows, int64_t columns, const int64_t *ids,
                                  int64_t n_ids, void *out, int dtype, void *stream);

/*
 * packed_matmul dispatch (src/ternel_mlx/modules.py:425-457): the LUT23 path
 * or an MFMA form and its split, from (M, rows, columns, dtype): fp32 always
 * the LUT23 path, bf16 above the LUT23 batches the WIDE form. ws sized by
 * ternel_tq1_linear_workspace_bytes, same contract as ternel_tq1_matmul's.
 */
int ternel_tq1_linear(const uint32_t *packed, const void *x, void *y, int64_t M, int64_t rows,
                      int64_t columns, int dtype, void *ws, size_t ws_bytes, void *stream);
size_t ternel_tq1_linear_workspace_bytes(int64_t M, int64_t rows, int64_t columns, int dtype);

/*
 * The kernel ternel_tq1_linear launches for this shape: TERNEL_TQ1_KERNEL_LUT23
 * or one of the TERNEL_TQ1_GEMM_* forms (never AUTO); negative on a rejected
 * shape or dtype. Host-only, touches no device. The counterpart of the
 * reference's select_gemm / select_lut23 decisions (src/ternel_mlx/modules.py
 * :320-423), exposed so that a dispatch sweep can be replayed through the rule.
 */
#define TERNEL_TQ1_KERNEL_LUT23 100
int ternel_tq1_linear_kernel(int64_t M, int64_t rows, int64_t columns, int dtype);

/*
 * A SwiGLU MLP's gate and up projections as one packed weight, with the
 * elementwise step fused: z[m][r] = SiLU(g) * u, where g and u are rows 2r and
 * 2r + 1 of x @ W^T (the packed weight's rows alternate gate, up -- see
 * ternel_amd.layout.interleave_gate_up) rounded to the activation type as the
 * two unfused layers would return them, and SiLU(g) * u is computed in fp32.
 * z is [M][rows / 2] in the activation type. No counterpart in the reference
 * (its MLP runs gate_proj, up_proj and the activation as separate mlx ops,
 * src/ternel_mlx/packed_model.py:72-92). Batches that ternel_tq1_linear sends
 * to the LUT23 kernel (up to 3 rows, 4 for matrices under 16 MiB, and every
 * fp32 batch) run it with the pair exchange in its epilogue; larger fp16 and
 * bf16 batches run the GEMM into the workspace and one elementwise pass. Workspace
 * from ternel_tq1_swiglu_workspace_bytes, same contract as ternel_tq1_linear's.
 */
int ternel_tq1_swiglu(const uint32_t *packed, const void *x, void *z, int64_t M, int64_t rows, int64_t columns,
                      int dtype, void *ws, size_t ws_bytes, void *stream);
size_t ternel_tq1_swiglu_workspace_bytes(int64_t M, int64_t rows, int64_t columns, int dtype);

/*
 * Reads a workspace's error word (synchronises `stream`): *error = 0, or a
 * bitmask of the kernels whose bounded wait for a published partial gave up
 * (the value 2 = the wide GEMM's stream-K reduction; the LUT23 and
 * direct-form fix-ups never wait). No counterpart in the reference, whose
 * fix-ups (cuda/tq1_lut23_streamk.cu:194-256) spin without a bound; here a
 * wait that cannot complete writes NaN tiles and is reported instead of
 * hanging the device or summing unpublished data.
 */
int ternel_tq1_workspace_error(const void *ws, size_t ws_bytes, int *error, void *stream);

/*
 * Sets how many times such a wait polls before giving up (default 2^22, about
 * 0.2 s); a negative limit makes every wait give up at once, which is how the
 * tests drive the error path from the host. Returns the previous limit. Takes
 * effect for launches issued after the call. No counterpart in the reference.
 */
int ternel_tq1_set_spin_limit(int limit);

#ifdef __cplusplus
}
#endif

#endif /* TERNEL_TQ1_H */
