/* include/gpuq.h - C ABI of libgpuq.so, the GGUF quantizer for AMD Instinct MI355X (gfx950).
 *
 * The first twelve entry points are the reference library's own (zephel01/trench-gguf gpuq/gpuq.hip), with the
 * same signatures, ggml type ids, return conventions and gpuq_tables.bin format, so the reference's ctypes callers
 * (tools/requant_experts.py, tools/convert_hf.py, tools/requant_table.py, tools/ldlq.py) load this library
 * unchanged. Each cites the reference function it replaces. The entry points after them are additions.
 *
 * Conventions (as the reference's):
 *   - ggml type ids: Q8_0 8, Q2_K 10, Q3_K 11, Q4_K 12, Q5_K 13, Q6_K 14, IQ2_XXS 16, IQ2_XS 17, IQ3_XXS 18,
 *     IQ1_S 19, IQ4_NL 20, IQ3_S 21, IQ2_S 22, IQ4_XS 23, IQ1_M 29; sources F32 0, F16 1, Q8_0 8, BF16 30, MXFP4 39.
 *   - Also quantized here (the reference leaves them to ggml on the CPU): llama-quantize's fallback types for rows
 *     that are not whole 256-weight super-blocks, Q4_0 2, Q5_0 6, Q5_1 7 (32-weight blocks, with or without an
 *     imatrix) and F16 1 (one value a block, rows of any length from F32 / F16 / BF16 sources; the imatrix ignored),
 *     through gpuq_quantize*, gpuq_requantize* and gpuq_requantize_dev (tools/requant_experts.py:180-192).
 *   - Host entry points take host pointers, are synchronous and return the bytes written, 0 on any error.
 *   - Device entry points (*_dev) take device pointers, enqueue on `stream` (a hipStream_t, NULL = the null
 *     stream) without synchronizing, and return the bytes the launch will write, 0 on error.
 *   - Output is the ggml block layout, byte-identical to ggml_quantize_chunk / to_float for the same tables.
 *   - The library keeps process-global staging buffers and tables: calls are serialized internally; the device is
 *     the one passed to gpuq_init.
 */
#ifndef GPUQ_H
#define GPUQ_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* gpuq/gpuq.hip:2059 gpuq_init. Selects the device and loads the search / dequantizer tables. 0 ok; 1 no such
 * device; 2 cannot open the file; 3 short or malformed record; 4 device allocation failed; 6 a table fails the
 * consistency checks (a point whose key does not map back to it, or a reachable key with no candidate). A file with
 * no records returns 0 (the k-quants, Q8_0 and IQ4 need no tables). A file that carries the stand-in mark (a record
 * of type 0x53594e54, written by this package's table generator, never by ggml's) loads its IQ1/IQ2/IQ3 tables only
 * when the environment sets GPUQ_ALLOW_SYNTHETIC_TABLES=1; otherwise it returns 0 with those types unavailable
 * (gpuq_can_quantize / gpuq_can_dequantize_type report 0), since their grid indices would not be ggml's. A second
 * call replaces the tables for later calls and keeps the earlier ones allocated until the process ends (graphs
 * captured before it go on reading them); it must not overlap calls from other threads. */
int gpuq_init(const char *tables_path, int device);

/* gpuq/gpuq.hip:2082 gpuq_block_bytes: bytes of one block of the type, 0 for an unknown type (F16: 2, a block
 * being one value, as ggml's type size) */
size_t gpuq_block_bytes(int type);

/* gpuq/gpuq.hip:2213 gpuq_can_quantize: 1 when gpuq_quantize* takes the type with (1) or without (0) an imatrix */
int gpuq_can_quantize(int type, int with_imatrix);

/* gpuq/gpuq.hip:2228 gpuq_quantize: nrow x n_per_row f32 (host) -> dst (host), imatrix: n_per_row weights or NULL */
size_t gpuq_quantize(int type, const float *src, void *dst, int64_t nrow, int64_t n_per_row, const float *imatrix);

/* gpuq/gpuq.hip:2219 gpuq_quantize_batch: nmat matrices, matrix m weighted by imatrix row m (nmat x n_per_row) */
size_t gpuq_quantize_batch(int type, const float *src, void *dst, int64_t nmat, int64_t nrow, int64_t n_per_row,
                           const float *imatrix);

/* gpuq/gpuq.hip:2235 gpuq_can_dequantize: 1 when gpuq_requantize* reads this source type */
int gpuq_can_dequantize(int src_type);

/* gpuq/gpuq.hip:2252 gpuq_requantize: source bytes (host, type src) -> decoded on the GPU -> quantized -> dst */
size_t gpuq_requantize(int src_type, const void *raw, int type, void *dst, int64_t nrow, int64_t n_per_row,
                       const float *imatrix);

/* gpuq/gpuq.hip:2239 gpuq_requantize_batch */
size_t gpuq_requantize_batch(int src_type, const void *raw, int type, void *dst, int64_t nmat, int64_t nrow,
                             int64_t n_per_row, const float *imatrix);

/* gpuq/gpuq.hip:2283 gpuq_quantize_dev: nblocks 256-weight super-blocks of d_x -> d_dst, block b weighted by
 * d_qw + ((b % qw_mod) / qw_div) * 256. Takes every 256-block type (the reference: the i-quants and IQ4_XS).
 * d_x and d_qw 16-byte aligned. */
size_t gpuq_quantize_dev(int type, const float *d_x, void *d_dst, int64_t nblocks, const float *d_qw, int64_t qw_mod,
                         int64_t qw_div, void *stream);

/* gpuq/gpuq.hip:2292 gpuq_can_dequantize_type: 1 for the i-quants with a dequantizer grid and IQ4_XS (the
 * reference's set), and the k-quants Q2_K..Q6_K (an addition: the reference reads them back through ggml) */
int gpuq_can_dequantize_type(int type);

/* gpuq/gpuq.hip:2302 gpuq_dequantize_dev: nblocks blocks (device) -> nblocks*256 f32 (device), ggml's to_float.
 * d_out 16-byte aligned, d_q 2-byte aligned (0 returned before any launch otherwise). */
size_t gpuq_dequantize_dev(int type, const void *d_q, float *d_out, int64_t nblocks, void *stream);

/* gpuq/gpuq.hip:2323 gpuq_dequantize_src_dev: n values (n % 32 == 0) of F32/F16/BF16/Q8_0/MXFP4 bytes -> f32.
 * d_out 16-byte aligned; d_raw 16-byte aligned for F32 / F16 / BF16, 2-byte for Q8_0 (0 returned otherwise). */
size_t gpuq_dequantize_src_dev(int src_type, const void *d_raw, float *d_out, int64_t n, void *stream);

/* ---- additions (no counterpart in the reference) ---- */

/* Device-resident requantize: nmat matrices of nrow x n_per_row values stored as src_type (F32, F16, BF16, Q8_0 or
 * MXFP4, decoded in registers inside the quantize kernel) -> d_dst, matrix m weighted by d_imatrix + m*n_per_row (or
 * none). d_raw 16-byte aligned for F32 / F16 / BF16 (2-byte for Q8_0), n_per_row a multiple of 32. For callers that
 * keep the source in HBM (the streaming driver, the benchmark). */
size_t gpuq_requantize_dev(int src_type, const void *d_raw, int type, void *d_dst, int64_t nmat, int64_t nrow,
                           int64_t n_per_row, const float *d_imatrix, void *stream);

/* The LDLQ error-feedback loop on the device, for nmat matrices that share (u_stride = 0) or own (u_stride =
 * ne0*ne0) a factor U: replaces the loop of tools/ldlq.py:391-431 (quantize_matrix_torch), which calls
 * gpuq_quantize_dev / gpuq_dequantize_dev per block and solves / updates in torch. d_wp [nmat][ne1][ne0] f32 in
 * permuted column order (updated in place), d_u [ne0][ne0] f64 row-major upper factor of the permuted inverse
 * Hessian, d_qw [nmat][ne0] f32 importances in permuted order, blk_order (host) the output slot of each permuted
 * 256-column block, d_out [nmat][ne1][ne0/256 blocks]. The f64 solve and update use fixed-order FMA chains (the CPU
 * oracle computes the same ones). Types: the i-quants with a dequantizer grid, IQ4_XS and Q2_K..Q6_K. Asynchronous
 * on `stream` (part of each update runs on an internal stream that is joined back into `stream` before the call
 * returns). Calls share one library scratch buffer; each call's launches wait for the previous call's, on whatever
 * stream that one ran, so calls from several streams are ordered on the device. Refused (returns 0 before any
 * launch) on a stream under capture: graphs use gpuq_ldlq_dev_noalloc. */
size_t gpuq_ldlq_dev(int type, float *d_wp, const double *d_u, int64_t u_stride, const float *d_qw, int64_t nmat,
                     int64_t ne1, int64_t ne0, const int64_t *blk_order, int feedback, void *d_out, void *stream);

/* gpuq_ldlq_dev that allocates nothing. No counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). Same arguments,
 * checks and bytes as gpuq_ldlq_dev; its Es scratch is a static 32 MiB device array of the library (each GPU it runs
 * on holds one until the process ends), every launch goes to `stream`, and it calls no allocator. Limit: with
 * feedback, nmat * ne1 <= 8192 rows; a larger call returns 0 (with a message on stderr) before any launch. Calls on
 * one GPU share the array: calls that overlap on one GPU race. */
size_t gpuq_ldlq_dev_noalloc(int type, float *d_wp, const double *d_u, int64_t u_stride, const float *d_qw,
                             int64_t nmat, int64_t ne1, int64_t ne0, const int64_t *blk_order, int feedback,
                             void *d_out, void *stream);

/* H += X^T X on the device, replacing the float32-GEMM / float64-sum loop of tools/hessian_from_dump.py:73-79:
 * d_X [nrows][ne0] f32, d_H [ne0][ne0] f64 (symmetric, kept symmetric), products exact in f64, sums over the rows in
 * order on the f64 matrix cores. Asynchronous on `stream`. Returns 0; 1 bad arguments (ne0 a multiple of 256, at
 * most 65280); 4 a HIP error. */
int gpuq_hessian_accumulate_dev(const float *d_X, int64_t nrows, int64_t ne0, double *d_H, void *stream);

/* The LDLQ factor built on the device, replacing prepare_hessian / prepare_hessian_torch (tools/ldlq.py:34-68,
 * 275-323), whose factorizations run in numpy or torch: d_H [ne0][ne0] f64 (device, row-major, the sum of x x^T over
 * n inputs; not modified) -> d_U [ne0][ne0] f64 (device, row-major upper factor: U^T U = the inverse of the damped,
 * normalized, block-permuted Hessian, with the reference's dead-column rule and its one retry with 10x more ridge),
 * perm [ne0] (host: the column permutation, whole 256-column blocks; order 0 'seq', 1 'act'), diag_n [ne0] (host,
 * diag(H)/n permuted; may be NULL) and dead [ne0] (host flags, original order; may be NULL). Uses rocSOLVER's potrf /
 * potri (loaded on first use). Returns 0; 1 bad arguments (ne0 a multiple of 256, at most 65280), 2 rocBLAS or
 * rocSOLVER not loadable, 3 not positive definite, 4 a HIP error. Synchronizes `stream`. */
int gpuq_prepare_hessian_dev(const double *d_H, int64_t ne0, double n, double damp, int order, double *d_U,
                             int64_t *perm, double *diag_n, unsigned char *dead, void *stream);

/* The 'schur' importance of each 256-column block of an LDLQ factor, replacing the numpy / torch inverse of
 * tools/ldlq.py:90-93, 424-426 (diag((U_BB^T U_BB)^-1)): d_u [ne0][ne0] f64 upper factor (device) -> d_w [nrep][ne0]
 * f32 (device; the same values in each of the nrep rows, one a matrix that shares U), in a fixed summation order the
 * CPU oracle repeats. Asynchronous on `stream`. Returns 0; 1 bad arguments; 4 a HIP error. */
int gpuq_schur_weights_dev(const double *d_u, int64_t ne0, float *d_w, int64_t nrep, void *stream);

/* The LDLQ loop from host memory, with no framework on the caller's side: the reference's tools/ldlq.py:71-107
 * (quantize_matrix) with the factor of gpuq_prepare_hessian_dev. W [nmat][ne1][ne0] f32 (original column order, not
 * modified), H [ne0][ne0] f64 shared by all matrices (h_stride 0) or one a matrix (h_stride ne0*ne0), n and damp and
 * order as gpuq_prepare_hessian_dev. weights (the reference's `weights`): 0 'imatrix' (imatrix [nmat][ne0]; NULL only
 * for a type that takes none), 1 'diag' (diag(H)/n), 2 'schur' (gpuq_schur_weights_dev); imatrix NULL for 1 and 2.
 * Writes every matrix's GGUF bytes to dst (blocks in their original slots) and returns their count, or 0 on an error.
 * Serializes on an internal lock; synchronous. */
size_t gpuq_ldlq(int type, const float *W, const double *H, int64_t h_stride, double n, double damp, int order,
                 int weights, const float *imatrix, int64_t nmat, int64_t ne1, int64_t ne0, void *dst);

/* Reads and clears the flag the kernels set where the reference would trap (a key with no candidate point: non-
 * finite input or an inconsistent table). Synchronizes the device. */
int gpuq_take_error(void);

#ifdef __cplusplus
}
#endif
#endif
