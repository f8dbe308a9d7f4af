/* oracle/gq_oracle.h - CPU oracle for the GGUF quantizer path.
 *
 * TEST INFRASTRUCTURE ONLY. This library restates, on the CPU and in plain C, the arithmetic of ggml's
 * ggml_quantize_chunk / to_float for the types the GPU library serves, following the reference implementation
 * gpuq/gpuq.hip (which restates ggml-quants.c). Only tests/, __graft_entry__.smoke() and bench.py's CPU-baseline leg
 * may load it, and only to check results or as the timed CPU baseline; the product library never links it.
 *
 * Built with gcc -O2 -ffp-contract=off (no -march=native): no FMA contraction, SSE scalar fp32 with IEEE division and
 * square root and no flush-to-zero, the arithmetic of a GGML_NATIVE=OFF libggml-base.
 */
#ifndef GQ_ORACLE_H
#define GQ_ORACLE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml type ids (gpuq/gpuq.hip:54-55, 2106) */
enum {
    GQO_F32 = 0, GQO_F16 = 1, GQO_Q4_0 = 2, GQO_Q5_0 = 6, GQO_Q5_1 = 7, GQO_Q8_0 = 8, GQO_Q2_K = 10, GQO_Q3_K = 11, GQO_Q4_K = 12, GQO_Q5_K = 13,
    GQO_Q6_K = 14, GQO_IQ2_XXS = 16, GQO_IQ2_XS = 17, GQO_IQ3_XXS = 18, GQO_IQ1_S = 19, GQO_IQ4_NL = 20,
    GQO_IQ3_S = 21, GQO_IQ2_S = 22, GQO_IQ4_XS = 23, GQO_IQ1_M = 29, GQO_BF16 = 30, GQO_MXFP4 = 39
};

/* search/dequant tables in the gpuq_tables.bin layout (gpuq/gpuq_tables.c:5-8); 0 on success */
int gqo_load_tables(const char *path);
int gqo_have_tables(int type);

size_t gqo_block_bytes(int type);
int gqo_block_len(int type);

/* ggml_quantize_chunk(type, src, dst, start, nrows, n_per_row, imatrix): start is an element offset that is a
 * multiple of n_per_row; imatrix holds n_per_row weights or is NULL. Returns the bytes written, 0 on error. */
size_t gqo_quantize_chunk(int type, const float *src, void *dst, int64_t start, int64_t nrows, int64_t n_per_row,
                         const float *imatrix);

/* ggml's to_float of a quantized type (IQ types, IQ4_XS, Q8_0): n values */
size_t gqo_dequantize(int type, const void *src, float *dst, int64_t n);

/* source decode (F32 / F16 / BF16 / Q8_0 / MXFP4 bytes -> f32): n values, a multiple of 32 */
size_t gqo_decode_src(int src_type, const void *raw, float *dst, int64_t n);
size_t gqo_src_bytes(int src_type, int64_t n);

/* scalar helpers, exported for the exhaustive tests */
uint16_t gqo_fp32_to_fp16(float f);
float gqo_fp16_to_fp32(uint16_t h);
int gqo_nearest_int(float f);
void gqo_fp32_to_fp16_range(uint32_t first_bits, uint32_t count, uint16_t *out);
void gqo_fp16_to_fp32_all(float *out /* 65536 */);

/* The CPU baseline: nmat matrices of nrow x n_per_row in source encoding src_type, decoded and quantized in units
 * of unit_rows rows (one single-threaded quantize call a unit) on nthreads threads. imatrix: nmat x n_per_row or
 * NULL. Returns the bytes written. */
size_t gqo_requantize_batch_mt(int src_type, const void *raw, int type, void *dst, int64_t nmat, int64_t nrow,
                               int64_t n_per_row, const float *imatrix, int64_t unit_rows, int nthreads);

/* The LDLQ error-feedback loop (tools/ldlq.py:71-107 with a fixed summation order, see gq_oracle.c) over nmat
 * matrices that share U: Wp [nmat][ne1][ne0] f32 in permuted column order (updated in place), U [ne0][ne0] f64 row
 * major (upper triangle read), qw [nmat][ne0] f32 importance in permuted order, blk_order [ne0/256] the output slot
 * of permuted block k, out [nmat][ne1][nblk*block_bytes]. Returns the bytes written. */
size_t gqo_ldlq(int type, float *Wp, const double *U, const float *qw, int64_t nmat, int64_t ne1, int64_t ne0,
                const int64_t *blk_order, int feedback, void *out);

/* The 'schur' importance (tools/ldlq.py:90-93, diag((U_BB^T U_BB)^-1) of each 256-column block of U [ne0][ne0] f64
 * row major, upper triangle read) in a fixed summation order, see gq_oracle.c: w [ne0] f32. */
void gqo_schur_weights(const double *U, int64_t ne0, float *w);

/* op counter (built with -DGQO_COUNT_OPS only; 0 otherwise) */
uint64_t gqo_ops_read_reset(void);

/* path counters, read and reset (all threads): cases of ggml's algorithm that the GPU treats apart, so that a test
 * can show its inputs reach them. NB8_SEARCHES / NB8_TIES: 8-value neighbour searches (iq2_find_best_neighbour), and
 * those whose least distance is shared by two or more candidates (the first wins; the GPU's filtered search cannot
 * decide them and runs the exact search). IQ2XXS_NEGCHAIN: IQ2_XXS sub-blocks whose acceptance chain ends at a
 * scale that is not positive (the final pass is skipped and the accepted trial's points are kept). NB1_NEGATIVE:
 * IQ1 neighbour searches (iq1_find_best_neighbour2) whose chosen distance is negative (negative importances).
 * IQ2X16_NEGCHAIN: IQ2_XS / IQ2_S sub-blocks whose acceptance chain ends at a scale that is not positive. */
enum { GQO_STAT_NB8_SEARCHES, GQO_STAT_NB8_TIES, GQO_STAT_IQ2XXS_NEGCHAIN, GQO_STAT_NB1_NEGATIVE,
       GQO_STAT_IQ2X16_NEGCHAIN, GQO_NSTAT };
uint64_t gqo_stat_read_reset(int which);

#ifdef __cplusplus
}
#endif
#endif
