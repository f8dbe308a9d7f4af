// trench-gguf_amd/csrc/hessian.cuh - the LDLQ Hessian preparation on the device (tools/ldlq.py:34-68 of the
// reference): Hp = Hn[perm][:, perm] with zero-energy columns replaced by unit rows, Hn = H / max(n, 1), plus a ridge
// on the diagonal; U = the upper Cholesky factor of Hp^-1. These kernels move the matrix between the steps that
// rocSOLVER's potrf / potri do (its Cholesky factor and the inverse from it, column-major, lower triangle).
#pragma once
#include "frame.cuh"

// d[i] = H[i][i] / nd
__global__ __launch_bounds__(256) void k_hess_diag(const double *__restrict__ H, int64_t ne0, double nd,
                                                   double *__restrict__ d) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < ne0) d[i] = H[i * ne0 + i] / nd;
}

// Hp[i][j] = Hn[perm[i]][perm[j]] (a dead column's row and column zero, its diagonal 1), plus ridge on the diagonal;
// grid (ceil(ne0 / 256), ne0)
__global__ __launch_bounds__(256) void k_hess_perm(const double *__restrict__ H, int64_t ne0, double nd,
                                                   const int64_t *__restrict__ perm, const uint8_t *__restrict__ dead,
                                                   double ridge, double *__restrict__ Hp) {
    const int64_t i = blockIdx.y, j = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (j >= ne0) return;
    const int64_t pi = perm[i], pj = perm[j];
    double v = dead[pi] || dead[pj] ? (pi == pj ? 1.0 : 0.0) : H[pi * ne0 + pj] / nd;
    if (i == j) v += ridge;
    Hp[i * ne0 + j] = v;
}

// A[i][i] += r
__global__ __launch_bounds__(256) void k_diag_add(double *__restrict__ A, int64_t ne0, double r) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < ne0) A[i * ne0 + i] += r;
}

// column-major A (n x n) whose lower triangle holds a symmetric matrix: copy it into the upper triangle;
// grid (ceil(n / 256), n)
__global__ __launch_bounds__(256) void k_sym_from_lower(double *__restrict__ A, int64_t n) {
    const int64_t c = blockIdx.y, r = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (r < c) A[c * n + r] = A[r * n + c];
}

// column-major A: zero the strict upper triangle (after a lower Cholesky factorization, the row-major reading of
// A is then the upper factor U); grid (ceil(n / 256), n)
__global__ __launch_bounds__(256) void k_zero_upper(double *__restrict__ A, int64_t n) {
    const int64_t c = blockIdx.y, r = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (r < c) A[c * n + r] = 0.0;
}

// Wp[row][c] = W[row][perm[c]] for rows [0, rows); grid (ceil(ne0 / 256), <= 65535), rows strided by gridDim.y
__global__ __launch_bounds__(256) void k_gather_cols(const float *__restrict__ W, float *__restrict__ Wp,
                                                     const int64_t *__restrict__ perm, int64_t rows, int64_t ne0) {
    const int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (c >= ne0) return;
    const int64_t pc = perm[c];
    for (int64_t r = blockIdx.y; r < rows; r += gridDim.y) Wp[r * ne0 + c] = W[r * ne0 + pc];
}
