// trench-gguf_amd/csrc/hessian.cuh - the LDLQ Hessian preparation on the device (tools/ldlq.py:34-68 of the
// reference): Hp = Hn[perm][:, perm] with zero-energy columns replaced by unit rows, Hn = H / max(n, 1), plus a ridge
// on the diagonal; U = the upper Cholesky factor of Hp^-1. These kernels move the matrix between the steps that
// rocSOLVER's potrf / potri do (its Cholesky factor and the inverse from it, column-major, lower triangle).
#pragma once
#include "ldlq.cuh"

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

// H += X^T X (tools/hessian_from_dump.py:73-79 of the reference: the Hessian sum over activation rows), X [nrows][ne0]
// f32 row-major, H [ne0][ne0] f64; every product exact in f64 and each output an fma chain over the rows in order on
// the f64 matrix cores. A workgroup of 4 waves owns a 128 x 128 tile of the lower triangle (grid: ne0/128 squared,
// tiles above the diagonal exit at once); rows run in chunks of 16 staged in LDS as f64 (two buffers, one barrier a
// chunk), the two panels of a chunk being X's columns of the tile's rows and of its columns. k_hess_mirror then copies
// the lower triangle's tiles over the upper ones.
#define XTX_BK 16
#define XTX_LDS_ROW 144
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void k_xtx(
    const float *__restrict__ X, int64_t nrows, int64_t ne0, double *__restrict__ H) {
    if (blockIdx.y < blockIdx.x) return;                  // (uniform: a tile above the diagonal)
    __shared__ __align__(16) double As[2][XTX_BK][XTX_LDS_ROW];
    __shared__ __align__(16) double Bs[2][XTX_BK][XTX_LDS_ROW];
    const int64_t row0 = (int64_t)blockIdx.y * 128, col0 = (int64_t)blockIdx.x * 128;
    const int tid = threadIdx.x, lane = lane_id(), wave = tid >> 6;
    const int wr0 = (wave >> 1) * 64, wc0 = (wave & 1) * 64;
    ldlq_d4 acc[4][4];
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int b = 0; b < 4; ++b) acc[a][b] = ldlq_d4{0.0, 0.0, 0.0, 0.0};
    const int lk = tid >> 4, le = tid & 15;                // loader: chunk row lk, elements le + 16 j
    double av[8], bv[8];
    auto load = [&](int64_t k0) {
        const int64_t k = k0 + lk;
        const bool in = k < nrows;
        const float *xr = X + (in ? k : 0) * ne0;
#pragma unroll
        for (int j = 0; j < 8; ++j) av[j] = in ? (double)xr[row0 + le + 16 * j] : 0.0;
#pragma unroll
        for (int j = 0; j < 8; ++j) bv[j] = in ? (double)xr[col0 + le + 16 * j] : 0.0;
    };
    auto stash = [&](int buf) {
#pragma unroll
        for (int j = 0; j < 8; ++j) As[buf][lk][le + 16 * j] = av[j];
#pragma unroll
        for (int j = 0; j < 8; ++j) Bs[buf][lk][le + 16 * j] = bv[j];
    };
    load(0);
    stash(0);
    __syncthreads();
    int buf = 0;
    for (int64_t k0 = 0; k0 < nrows; k0 += XTX_BK) {
        const bool more = k0 + XTX_BK < nrows;
        if (more) load(k0 + XTX_BK);
#pragma unroll
        for (int ks = 0; ks < XTX_BK; ks += 4) {
            const int kk = ks + lane / 16;
            double a[4], b[4];
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                a[t] = As[buf][kk][wr0 + 16 * t + lane % 16];
                b[t] = Bs[buf][kk][wc0 + 16 * t + lane % 16];
            }
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_amdgcn_mfma_f64_16x16x4f64(a[i], b[j], acc[i][j], 0, 0, 0);
        }
        if (more) stash(buf ^ 1);
        __syncthreads();
        buf ^= 1;
    }
    // output element e of lane l: row 4e + l/16, column l%16 of its 16 x 16 tile
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            double *hr = H + (row0 + wr0 + 16 * i + 4 * e + lane / 16) * ne0 + col0 + wc0 + lane % 16;
#pragma unroll
            for (int j = 0; j < 4; ++j) hr[16 * j] += acc[i][j][e];
        }
}

// H[i][j] = H[j][i] for the tiles above the diagonal (i < j and their 128-tiles differ); grid (ceil(ne0 / 256), ne0)
__global__ __launch_bounds__(256) void k_hess_mirror(double *__restrict__ H, int64_t ne0) {
    const int64_t i = blockIdx.y, j = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (j < ne0 && i / 128 < j / 128) H[i * ne0 + j] = H[j * ne0 + i];
}
