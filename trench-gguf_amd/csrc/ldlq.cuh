// trench-gguf_amd/csrc/ldlq.cuh - the LDLQ error-feedback loop on the device (tools/ldlq.py:71-107, 391-431).
//
// For column block k (256 permuted columns, c0 = 256k) of nmat matrices of ne1 rows:
//   1. the quantizer runs on the strided view of block k of every row (frame.cuh) and writes each row's block
//      into its output slot;
//   2. k_ldlq_solve: E = blk - to_float(block bytes) in f32, then Es = E U_BB^-1 by forward substitution in f64:
//      Es[j] = (E[j] - sum_{i<j} Es[i] U[c0+i][c0+j]) / U[c0+j][c0+j], each sum a fused multiply-add chain over i in
//      ascending order (the part over earlier 32-column chunks on the matrix cores);
//   3. k_ldlq_update, an f64 GEMM on the matrix cores: W[r][c] -= (float)(sum_{i<256} Es[r][i] U[c0+i][c]) for the
//      later columns c, each output a fused multiply-add chain over i in ascending order from 0.0.
// The reference leaves the order of those sums to LAPACK / BLAS (numpy's LU solve, torch's solve_triangular and
// GEMM); this library fixes it as above, and its CPU oracle computes the same chains, so the bytes are reproducible
// on any hardware. v_mfma_f64_16x16x4f64 accumulates its four products into each output as four IEEE fused
// multiply-adds in k order (checked bit for bit on gfx950 against a sequential fma chain, subnormal results
// included), so a chain of them over k = 0, 4, ..., 252 is exactly the ascending fma chain; its output layout is
// lane l, element e -> row 4e + l/16, column l%16.
#pragma once
#include "frame.cuh"
#include "dequant.cuh"

#ifndef LDLQ_BK
#define LDLQ_BK 16            // k-chunk of the update GEMM
#endif
#define LDLQ_TM 128           // update tile rows
#define LDLQ_TN 128           // update tile columns

typedef double ldlq_d4 __attribute__((ext_vector_type(4)));

// One wave = 64 rows of one matrix (blockIdx.y); the block's 256 columns in chunks of 32. Chunk c:
//   E = blk - to_float(bytes) (f32, then f64), one lane a row, into LDS;
//   E -= Es[:, 0 .. 32c) U[0 .. 32c, chunk] on the f64 matrix cores (each output an fma chain over ascending k,
//   started from E: the serial loop's order), with Es read back (k-major) from the earlier chunks' stores;
//   the 32 x 32 triangle by forward substitution, one lane a row, U's diagonal block broadcast from LDS.
template <int TYPE>
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(2))) void k_ldlq_solve(const float *__restrict__ W, const uint8_t *__restrict__ q,
                                                   int64_t q_stride, int64_t q_off, const double *__restrict__ U,
                                                   int64_t u_stride, int64_t ne1, int64_t ne0, int64_t c0,
                                                   double *__restrict__ Es, const uint64_t *__restrict__ grid) {
    __shared__ double T[64][33];            // the chunk's 64 rows x 32 columns (33: a row per lane hits distinct banks)
    __shared__ double Ud[32][32];           // U's diagonal block of the chunk
    const int64_t m = blockIdx.y;
    const int lane = lane_id();
    const int64_t row0 = (int64_t)blockIdx.x * 64, row = row0 + lane;
    const bool live = row < ne1;
    const int64_t r = m * ne1 + (live ? row : ne1 - 1);
    const int64_t R = (int64_t)gridDim.y * ne1;            // Es rows (k-major: Es[k * R + r])
    const double *Um = U + m * u_stride;
    const float *wrow = W + r * ne0 + c0;
    const uint8_t *qb = q + r * q_stride + q_off;
    // MFMA operand rows of this lane (rows past the matrix read row ne1 - 1: their results are not stored)
    int64_t arow[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        const int64_t rr = row0 + 16 * t + lane % 16;
        arow[t] = m * ne1 + (rr < ne1 ? rr : ne1 - 1);
    }
    for (int c = 0; c < 8; ++c) {
        const int64_t cc = c0 + 32 * c;                     // the chunk's first column
        {
            float y[32];
            dq_chunk<TYPE>(qb, c, y, grid);
            const float4 *wp = (const float4 *)(wrow + 32 * c);
#pragma unroll
            for (int t = 0; t < 8; ++t) {
                const float4 v = wp[t];
                T[lane][4 * t + 0] = (double)(v.x - y[4 * t + 0]);
                T[lane][4 * t + 1] = (double)(v.y - y[4 * t + 1]);
                T[lane][4 * t + 2] = (double)(v.z - y[4 * t + 2]);
                T[lane][4 * t + 3] = (double)(v.w - y[4 * t + 3]);
            }
        }
        {
            const double *up = Um + (cc + lane / 32) * ne0 + cc + lane % 32;
#pragma unroll
            for (int i = 0; i < 16; ++i, up += 2 * ne0) Ud[lane / 32 + 2 * i][lane % 32] = *up;
        }
        wave_sync();
        if (c > 0) {
            ldlq_d4 acc[4][2];
#pragma unroll
            for (int ti = 0; ti < 4; ++ti)
#pragma unroll
                for (int tj = 0; tj < 2; ++tj)
#pragma unroll
                    for (int e = 0; e < 4; ++e) acc[ti][tj][e] = T[16 * ti + 4 * e + lane / 16][16 * tj + lane % 16];
            // k in steps of 16: the operands of four MFMA k-steps are read together, so one memory latency covers
            // four steps (the MFMAs still run in ascending k)
            for (int k0 = 0; k0 < 32 * c; k0 += 16) {
                double a[4][4], b[4][2];
#pragma unroll
                for (int s = 0; s < 4; ++s) {
                    const int k = k0 + 4 * s + lane / 16;
#pragma unroll
                    for (int ti = 0; ti < 4; ++ti) a[s][ti] = -Es[k * R + arow[ti]];
#pragma unroll
                    for (int tj = 0; tj < 2; ++tj) b[s][tj] = Um[(c0 + k) * ne0 + cc + 16 * tj + lane % 16];
                }
#pragma unroll
                for (int s = 0; s < 4; ++s)
#pragma unroll
                    for (int ti = 0; ti < 4; ++ti)
#pragma unroll
                        for (int tj = 0; tj < 2; ++tj)
                            acc[ti][tj] = __builtin_amdgcn_mfma_f64_16x16x4f64(a[s][ti], b[s][tj], acc[ti][tj], 0, 0, 0);
            }
#pragma unroll
            for (int ti = 0; ti < 4; ++ti)
#pragma unroll
                for (int tj = 0; tj < 2; ++tj)
#pragma unroll
                    for (int e = 0; e < 4; ++e) T[16 * ti + 4 * e + lane / 16][16 * tj + lane % 16] = acc[ti][tj][e];
            wave_sync();
        }
        double x[32];
#pragma unroll
        for (int t = 0; t < 32; ++t) x[t] = T[lane][t];
        // (branch-free, the results stored after: a store inside would split the unrolled rows into blocks whose
        // reordering keeps many of U's values live at once)
#pragma unroll
        for (int i = 0; i < 32; ++i) {
            x[i] = x[i] / Ud[i][i];
#pragma unroll
            for (int t = i + 1; t < 32; ++t) x[t] = fma(-x[i], Ud[i][t], x[t]);
        }
        if (live) {
            double *ep = Es + (int64_t)(32 * c) * R + r;
#pragma unroll
            for (int i = 0; i < 32; ++i, ep += R) *ep = x[i];
        }
        // this chunk's Es (stored by other lanes) is read back as MFMA operands by the later chunks
        __threadfence_block();
        wave_sync();
    }
}

// W[m][row][c] -= (float)(sum_i Es[c0+i][m*ne1+row] U_m[c0+i][c]) for c in [cb, ce) (later columns than block
// c0's: cb >= c0 + 256). Es is k-major (Es[k][row], k < 256). A workgroup of 4 waves owns a 128 x 128 tile (each
// wave 64 x 64: 4 x 4 MFMA tiles of 16 x 16); k runs in chunks of 16 staged in LDS, k-major, two buffers (one barrier
// a chunk). A loader thread moves k row t/16, elements t%16 + 16j: 16 lanes read 128 contiguous bytes and write 16
// consecutive LDS doubles; LDS rows are 144 doubles apart (1152 B = 128 mod 256), so the MFMA operand reads (4 k
// rows x 16 consecutive doubles a wave) and the loader's writes fall in distinct banks.
//
// Tiles are numbered matrix by matrix, and within a matrix in groups of LDLQ_GM row tiles, rows fastest, so that the
// workgroups running together share LDLQ_GM Es panels and as many U panels. The 1-D grid (padded to a multiple of
// 8) is dealt to the 8 XCDs round-robin, so workgroup i takes tile (i % 8) * nper + i / 8: each XCD works through one
// contiguous range of tiles and its L2 holds the panels they share (128 x 256 doubles each, 256 KB).
#define LDLQ_LDS_ROW 144
#define LDLQ_GM 8
DEV bool ldlq_tile(int64_t ntr, int64_t ntc, int64_t nmat, int64_t &m, int64_t &tr, int64_t &tc) {
    const int64_t nt = ntr * ntc * nmat, nper = (nt + 7) / 8;
    const int64_t t = (int64_t)(blockIdx.x % 8) * nper + blockIdx.x / 8;
    if (t >= nt) return false;
    const int64_t per = ntr * ntc, u = t % per;
    m = t / per;
    const int64_t gsz = LDLQ_GM * ntc, g = u / gsz, r0 = g * LDLQ_GM;
    const int64_t gm = ntr - r0 < LDLQ_GM ? ntr - r0 : LDLQ_GM;   // rows of this group
    const int64_t v = u % gsz;
    tr = r0 + v % gm;
    tc = v / gm;
    return true;
}
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void k_ldlq_update(
    float *__restrict__ W, const double *__restrict__ Es, const double *__restrict__ U, int64_t u_stride, int64_t nmat,
    int64_t ne1, int64_t ne0, int64_t c0, int64_t cb, int64_t ce) {
    __shared__ __align__(16) double As[2][LDLQ_BK][LDLQ_LDS_ROW];
    __shared__ __align__(16) double Bs[2][LDLQ_BK][LDLQ_LDS_ROW];
    int64_t m, tr, tc;
    if (!ldlq_tile((ne1 + LDLQ_TM - 1) / LDLQ_TM, (ce - cb + LDLQ_TN - 1) / LDLQ_TN, nmat, m, tr, tc)) return;
    const int64_t R = nmat * ne1;
    const int64_t row0 = tr * LDLQ_TM;
    const int64_t col0 = cb + tc * LDLQ_TN;
    const double *Um = U + m * u_stride;
    const int tid = threadIdx.x, lane = lane_id(), wave = tid >> 6;
    const int wr0 = (wave >> 1) * 64, wc0 = (wave & 1) * 64;   // the wave's 64 x 64 sub-tile
    ldlq_d4 acc[4][4];
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int b = 0; b < 4; ++b) acc[a][b] = ldlq_d4{0.0, 0.0, 0.0, 0.0};
    static_assert(LDLQ_BK * 16 == 256 && LDLQ_TM == 128 && LDLQ_TN == 128, "loader: 16 k rows x 16 lanes, 8 a thread");
    const int lk = tid >> 4, le = tid & 15;
    const double *abase = Es + m * ne1 + row0 + le;          // + k * R + 16 j
    const double *bbase = Um + col0 + le;                     // + (c0 + k) * ne0 + 16 j
    double av[8], bv[8];
    // a tile inside the matrix (the usual case) loads unguarded: no per-element branches
    const bool full = row0 + LDLQ_TM <= ne1 && col0 + LDLQ_TN <= ce;
    auto load = [&](int k0) {
        const double *ap = abase + (int64_t)(k0 + lk) * R;
        const double *bp = bbase + (c0 + k0 + lk) * ne0;
        if (full) {
#pragma unroll
            for (int j = 0; j < 8; ++j) av[j] = ap[16 * j];
#pragma unroll
            for (int j = 0; j < 8; ++j) bv[j] = bp[16 * j];
        } else {
#pragma unroll
            for (int j = 0; j < 8; ++j) av[j] = row0 + le + 16 * j < ne1 ? ap[16 * j] : 0.0;
#pragma unroll
            for (int j = 0; j < 8; ++j) bv[j] = col0 + le + 16 * j < ce ? bp[16 * j] : 0.0;
        }
    };
    auto stash = [&](int buf) {
#pragma unroll
        for (int j = 0; j < 8; ++j) As[buf][lk][le + 16 * j] = av[j];
#pragma unroll
        for (int j = 0; j < 8; ++j) Bs[buf][lk][le + 16 * j] = bv[j];
    };
    float wv[4][4][4];                      // the wave's W values (full tiles: read during the last chunk)
    auto read_w = [&](int i0, int i1) {
#pragma unroll
        for (int i = i0; i < i1; ++i)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float *wr = W + (m * ne1 + row0 + wr0 + 16 * i + 4 * e + lane / 16) * ne0 + col0 + wc0 + lane % 16;
#pragma unroll
                for (int j = 0; j < 4; ++j) wv[i][e][j] = wr[16 * j];
            }
    };
    auto chunk = [&](int buf) {             // this wave's MFMAs over the staged k-chunk
#pragma unroll
        for (int ks = 0; ks < LDLQ_BK; ks += 4) {
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
    };
    load(0);
    stash(0);
    __syncthreads();
    int buf = 0;
    for (int k0 = 0; k0 + LDLQ_BK < QK; k0 += LDLQ_BK) {
        load(k0 + LDLQ_BK);                 // the next chunk's global reads overlap this chunk's MFMAs
        chunk(buf);
        stash(buf ^ 1);                     // (the other buffer was last read before the previous barrier)
        __syncthreads();
        buf ^= 1;
    }
    if (full) read_w(0, 1);                 // half the epilogue's reads overlap the last chunk's MFMAs (all of
    chunk(buf);                             // them would not fit in the registers beside the accumulators)
    if (full) read_w(1, 4);
    // epilogue: every W value of the wave's sub-tile is read before the first store (a store between the reads
    // would make each read wait for the one before it); a full tile runs unguarded, so the stores need no
    // per-element branches (and their waits no conservative counts)
    if (full) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                float *wr = W + (m * ne1 + row0 + wr0 + 16 * i + 4 * e + lane / 16) * ne0 + col0 + wc0 + lane % 16;
#pragma unroll
                for (int j = 0; j < 4; ++j) wr[16 * j] = wv[i][e][j] - (float)acc[i][j][e];
            }
        return;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int64_t row = row0 + wr0 + 16 * i + 4 * e + lane / 16;
            const float *wr = W + (m * ne1 + (row < ne1 ? row : 0)) * ne0;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int64_t col = col0 + wc0 + 16 * j + lane % 16;
                wv[i][e][j] = row < ne1 && col < ce ? wr[col] : 0.f;
            }
        }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int64_t row = row0 + wr0 + 16 * i + 4 * e + lane / 16;
            if (row >= ne1) continue;
            float *wr = W + (m * ne1 + row) * ne0;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int64_t col = col0 + wc0 + 16 * j + lane % 16;
                if (col < ce) wr[col] = wv[i][e][j] - (float)acc[i][j][e];
            }
        }
}

// ------------------------------------------------------------------ the 'schur' importance of a block's columns
// tools/ldlq.py:90-93 (and 424-426): qw = diag((U_BB^T U_BB)^-1) of each 256-column diagonal block U_BB, which the
// reference leaves to LAPACK (np.linalg.inv) or torch. Here the order is fixed: (U_BB^T U_BB)^-1 = X X^T with
// X = U_BB^-1, so qw[i] is the squared norm of X's row i. The row comes from X U_BB = I by substitution along it:
//   x_t = ((t == i ? 1 : 0) - acc_t) / U[t][t] for t = i .. 255, acc_t = sum_{s=i}^{t-1} x_s U[s][t],
// each acc_t an fma chain over s ascending from 0.0 (kept as running sums: after x_s, acc_j = fma(x_s, U[s][j], acc_j)
// for the later columns), and qw[i] = (float)(sum_t x_t^2), an fma chain over t ascending from 0.0.
// One wave a row (grid: 256 rows x the blocks): lane L keeps acc for the block's columns L, L+64, L+128, L+192; row
// t + 1 of U is read while row t is used. Columns at or before t are updated too (their sums are no longer read).
// The result goes to nrep rows of w, ne0 apart (matrices that share U).
DEV double readlane_f64(double v, int lane) {
    const unsigned long long b = (unsigned long long)__double_as_longlong(v);
    const unsigned lo = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)b, lane);
    const unsigned hi = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)(b >> 32), lane);
    return __longlong_as_double((long long)(((unsigned long long)hi << 32) | lo));
}

__global__ __launch_bounds__(64) void k_schur_weights(const double *__restrict__ U, int64_t ne0, float *__restrict__ w,
                                                      int64_t nrep) {
    const int64_t c0 = (int64_t)blockIdx.y * QK;
    const int i = (int)blockIdx.x, lane = lane_id();
    const double *ub = U + c0 * ne0 + c0;          // U_BB[s][t] = ub[s * ne0 + t]
    double acc[4] = {0.0, 0.0, 0.0, 0.0}, u[4], un[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) u[q] = ub[(int64_t)i * ne0 + 64 * q + lane];
    double ws = 0.0;
    for (int t = i; t < QK; ++t) {
        const int tn = t + 1 < QK ? t + 1 : t;
#pragma unroll
        for (int q = 0; q < 4; ++q) un[q] = ub[(int64_t)tn * ne0 + 64 * q + lane];
        const int qt = t >> 6, lt = t & 63;        // column t: lane lt, slot qt
        const double at = readlane_f64(qt == 0 ? acc[0] : qt == 1 ? acc[1] : qt == 2 ? acc[2] : acc[3], lt);
        const double dt = readlane_f64(qt == 0 ? u[0] : qt == 1 ? u[1] : qt == 2 ? u[2] : u[3], lt);
        const double x = ((t == i ? 1.0 : 0.0) - at) / dt;
        ws = fma(x, x, ws);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            acc[q] = fma(x, u[q], acc[q]);
            u[q] = un[q];
        }
    }
    if (lane == 0)
        for (int64_t r = 0; r < nrep; ++r) w[r * ne0 + c0 + i] = (float)ws;
}
