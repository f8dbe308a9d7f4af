// trench-gguf_amd/csrc/dequant.cuh - ggml's to_float of the i-quants and IQ4_XS, and the source decoder.
//
// Semantics: dequantize_row_iq* (gpuq/gpuq.hip:1850-2021): only products of small integers, fp16 scales and powers
// of two, in ggml's operand order, so fp32 reproduces ggml bit for bit. One thread produces one 32-value chunk
// (8 threads a super-block) with 16-byte stores; the dequantizer grid (uint64 points) is read through the cache.
#pragma once
#include "common.cuh"

DEV uint32_t ksigns7(uint32_t k) { return k | ((uint32_t)(__popc(k) & 1) << 7); }
DEV float sgnb(uint32_t s, int j) { return (s >> j) & 1 ? -1.f : 1.f; }
DEV uint32_t rd8(const uint8_t *p) { return *p; }
DEV uint32_t rd16(const uint8_t *p) { return (uint32_t)*(const uint16_t *)p; }     // 2-byte aligned fields
DEV uint32_t rd32u(const uint8_t *p) { return rd16(p) | (rd16(p + 2) << 16); }     // 2-byte aligned dword
DEV uint32_t gbyte(uint64_t pt, int j) { return (uint32_t)(pt >> (8 * j)) & 0xffu; }

__constant__ int8_t k_iq4nl_i8[16] = {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113};

template <int TYPE> DEV void dq_chunk(const uint8_t *x, int ib, float (&y)[32], const uint64_t *grid) {
    if (TYPE == T_IQ2_XXS) {
        const float d = h2f(rd16(x));
        const uint32_t a0 = rd32u(x + 2 + 8 * ib), a1 = rd32u(x + 6 + 8 * ib);
        const float db = d * (0.5f + (a1 >> 28)) * 0.25f;
#pragma unroll
        for (int l = 0; l < 4; ++l) {
            const uint64_t pt = grid[(a0 >> (8 * l)) & 255];
            const uint32_t s = ksigns7((a1 >> (7 * l)) & 127);
#pragma unroll
            for (int j = 0; j < 8; ++j) y[8 * l + j] = db * gbyte(pt, j) * sgnb(s, j);
        }
    } else if (TYPE == T_IQ2_XS) {
        const float d = h2f(rd16(x));
        const uint32_t sc = rd8(x + 66 + ib);
        const float db0 = d * (0.5f + (sc & 0xf)) * 0.25f;
        const float db1 = d * (0.5f + (sc >> 4)) * 0.25f;
#pragma unroll
        for (int l = 0; l < 4; ++l) {
            const uint32_t q = rd16(x + 2 + 2 * (4 * ib + l));
            const uint64_t pt = grid[q & 511];
            const uint32_t s = ksigns7(q >> 9);
#pragma unroll
            for (int j = 0; j < 8; ++j) y[8 * l + j] = (l < 2 ? db0 : db1) * gbyte(pt, j) * sgnb(s, j);
        }
    } else if (TYPE == T_IQ2_S) {
        const float d = h2f(rd16(x));
        const uint32_t sc = rd8(x + 74 + ib), qh = rd8(x + 66 + ib);
        const float db0 = d * (0.5f + (sc & 0xf)) * 0.25f;
        const float db1 = d * (0.5f + (sc >> 4)) * 0.25f;
#pragma unroll
        for (int l = 0; l < 4; ++l) {
            const uint32_t gi = rd8(x + 2 + 4 * ib + l) | ((qh << (8 - 2 * l)) & 0x300);
            const uint32_t s = rd8(x + 2 + 32 + 4 * ib + l);
            const uint64_t pt = grid[gi];
#pragma unroll
            for (int j = 0; j < 8; ++j) y[8 * l + j] = (l < 2 ? db0 : db1) * gbyte(pt, j) * sgnb(s, j);
        }
    } else if (TYPE == T_IQ3_XXS) {
        const float d = h2f(rd16(x));
        const uint32_t a = rd32u(x + 2 + 64 + 4 * ib);
        const float db = d * (0.5f + (a >> 28)) * 0.5f;
#pragma unroll
        for (int l = 0; l < 4; ++l) {
            const uint32_t s = ksigns7((a >> (7 * l)) & 127);
            const uint64_t g1 = grid[rd8(x + 2 + 8 * ib + 2 * l)], g2 = grid[rd8(x + 2 + 8 * ib + 2 * l + 1)];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                y[8 * l + j] = db * gbyte(g1, j) * sgnb(s, j);
                y[8 * l + j + 4] = db * gbyte(g2, j) * sgnb(s, j + 4);
            }
        }
    } else if (TYPE == T_IQ3_S) {
        const float d = h2f(rd16(x));
        const uint32_t sc = rd8(x + 106 + ib / 2);
        const float db = d * (1 + 2 * ((sc >> (4 * (ib % 2))) & 0xf));
        const uint32_t qh = rd8(x + 66 + ib);
#pragma unroll
        for (int l = 0; l < 4; ++l) {
            const uint32_t s = rd8(x + 74 + 4 * ib + l);
            const uint64_t g1 = grid[rd8(x + 2 + 8 * ib + 2 * l) | ((qh << (8 - 2 * l)) & 256)];
            const uint64_t g2 = grid[rd8(x + 2 + 8 * ib + 2 * l + 1) | ((qh << (7 - 2 * l)) & 256)];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                y[8 * l + j] = db * gbyte(g1, j) * sgnb(s, j);
                y[8 * l + j + 4] = db * gbyte(g2, j) * sgnb(s, j + 4);
            }
        }
    } else if (TYPE == T_IQ1_S) {
        const float d = h2f(rd16(x));
        const uint32_t qh = rd16(x + 34 + 2 * ib);
        const float dl = d * (2 * ((qh >> 12) & 7) + 1);
        const float delta = qh & 0x8000 ? -0.125f : 0.125f;
#pragma unroll
        for (int l = 0; l < 4; ++l) {
            const uint64_t pt = grid[rd8(x + 2 + 4 * ib + l) | (((qh >> (3 * l)) & 7) << 8)];
#pragma unroll
            for (int j = 0; j < 8; ++j) y[8 * l + j] = dl * ((float)(int8_t)gbyte(pt, j) + delta);
        }
    } else if (TYPE == T_IQ1_M) {
        uint32_t sc[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) sc[i] = rd16(x + 48 + 2 * i);
        const uint32_t scale = (sc[0] >> 12) | ((sc[1] >> 8) & 0x00f0) | ((sc[2] >> 4) & 0x0f00) | (sc[3] & 0xf000);
        const float d = h2f(scale);
        const uint32_t s2 = sc[ib / 2];
        const float dl1 = d * (2 * ((s2 >> (6 * (ib % 2) + 0)) & 0x7) + 1);
        const float dl2 = d * (2 * ((s2 >> (6 * (ib % 2) + 3)) & 0x7) + 1);
        const uint32_t qh0 = rd8(x + 32 + 2 * ib), qh1 = rd8(x + 32 + 2 * ib + 1);
        const uint32_t idx[4] = {rd8(x + 4 * ib + 0) | ((qh0 << 8) & 0x700), rd8(x + 4 * ib + 1) | ((qh0 << 4) & 0x700),
                                 rd8(x + 4 * ib + 2) | ((qh1 << 8) & 0x700), rd8(x + 4 * ib + 3) | ((qh1 << 4) & 0x700)};
        const float delta[4] = {qh0 & 0x08 ? -0.125f : 0.125f, qh0 & 0x80 ? -0.125f : 0.125f,
                                qh1 & 0x08 ? -0.125f : 0.125f, qh1 & 0x80 ? -0.125f : 0.125f};
#pragma unroll
        for (int l = 0; l < 4; ++l) {
            const uint64_t pt = grid[idx[l]];
#pragma unroll
            for (int j = 0; j < 8; ++j) y[8 * l + j] = (l < 2 ? dl1 : dl2) * ((float)(int8_t)gbyte(pt, j) + delta[l]);
        }
    } else if (TYPE == T_IQ4_XS) {
        const float d = h2f(rd16(x));
        const uint32_t sh = rd16(x + 2);
        const int ls = (int)(((rd8(x + 4 + ib / 2) >> (4 * (ib % 2))) & 0xf) | (((sh >> (2 * ib)) & 3) << 4));
        const float dl = d * (ls - 32);
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const uint32_t q = rd8(x + 8 + 16 * ib + j);
            y[j] = dl * k_iq4nl_i8[q & 0xf];
            y[j + 16] = dl * k_iq4nl_i8[q >> 4];
        }
    }
}

template <int TYPE, int BB>
__global__ __launch_bounds__(256) void k_dequant(const uint8_t *q, float *out, int64_t nblocks, const uint64_t *grid) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= nblocks * 8) return;
    const int64_t b = t / 8;
    const int ib = (int)(t % 8);
    float y[32];
    dq_chunk<TYPE>(q + b * BB, ib, y, grid);
    float4 *o = (float4 *)(out + b * QK + 32 * ib);
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = make_float4(y[4 * i], y[4 * i + 1], y[4 * i + 2], y[4 * i + 3]);
}

// source bytes -> f32, one thread a 32-value block (gpuq/gpuq.hip:2123-2141)
template <int SRC> __global__ __launch_bounds__(256) void k_decode(const uint8_t *in, float *out, int64_t nblk) {
    const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= nblk) return;
    float v[32];
    SrcLoad<SRC, 32>::load(in, b * 32, v);
    float4 *o = (float4 *)(out + b * 32);
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = make_float4(v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]);
}
