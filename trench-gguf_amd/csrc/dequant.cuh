// trench-gguf_amd/csrc/dequant.cuh - ggml's to_float of the i-quants, IQ4_XS and the k-quants, and the source decoder.
//
// Semantics: dequantize_row_iq* (gpuq/gpuq.hip:1850-2021) and ggml's dequantize_row_q2_K .. q6_K (the reference
// reads the k-quants back through libggml-base's to_float, tools/requant_experts.py:588-591): only products of small
// integers, fp16 scales and powers of two, in ggml's operand order, so fp32 reproduces ggml bit for bit. One thread
// produces one 32-value chunk (8 threads a super-block) with 16-byte stores; the dequantizer grid (uint64 points) is
// read through the cache.
#pragma once
#include "frame.cuh"

DEV uint32_t ksigns7(uint32_t k) { return k | ((uint32_t)(__popc(k) & 1) << 7); }
DEV float sgnb(uint32_t s, int j) { return (s >> j) & 1 ? -1.f : 1.f; }
DEV uint32_t rd8(const uint8_t *p) { return *p; }
DEV uint32_t rd16(const uint8_t *p) { return (uint32_t)*(const uint16_t *)p; }     // 2-byte aligned fields
DEV uint32_t rd32u(const uint8_t *p) { return rd16(p) | (rd16(p + 2) << 16); }     // 2-byte aligned dword
DEV uint32_t gbyte(uint64_t pt, int j) { return (uint32_t)(pt >> (8 * j)) & 0xffu; }

__constant__ int8_t k_iq4nl_i8[16] = {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113};

// Q4_K / Q5_K: sub-block j's 6-bit scale and min from the 12-byte scales field (j < 4: low 6 bits of bytes j and j+4;
// j >= 4: a nibble of byte j+4 and the top 2 bits of bytes j-4 and j)
DEV void k4_scale_min(const uint8_t *s, int j, uint32_t &sc, uint32_t &mn) {
    if (j < 4) {
        sc = rd8(s + j) & 63;
        mn = rd8(s + j + 4) & 63;
    } else {
        sc = (rd8(s + j + 4) & 0xf) | ((rd8(s + j - 4) >> 6) << 4);
        mn = (rd8(s + j + 4) >> 4) | ((rd8(s + j) >> 6) << 4);
    }
}

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
    } else if (TYPE == T_Q4_K || TYPE == T_Q5_K) {
        // block d dmin scales[12] (qh[32], Q5_K) qs[128]; chunk ib: sub-block ib's 6-bit scale and min, the low
        // (even ib) or high (odd ib) nibbles of qs[32 (ib/2) ..], Q5_K's fifth bit from bit ib of qh[j]
        const float d = h2f(rd16(x)), dmin = h2f(rd16(x + 2));
        uint32_t sc, mn;
        k4_scale_min(x + 4, ib, sc, mn);
        const float dl = d * (float)sc, ml = dmin * (float)mn;
        const uint8_t *q = x + (TYPE == T_Q5_K ? 48 : 16) + 32 * (ib / 2);
        const int sh = 4 * (ib & 1);
#pragma unroll
        for (int j = 0; j < 32; ++j) {
            int v = (int)((rd8(q + j) >> sh) & 0xf);
            if (TYPE == T_Q5_K) v += (rd8(x + 16 + j) >> ib) & 1 ? 16 : 0;
            y[j] = dl * (float)v - ml;
        }
    } else if (TYPE == T_Q6_K) {
        // block ql[128] qh[64] scales[16] (int8) d; chunk ib = 4n + part of the 128-value half n: ql[64n + 32 (part
        // & 1) + j], its low (part < 2) or high nibble, bits 2 part of qh[32n + j], scale scales[8n + 2 part + j/16]
        const float d = h2f(rd16(x + 208));
        const int n = ib / 4, part = ib % 4;
        const uint8_t *ql = x + 64 * n + 32 * (part & 1), *qh = x + 128 + 32 * n;
        const int qsh = 4 * (part >> 1), hsh = 2 * part;
#pragma unroll
        for (int j = 0; j < 32; ++j) {
            const int q = (int)(((rd8(ql + j) >> qsh) & 0xf) | (((rd8(qh + j) >> hsh) & 3) << 4)) - 32;
            const int s = (int)(int8_t)rd8(x + 192 + 8 * n + 2 * part + j / 16);
            y[j] = d * (float)s * (float)q;
        }
    } else if (TYPE == T_Q2_K) {
        // block scales[16] qs[64] d dmin; chunk ib = 4n + j: 2-bit fields at shift 2j of qs[32n + 16h + l], scale
        // byte 8n + 2j + h (low nibble the scale, high the min) for its halves h
        const float d = h2f(rd16(x + 80)), dmin = h2f(rd16(x + 82));
        const int n = ib / 4, jj = ib % 4;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const uint32_t sc = rd8(x + 8 * n + 2 * jj + h);
            const float dl = d * (float)(sc & 0xf), ml = dmin * (float)(sc >> 4);
#pragma unroll
            for (int l = 0; l < 16; ++l)
                y[16 * h + l] = dl * (float)((rd8(x + 16 + 32 * n + 16 * h + l) >> (2 * jj)) & 3) - ml;
        }
    } else if (TYPE == T_Q3_K) {
        // block hmask[32] qs[64] scales[12] d; chunk ib = 4n + j: 2-bit fields at shift 2j of qs[32n + 16h + l],
        // minus 4 where bit 4n + j of hmask[16h + l] is clear; 6-bit scale 8n + 2j + h (low 4 bits from a nibble of
        // scales[0..7], high 2 bits from scales[8..11]), minus 32
        const float d = h2f(rd16(x + 108));
        const int n = ib / 4, jj = ib % 4;
        const uint8_t *s = x + 96;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int i = 8 * n + 2 * jj + h;
            const uint32_t lo = i < 8 ? rd8(s + i) & 0xf : rd8(s + i - 8) >> 4;
            const int sc = (int)(lo | (((rd8(s + 8 + i % 4) >> (2 * (i / 4))) & 3) << 4)) - 32;
            const float dl = d * (float)sc;
#pragma unroll
            for (int l = 0; l < 16; ++l) {
                const int q = (int)((rd8(x + 32 + 32 * n + 16 * h + l) >> (2 * jj)) & 3) -
                              ((rd8(x + 16 * h + l) >> (4 * n + jj)) & 1 ? 0 : 4);
                y[16 * h + l] = dl * (float)q;
            }
        }
    }
}

// A wave's 64 threads each decode 32 consecutive values (thread t: values 32t .. 32t+31 of the launch), so the wave's
// output is one contiguous run of 2,048 floats. Written straight from the threads, each 16-byte store instruction
// would touch 64 lines 128 bytes apart; the values go through the wave's LDS rows instead (a thread's eight float4
// 144 bytes apart: a quarter-wave's 16-byte writes fall in distinct banks) and leave as eight stores of 1 KB runs.
// n32: the launch's 32-value units; a unit past it is neither read nor written.
DEV void store_runs(float4 *st, float *out, int64_t t, int64_t n32, const float (&y)[32]) {
    const int lane = lane_id();
#pragma unroll
    for (int i = 0; i < 8; ++i) st[lane * 9 + i] = make_float4(y[4 * i], y[4 * i + 1], y[4 * i + 2], y[4 * i + 3]);
    wave_sync();
    const int64_t t0 = t - lane;                        // the wave's first unit
    float4 *o = (float4 *)(out + t0 * 32);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int f = lane + 64 * i;                    // float4 f of the wave's run: unit f / 8, part f % 8
        if (t0 + f / 8 < n32) o[f] = st[(f / 8) * 9 + f % 8];
    }
}

template <int TYPE, int BB>
__global__ __launch_bounds__(256) void k_dequant(const uint8_t *q, float *out, int64_t nblocks, const uint64_t *grid) {
    __shared__ float4 st[4][64 * 9];
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    float y[32];
    if (t < nblocks * 8) {
        dq_chunk<TYPE>(q + (t / 8) * BB, (int)(t % 8), y, grid);
    } else {
#pragma unroll
        for (int i = 0; i < 32; ++i) y[i] = 0.f;
    }
    store_runs(st[threadIdx.x >> 6], out, t, nblocks * 8, y);
}

// source bytes -> f32, one thread a 32-value block (gpuq/gpuq.hip:2123-2141)
template <int SRC> __global__ __launch_bounds__(256) void k_decode(const uint8_t *in, float *out, int64_t nblk) {
    __shared__ float4 st[4][64 * 9];
    const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    float v[32];
    if (b < nblk) {
        SrcLoad<SRC, 32>::load(in, b * 32, v);
    } else {
#pragma unroll
        for (int i = 0; i < 32; ++i) v[i] = 0.f;
    }
    store_runs(st[threadIdx.x >> 6], out, b, nblk, v);
}
