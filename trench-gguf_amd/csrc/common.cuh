// trench-gguf_amd/csrc/common.cuh - device helpers shared by the quantizer kernels (gfx950, wave64).
//
// Exactness: this library is compiled with -ffp-contract=off and without fast-math, so every float expression below
// is evaluated as written (no FMA contraction, IEEE "/" and sqrtf, fp32 subnormals kept). The scalar helpers restate
// ggml's fp32->fp16 rounding (gpuq/gpuq.hip:91-106), exact fp16->fp32 (gpuq/gpuq.hip:2108-2120), the magic-number
// nearest_int (gpuq/gpuq.hip:108-112) and e8m0 scales (gpuq/gpuq.hip:2121).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define QK 256
#define DEV __device__ __forceinline__
#define GQ_WAVE 64

enum {
    T_F32 = 0, T_F16 = 1, T_Q4_0 = 2, T_Q5_0 = 6, T_Q5_1 = 7, T_Q8_0 = 8, T_Q2_K = 10, T_Q3_K = 11, T_Q4_K = 12, T_Q5_K = 13, T_Q6_K = 14,
    T_IQ2_XXS = 16, T_IQ2_XS = 17, T_IQ3_XXS = 18, T_IQ1_S = 19, T_IQ4_NL = 20, T_IQ3_S = 21, T_IQ2_S = 22,
    T_IQ4_XS = 23, T_IQ1_M = 29, T_BF16 = 30, T_MXFP4 = 39
};

DEV uint32_t fbits(float f) { return __float_as_uint(f); }
DEV float ffrom(uint32_t u) { return __uint_as_float(u); }
DEV float fmax_sel(float a, float b) { return a > b ? a : b; }   // ggml's MAX macro: a > b ? a : b
DEV float fmin_sel(float a, float b) { return a < b ? a : b; }
// a compile-time int as a type (a generic lambda's size parameter)
template <int V> struct IntC { static constexpr int value = V; };
DEV int imax(int a, int b) { return a > b ? a : b; }
DEV int imin(int a, int b) { return a < b ? a : b; }
// make v opaque to the optimizer at this point (no instruction): expressions of v are not hoisted across it
DEV void opaque(float &v) { asm volatile("" : "+v"(v)); }
// hide a float holding a small non-negative integer from the optimizer (no instruction), so that q * q stays one float
// multiply (exact below 2^12): left to itself the compiler squares the integer instead, with v_mul_u32_u24 and
// v_cvt_f32_u32, both four-clock instructions, where v_mul_f32 issues at twice their rate
DEV float small_int_f(float q) {
    asm("" : "+v"(q));
    return q;
}

// RNE fp32 -> fp16 through the fp32 adder; NaN -> 0x7E00
DEV uint16_t f2h(float f) {
    float base = (fabsf(f) * 0x1.0p+112f) * 0x1.0p-110f;
    const uint32_t w = fbits(f);
    const uint32_t w2 = w + w;
    const uint32_t sgn = w & 0x80000000u;
    uint32_t bias = w2 & 0xFF000000u;
    bias = bias < 0x71000000u ? 0x71000000u : bias;
    base = ffrom((bias >> 1) + 0x07800000u) + base;
    const uint32_t b = fbits(base);
    const uint32_t nonsign = ((b >> 13) & 0x00007C00u) + (b & 0x00000FFFu);
    return (uint16_t)((sgn >> 16) | (w2 > 0xFF000000u ? 0x7E00u : nonsign));
}

// exact fp16 -> fp32 (subnormal halves are normalised with a count of leading zeros, no loop)
DEV float h2f(uint32_t h) {
    const uint32_t sgn = (h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1f, m = h & 0x3ffu;
    if (e == 0) {
        if (m == 0) return ffrom(sgn);
        const int sh = __clz(m) - 21;                      // shifts that bring the top set bit to bit 10
        return ffrom(sgn | ((uint32_t)(113 - sh) << 23) | (((m << sh) & 0x3ffu) << 13));
    }
    if (e == 31) return ffrom(sgn | 0x7f800000u | (m << 13));
    return ffrom(sgn | ((e + 112) << 23) | (m << 13));
}

DEV int nint(float v) {
    const float t = v + 12582912.f;
    return (int)(fbits(t) & 0x007fffffu) - 0x00400000;
}

DEV float e8m0_half(uint32_t e) { return ffrom(e < 2 ? 0x00200000u << e : (e - 1) << 23); }

// ------------------------------------------------------------------ lane groups
// A super-block is owned by G consecutive lanes of a wave (lane g holds sub-block g); G is 8 or 16, so a group never
// crosses a row of 16 lanes and 64/G super-blocks share a wave.
DEV int lane_id() { return (int)(threadIdx.x & 63); }

template <int G> DEV float grp_bcast(float v, int src_g) {
    return __shfl(v, (lane_id() & ~(G - 1)) + src_g, 64);
}
template <int G> DEV int grp_bcast_i(int v, int src_g) {
    return __shfl(v, (lane_id() & ~(G - 1)) + src_g, 64);
}
// max over the group's values with ggml's MAX (non-negative, non-NaN inputs give the order-free maximum)
template <int G> DEV float grp_max(float v) {
#pragma unroll
    for (int o = 1; o < G; o <<= 1) v = fmax_sel(__shfl_xor(v, o, 64), v);
    return v;
}
template <int G> DEV int grp_or(int v) {
#pragma unroll
    for (int o = 1; o < G; o <<= 1) v |= __shfl_xor(v, o, 64);
    return v;
}

// An index-order sum that spans the group: lane g adds its n terms (in order) to the running total of lanes 0..g-1,
// so the result is the serial left-to-right sum over all G*n terms. Returned to every lane of the group.
template <int G, int N> DEV float grp_chain_sum(const float (&t)[N], int g) {
    float acc = 0.f;
#pragma unroll
    for (int j = 0; j < G; ++j) {
        float s = acc;
        if (g == j) {
#pragma unroll
            for (int i = 0; i < N; ++i) s += t[i];
        }
        acc = grp_bcast<G>(s, j);
    }
    return acc;
}

// ------------------------------------------------------------------ fused source decode
// A lane's N consecutive values of the source tensor, starting at element e0 (a multiple of N; N = 16 or 32),
// decoded in registers exactly as ggml's to_float (gpuq/gpuq.hip:2123-2141): F32 copy, F16 exact, BF16 bits << 16,
// Q8_0 int8 * fp16(d), MXFP4 kv[nibble] * 2^(e-128) with the low nibbles -> 0..15 and the high -> 16..31.
DEV uint32_t ld_u8(const uint8_t *p) { return *p; }

template <int SRC, int N> struct SrcLoad;

template <int N> struct SrcLoad<T_F32, N> {
    static DEV void load(const uint8_t *raw, int64_t e0, float (&v)[N]) {
        const float4 *p = (const float4 *)(raw + e0 * 4);
#pragma unroll
        for (int i = 0; i < N / 4; ++i) {
            const float4 q = p[i];
            v[4 * i + 0] = q.x; v[4 * i + 1] = q.y; v[4 * i + 2] = q.z; v[4 * i + 3] = q.w;
        }
    }
};
template <int N> struct SrcLoad<T_BF16, N> {
    static DEV void load(const uint8_t *raw, int64_t e0, float (&v)[N]) {
        const uint4 *p = (const uint4 *)(raw + e0 * 2);
#pragma unroll
        for (int i = 0; i < N / 8; ++i) {
            const uint4 q = p[i];
            const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                v[8 * i + 2 * k + 0] = ffrom(w[k] << 16);
                v[8 * i + 2 * k + 1] = ffrom(w[k] & 0xffff0000u);
            }
        }
    }
};
template <int N> struct SrcLoad<T_F16, N> {
    static DEV void load(const uint8_t *raw, int64_t e0, float (&v)[N]) {
        const uint4 *p = (const uint4 *)(raw + e0 * 2);
#pragma unroll
        for (int i = 0; i < N / 8; ++i) {
            const uint4 q = p[i];
            const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                v[8 * i + 2 * k + 0] = h2f(w[k] & 0xffffu);
                v[8 * i + 2 * k + 1] = h2f(w[k] >> 16);
            }
        }
    }
};
template <int N> struct SrcLoad<T_Q8_0, N> {
    // 34-byte blocks (fp16 d, int8 qs[32]), 2-byte aligned: read as 16-bit words
    static DEV void load(const uint8_t *raw, int64_t e0, float (&v)[N]) {
        const uint8_t *blk = raw + (e0 / 32) * 34;
        const int off = (int)(e0 % 32);                    // 0, or 16 for the second half of a block
        const uint16_t *w = (const uint16_t *)blk;
        const float d = h2f(w[0]);
#pragma unroll
        for (int i = 0; i < N / 2; ++i) {
            const uint32_t q = w[1 + off / 2 + i];
            v[2 * i + 0] = (float)(int8_t)(q & 0xff) * d;
            v[2 * i + 1] = (float)(int8_t)(q >> 8) * d;
        }
    }
};
template <int N> struct SrcLoad<T_MXFP4, N> {
    // 17-byte blocks (e8m0 e, 16 bytes of e2m1 pairs), byte aligned
    static DEV void load(const uint8_t *raw, int64_t e0, float (&v)[N]) {
        const int8_t kv[16] = {0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12};
        const uint8_t *blk = raw + (e0 / 32) * 17;
        const float d = e8m0_half(ld_u8(blk));
        if (N == 32) {
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                const uint32_t q = ld_u8(blk + 1 + j);
                v[j] = (float)kv[q & 0x0f] * d;
                v[(j + 16) % N] = (float)kv[q >> 4] * d;
            }
        } else {
            const int hi = (int)(e0 % 32) != 0;            // the second 16 values are the high nibbles
#pragma unroll
            for (int j = 0; j < N; ++j) {
                const uint32_t q = ld_u8(blk + 1 + j);
                v[j] = (float)kv[hi ? (q >> 4) : (q & 0x0f)] * d;
            }
        }
    }
};

DEV int64_t src_bytes_per(int src, int64_t n) {
    switch (src) {
        case T_F32: return n * 4;
        case T_F16: case T_BF16: return n * 2;
        case T_Q8_0: return n / 32 * 34;
        case T_MXFP4: return n / 32 * 17;
        default: return 0;
    }
}
