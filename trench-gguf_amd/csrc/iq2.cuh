// trench-gguf_amd/csrc/iq2.cuh - IQ2_XXS, IQ2_XS and IQ2_S on gfx950.
//
// Semantics: ggml's quantize_row_iq2_{xxs,xs,s}_impl as the reference restates them (gpuq/gpuq.hip:178-197,
// 245-387, 690-969). Per lane: one 32-weight (IQ2_XXS) or 16-weight (IQ2_XS / IQ2_S) sub-block, its trial scales run
// serially in ggml's order, including the non-transitive `sumqx^2 > best*sumq2` acceptance chain.
//
// Tables in LDS (per workgroup): the grid points (uint64: byte i = 2l+1) and the key map re-indexed by the base-3
// key sum(l_i * 3^i) of the 3^8 level vectors the trial rounding can produce (levels 0..2), 6561 int32 instead of the
// 43692-entry 2-bit map. The map's meaning is unchanged (>= 0: grid index, < 0: neighbour list offset); neighbour
// lists stay in HBM (L2-resident). The final encode's lookup, whose levels come from grid points (up to 3), reads
// the full 2-bit map in HBM as the reference does.
//
// Level bytes: a group's 8 levels are kept as the grid point's bytes (2l+1), so q = 2l+1 converts straight from a
// byte and a group taken from a grid point is a single 8-byte LDS read. A key found on the grid is replaced by its
// grid point, which holds the same levels (the loader checks map[key(grid[g])] == g for every point).
#pragma once
#include <float.h>
#include "kquants.cuh"

#define EPS_IQ2S 1e-8f
#define NKEY3 6561

template <int GRID> struct Iq8Tab {
    static constexpr int GRIDB = GRID * 8;
    static constexpr int TAB = (GRIDB + NKEY3 * 4 + 15) & ~15;
    static DEV void stage(const QParams &p, uint8_t *lds) {
        const uint4 *gs = (const uint4 *)p.grid;
        uint4 *gd = (uint4 *)lds;
        for (int i = threadIdx.x; i < GRIDB / 16; i += WG_THREADS) gd[i] = gs[i];
        int32_t *md = (int32_t *)(lds + GRIDB);
        for (int i = threadIdx.x; i < NKEY3; i += WG_THREADS) md[i] = p.map3[i];
    }
    static DEV const uint64_t *grid(const uint8_t *lds) { return (const uint64_t *)lds; }
    static DEV const int32_t *map3(const uint8_t *lds) { return (const int32_t *)(lds + GRIDB); }
};

// key of 8 levels from the group's point bytes (2l+1): the reference's 2-bit key sum(l_i << 2i)
DEV int key2_of_point(uint32_t lo, uint32_t hi) {
    int u = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        u |= (int)((((lo >> (8 * i)) & 0xffu) - 1) >> 1) << (2 * i);
        u |= (int)((((hi >> (8 * i)) & 0xffu) - 1) >> 1) << (2 * (i + 4));
    }
    return u;
}

// iq2_find_best_neighbour over a neighbour list (gpuq/gpuq.hip:178-197): weighted-nearest point, first wins on
// ties. Returns the grid index (-1: none, the reference traps).
DEV int nb_best8(const uint16_t *nb, const uint64_t *grid, const float *xv, const float *wa, float scale) {
    const int cnt = nb[0];
    float best = FLT_MAX;
    int gi = -1;
    for (int j = 1; j <= cnt; ++j) {
        const int idx = nb[j];
        const uint64_t pt = grid[idx];
        const uint32_t lo = (uint32_t)pt, hi = (uint32_t)(pt >> 32);
        float d2 = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float q = (float)(((i < 4 ? lo : hi) >> (8 * (i % 4))) & 0xffu);
            const float diff = scale * q - xv[i];
            d2 += wa[i] * diff * diff;
        }
        if (d2 < best) { best = d2; gi = idx; }
    }
    return gi;
}

// the trial rounding of one group: levels clamp(nearest(0.5*(id*x - 1)), 0, 2) and their base-3 key
DEV int group_key3(const float *xv, float id) {
    int k3 = 0, p3 = 1;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int l = imax(0, imin(2, nint(0.5f * (id * xv[i] - 1))));
        k3 += l * p3;
        p3 *= 3;
    }
    return k3;
}

// the group's point for a key: on the grid directly, else the best neighbour (gi < 0 flags a failed search)
DEV int group_point(int k3, const int32_t *map3, const QParams &p, const uint64_t *grid, const float *xv,
                    const float *wa, float scale) {
    const int m = map3[k3];
    if (m >= 0) return m;
    return nb_best8(p.neigh + (-m - 1), grid, xv, wa, scale);
}

DEV void flag_err(const QParams &p) { atomicOr(p.err, 1); }

// signs of 8 values with even parity: an odd count flips the weight with the least w*x^2 (gpuq/gpuq.hip:272-289)
DEV uint32_t signs_even8(const float *xb, const float *weight, float *xval) {
    int nflip = 0;
    uint32_t s = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        if (xb[i] >= 0) xval[i] = xb[i];
        else { xval[i] = -xb[i]; ++nflip; s |= 1u << i; }
    }
    if (nflip % 2) {
        int imn = 0;
        float mn = weight[0] * xb[0] * xb[0];
#pragma unroll
        for (int i = 1; i < 8; ++i) {
            const float ax = weight[i] * xb[i] * xb[i];
            if (ax < mn) { mn = ax; imn = i; }
        }
#pragma unroll
        for (int i = 0; i < 8; ++i)
            if (i == imn) xval[i] = -xval[i];
        s ^= 1u << imn;
    }
    return s & 127;
}
DEV uint32_t signs_plain8(const float *xb, float *xval) {
    uint32_t s = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        if (xb[i] >= 0) xval[i] = xb[i];
        else { xval[i] = -xb[i]; s |= 1u << i; }
    }
    return s;
}

// sum over the sub-block of w*x*q and w*q*q with q = 2l+1 from the packed point bytes (index order)
template <int N> DEV void sums_q(const float (&weight)[N], const float (&xval)[N], const uint32_t (&P)[N / 4],
                                 float &sumqx, float &sumq2) {
    sumqx = 0;
    sumq2 = 0;
#pragma unroll
    for (int i = 0; i < N; ++i) {
        const float w = weight[i];
        const float q = (float)((P[i / 4] >> (8 * (i % 4))) & 0xffu);
        sumqx += w * xval[i] * q;
        sumq2 += w * q * q;
    }
}

// ------------------------------------------------------------------ IQ2_XXS (gpuq/gpuq.hip:245-387)
// block: d qs[32] u16 (66 bytes); lane g = 32-weight sub-block g; q2[2g] at 2+8g, q2[2g+1] at 6+8g
struct KIQ2XXS : Iq8Tab<256> {
    static constexpr int BS = QK, G = 8, N = 32, BB = 66;
    static DEV void quant(const float (&x)[N], const float *qwp, int g, uint8_t *img, int boff, uint8_t *lds,
                          const QParams &p) {
        const uint64_t *grid = Iq8Tab<256>::grid(lds);
        const int32_t *map3 = Iq8Tab<256>::map3(lds);
        float qv[N], sq[N], weight[N], waux[N], xval[N];
        load_qw<N>(qwp, qv);
#pragma unroll
        for (int i = 0; i < N; ++i) sq[i] = x[i] * x[i];
        const float sigma2 = grp_chain_sum<G, N>(sq, g) / QK;
#pragma unroll
        for (int i = 0; i < N; ++i) weight[i] = qv[i] * sqrtf(sigma2 + sq[i]);
#pragma unroll
        for (int i = 0; i < N; ++i) waux[i] = sqrtf(weight[i]);
        uint32_t bsg[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) bsg[k] = signs_even8(x + 8 * k, weight + 8 * k, xval + 8 * k);
        float mx = xval[0];
#pragma unroll
        for (int i = 1; i < N; ++i) mx = fmax_sel(mx, xval[i]);
        float scale = 0.f;
        uint32_t q2lo = 0, q2hi = 0;
        bool live = false;
        if (!(mx < EPS_GROUP)) {
            Lv<N> Lqp;
            scale = qp_levels<N>(4, xval, Lqp, weight);
            const float eff_max = scale * 3;
            if (eff_max <= 0) {
                scale = 0.f;
            } else {
                live = true;
                float best = 0;
                uint32_t P[8];      // accepted trial's point bytes (levels as 2l+1)
#pragma unroll
                for (int k = 0; k < 8; ++k) P[k] = 0u;
                for (int is = -6; is <= 6; ++is) {
                    const float id = (5 + is * 0.1f) / eff_max;
                    const float this_scale = 1 / id;
                    uint32_t Pa[8];
#pragma unroll
                    for (int k = 0; k < 4; ++k) {
                        const int gi = group_point(group_key3(xval + 8 * k, id), map3, p, grid, xval + 8 * k,
                                                   waux + 8 * k, this_scale);
                        if (gi < 0) flag_err(p);
                        const uint64_t pt = grid[gi < 0 ? 0 : gi];
                        Pa[2 * k] = (uint32_t)pt;
                        Pa[2 * k + 1] = (uint32_t)(pt >> 32);
                    }
                    float sumqx, sumq2;
                    sums_q<N>(weight, xval, Pa, sumqx, sumq2);
                    if (sumq2 > 0 && sumqx * sumqx > best * sumq2) {
                        scale = sumqx / sumq2;
                        best = scale * sumqx;
#pragma unroll
                        for (int k = 0; k < 8; ++k) P[k] = Pa[k];
                    }
                }
                // (after the trials scale > 0: either make_qp_quants' positive scale or an accepted positive one)
                if (scale > 0) {
                    const float id = 1 / scale;
#pragma unroll
                    for (int k = 0; k < 4; ++k) {
                        const int gi = group_point(group_key3(xval + 8 * k, id), map3, p, grid, xval + 8 * k,
                                                   waux + 8 * k, scale);
                        if (gi < 0) flag_err(p);
                        const uint64_t pt = grid[gi < 0 ? 0 : gi];
                        P[2 * k] = (uint32_t)pt;
                        P[2 * k + 1] = (uint32_t)(pt >> 32);
                    }
                    float sumqx, sumq2;
                    sums_q<N>(weight, xval, P, sumqx, sumq2);
                    if (sumq2 > 0) scale = sumqx / sumq2;
                }
                if (scale < 0) {
                    scale = -scale;
#pragma unroll
                    for (int k = 0; k < 4; ++k) bsg[k] = (~bsg[k]) & 127;
                }
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const int gi = p.map[key2_of_point(P[2 * k], P[2 * k + 1])];
                    if (gi < 0) flag_err(p);
                    q2lo |= (uint32_t)gi << (8 * k);
                    q2hi |= bsg[k] << (7 * k);
                }
            }
        }
        const float max_scale = grp_max<G>(scale);
        if (!max_scale) return;                     // all-zero block: d = 0, qs = 0 (the image is zero)
        const float d = max_scale / 31;
        const uint16_t d16 = f2h(d);
        const float id = 1 / d;
        if (live) {
            const int l = imax(0, imin(15, nint(0.5f * (id * scale - 1))));
            q2hi |= (uint32_t)l << 28;
        }
        if (g == 0) img_or16(img, boff, d16);
        img_or32(img, boff + 2 + 8 * g, q2lo);
        img_or32(img, boff + 6 + 8 * g, q2hi);
    }
};

// ------------------------------------------------------------------ IQ2_XS / IQ2_S: the 16-weight search
// (gpuq/gpuq.hip:690-822, 824-969). Returns the sub-block scale; gidx the two grid indices, bsg the two sign bytes;
// live = false for a skipped (negligible) sub-block.
template <bool PARITY, int GRID>
DEV float iq2_16_search(const float (&x)[16], const float (&qv)[16], float sigma2, float eps, const QParams &p,
                        const uint8_t *lds, int (&gidx)[2], uint32_t (&bsg)[2], bool &live) {
    const uint64_t *grid = Iq8Tab<GRID>::grid(lds);
    const int32_t *map3 = Iq8Tab<GRID>::map3(lds);
    float weight[16], waux[16], xval[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) weight[i] = qv[i] * sqrtf(sigma2 + x[i] * x[i]);
#pragma unroll
    for (int i = 0; i < 16; ++i) waux[i] = sqrtf(weight[i]);
#pragma unroll
    for (int k = 0; k < 2; ++k)
        bsg[k] = PARITY ? signs_even8(x + 8 * k, weight + 8 * k, xval + 8 * k) : signs_plain8(x + 8 * k, xval + 8 * k);
    float mx = xval[0];
#pragma unroll
    for (int i = 1; i < 16; ++i) mx = fmax_sel(mx, xval[i]);
    live = !(mx < eps);
    gidx[0] = gidx[1] = 0;
    if (!live) return 0.f;
    float best = 0;
    float scale = mx / 5;
    uint32_t P[4] = {0x01010101u, 0x01010101u, 0x01010101u, 0x01010101u};   // L = 0
    bool on_grid[2] = {true, true};
    for (int is = -9; is <= 9; ++is) {
        const float id = (5 + is * 0.1f) / mx;
        const float this_scale = 1 / id;
        uint32_t Pa[4];
        bool og[2];
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const int m = map3[group_key3(xval + 8 * k, id)];
            og[k] = m >= 0;
            const int gi = m >= 0 ? m : nb_best8(p.neigh + (-m - 1), grid, xval + 8 * k, waux + 8 * k, this_scale);
            if (gi < 0) flag_err(p);
            const uint64_t pt = grid[gi < 0 ? 0 : gi];
            Pa[2 * k] = (uint32_t)pt;
            Pa[2 * k + 1] = (uint32_t)(pt >> 32);
        }
        float sumqx, sumq2;
        sums_q<16>(weight, xval, Pa, sumqx, sumq2);
        if (sumq2 > 0 && sumqx * sumqx > best * sumq2) {
            scale = sumqx / sumq2;
            best = scale * sumqx;
#pragma unroll
            for (int k = 0; k < 4; ++k) P[k] = Pa[k];
            on_grid[0] = og[0];
            on_grid[1] = og[1];
        }
    }
    if ((!on_grid[0] || !on_grid[1]) && scale > 0) {
        const float id = 1 / scale;
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            if (on_grid[k]) continue;
            const int gi = group_point(group_key3(xval + 8 * k, id), map3, p, grid, xval + 8 * k, waux + 8 * k, scale);
            if (gi < 0) flag_err(p);
            const uint64_t pt = grid[gi < 0 ? 0 : gi];
            P[2 * k] = (uint32_t)pt;
            P[2 * k + 1] = (uint32_t)(pt >> 32);
        }
        float sumqx, sumq2;
        sums_q<16>(weight, xval, P, sumqx, sumq2);
        if (sumq2 > 0) scale = sumqx / sumq2;
    }
    if (scale < 0) {
        scale = -scale;
#pragma unroll
        for (int k = 0; k < 2; ++k) bsg[k] = PARITY ? ((~bsg[k]) & 127) : ((~bsg[k]) & 255);
    }
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        gidx[k] = p.map[key2_of_point(P[2 * k], P[2 * k + 1])];
        if (gidx[k] < 0) { flag_err(p); gidx[k] = 0; }
    }
    return scale;
}

// IQ2_S: block d qs[64] (32 grid bytes, 32 sign bytes) qh[8] scales[8] (82 bytes); lane g = 16-weight sub-block g
struct KIQ2S : Iq8Tab<1024> {
    static constexpr int BS = QK, G = 16, N = 16, BB = 82;
    static DEV void quant(const float (&x)[N], const float *qwp, int g, uint8_t *img, int boff, uint8_t *lds,
                          const QParams &p) {
        float qv[N], sq[N];
        load_qw<N>(qwp, qv);
#pragma unroll
        for (int i = 0; i < N; ++i) sq[i] = x[i] * x[i];
        const float sigma2 = 2 * grp_chain_sum<G, N>(sq, g) / QK;
        int gidx[2];
        uint32_t bsg[2];
        bool live;
        const float scale = iq2_16_search<false, 1024>(x, qv, sigma2, EPS_IQ2S, p, lds, gidx, bsg, live);
        if (live) {
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                const int i8 = 2 * g + k;
                img_or8(img, boff + 2 + i8, (uint32_t)(gidx[k] & 255));
                img_or8(img, boff + 66 + i8 / 4, (uint32_t)((gidx[k] >> 8) << (2 * (i8 % 4))));
                img_or8(img, boff + 2 + 32 + i8, bsg[k]);
            }
        }
        const float max_scale = grp_max<G>(live ? scale : 0.f);
        if (!max_scale) return;
        const float d = max_scale / 31;
        if (g == 0) img_or16(img, boff, f2h(d * 0.9875f));
        const float id = 1 / d;
        const int l = imax(0, imin(15, nint(0.5f * (id * (live ? scale : 0.f) - 1))));
        img_or8(img, boff + 74 + g / 2, (uint32_t)(l << (4 * (g % 2))));
    }
};

// IQ2_XS: block d qs[32] u16 scales[8] (74 bytes); qs[2g+k] = grid index | signs << 9
struct KIQ2XS : Iq8Tab<512> {
    static constexpr int BS = QK, G = 16, N = 16, BB = 74;
    static DEV void quant(const float (&x)[N], const float *qwp, int g, uint8_t *img, int boff, uint8_t *lds,
                          const QParams &p) {
        float qv[N], sq[N];
        load_qw<N>(qwp, qv);
#pragma unroll
        for (int i = 0; i < N; ++i) sq[i] = x[i] * x[i];
        const float sigma2 = grp_chain_sum<G, N>(sq, g) / QK;
        int gidx[2];
        uint32_t bsg[2];
        bool live;
        const float scale = iq2_16_search<true, 512>(x, qv, sigma2, EPS_GROUP, p, lds, gidx, bsg, live);
        const float max_scale = grp_max<G>(live ? scale : 0.f);
        if (!max_scale) return;                     // qs all zero, scales zero, d = 0
        if (live) {
            const uint32_t w = (uint32_t)(gidx[0] | (bsg[0] << 9)) | ((uint32_t)(gidx[1] | (bsg[1] << 9)) << 16);
            img_or32(img, boff + 2 + 4 * g, w);
        }
        const float d = max_scale / 31;
        if (g == 0) img_or16(img, boff, f2h(d));
        const float id = 1 / d;
        const int l = imax(0, imin(15, nint(0.5f * (id * (live ? scale : 0.f) - 1))));
        img_or8(img, boff + 66 + g / 2, (uint32_t)(l << (4 * (g % 2))));
    }
};
