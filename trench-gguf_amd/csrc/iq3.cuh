// trench-gguf_amd/csrc/iq3.cuh - IQ3_XXS and IQ3_S on gfx950.
//
// Semantics: ggml's quantize_row_iq3_xxs_impl / quantize_row_iq3_s_impl as the reference restates them
// (gpuq/gpuq.hip:971-1283). Per lane: one 32-weight sub-block of eight 4-value groups. The whole 4096-entry 3-bit
// key map (every key is reachable: levels 0..7; off-grid entries packed with their list's offset and length) and the
// grid (uint32 points, byte i = 2l+1) sit in LDS; neighbour lists stay in HBM. A group's levels are kept as its
// point's 4 bytes, one dword a group. The neighbour searches are wave-wide (coop.cuh): two trials' 8 groups in two
// calls of 8 lists a lane (a half's 4 groups at both scales, its groups' values staged once), the final pass in two
// calls of 4; one 8-wave workgroup a CU (the 8-list workspace).
#pragma once
#include "iq2.cuh"

#define EPS_IQ3XXS 1e-8f
#define NKEY8 4096

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

template <int GRID> struct Iq4Tab {
    static constexpr int GRIDB = GRID * 4;
    static constexpr int TAB = (GRIDB + NKEY8 * 4 + 15) & ~15;
    static DEV void stage(const QParams &p, uint8_t *lds) {
        uint32_t *gd = (uint32_t *)lds;
        for (int i = threadIdx.x; i < GRID; i += blockDim.x) gd[i] = (uint32_t)p.grid[i];
        int32_t *md = (int32_t *)(lds + GRIDB);
        for (int i = threadIdx.x; i < NKEY8; i += blockDim.x) md[i] = p.map3[i];
    }
    static DEV const uint32_t *grid(const uint8_t *lds) { return (const uint32_t *)lds; }
    static DEV const int32_t *map(const uint8_t *lds) { return (const int32_t *)(lds + GRIDB); }
};

DEV int key3_of_point(uint32_t pt) {
    int u = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) u |= (int)((((pt >> (8 * i)) & 0xffu) - 1) >> 1) << (3 * i);
    return u;
}

// iq3_find_best_neighbour's distance of one grid point (gpuq/gpuq.hip:971-992) for an owner's staged values
// (st[0..3] the x's, st[4..7] the weights), in the serial scan's operation order
struct EvalIq4 {
    const uint32_t *grid;
    const uint32_t *npt;                            // the lists' points (QParams::npt)
    static constexpr bool LIST_POINTS = true;
    DEV uint32_t point(int idx) const { return grid[idx]; }
    DEV float operator()(const float *st, float scale, uint32_t pt) const {
        float d2 = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float q = (float)((pt >> (8 * i)) & 0xffu);
            const float diff = scale * q - st[i];
            d2 += st[4 + i] * diff * diff;
        }
        return d2;
    }
};

DEV int group_key8(const float *xv, float id) {
    int u = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) u |= imax(0, imin(7, nint(0.5f * (id * xv[i] - 1)))) << (3 * i);
    return u;
}

using Iq3WS = CoopWSM<4, 8, true>;
// two trials a call: list m = t*4 + k (trial t, group k of the half), the half's 4 groups staged once (rows k), one
// scale row a trial
using Iq3WS2 = CoopWSM<8, 8, true, 4, 2>;
// the neighbour search's piece size (candidates a round): 4 for IQ3_XXS's lists of 4.7 points on average, 8 for
// IQ3_S's of 9.7 (4.6% faster than 4; 8 makes IQ3_XXS 9% slower, 2 either 9-18% slower)
template <int GRID> constexpr int iq3_ch() { return GRID == 512 ? 8 : 4; }

// The 8 groups' points of every lane at one scale (all lanes call it together): a group with act[k] takes the grid
// point of its key (id) if the key is on the grid, else the winner of its neighbour list (the distances at `scale`);
// 4 groups a wave-wide call, each list with its group's staged values. A search that accepts nothing flags the error
// (the reference traps) and yields point 0. P[k] and og[k] (the key was on the grid) are written where act[k].
template <int GRID>
DEV void iq3_points(const bool (&act)[8], float id, float scale, const float (&xval)[32], const float (&waux)[32],
                    const int32_t *map, const uint32_t *grid, const QParams &p, Iq3WS &ws, uint32_t (&P)[8],
                    bool (&og)[8]) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        int mk[4], cnt[4], off[4], gi[4];
        float sc[4];
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            const int k = 4 * h + m;
            mk[m] = 0;
            if (act[k]) mk[m] = map[group_key8(xval + 4 * k, id)];
            const bool srch = act[k] && mk[m] < 0;
            cnt[m] = srch ? m3_cnt(mk[m]) : 0;
            off[m] = srch ? m3_off(mk[m]) : 0;
            sc[m] = scale;
            if (srch) coop_stage<4>(ws, xval + 4 * k, waux + 4 * k, m * 64 + lane_id());
        }
        coop_search_m<4, iq3_ch<GRID>()>(cnt, off, sc, p.neigh, p.neigh_len, ws, EvalIq4{grid, p.npt}, gi);
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            const int k = 4 * h + m;
            if (!act[k]) continue;
            og[k] = mk[m] >= 0;
            int g = mk[m];
            if (g < 0) {
                g = gi[m];
                if (g < 0) {
                    flag_err(p);
                    g = 0;
                }
            }
            P[k] = grid[g];
        }
    }
}

// the 8 groups' points of every lane at two scales (trial 1 only where `two`; a lane that is not live searches
// nothing), as iq3_points: per half of the groups one call of 8 lists a lane. P[t][k]: group k's point at trial t;
// og: bit 8t + k set where that group's key is on the grid (bits kept in one register, not 16 flags)
template <int GRID>
DEV void iq3_points2(bool live, const float (&id)[2], const float (&scale)[2], bool two,
                     const float (&xval)[32], const float (&waux)[32], const int32_t *map, const uint32_t *grid,
                     const QParams &p, Iq3WS2 &ws, uint32_t (&P)[2][8], uint32_t &og) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        int mk[8], cnt[8], off[8], gi[8];
        float sc[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int t = e >> 2, k = 4 * h + (e & 3);
            const bool a = live && (t == 0 || two);
            mk[e] = a ? map[group_key8(xval + 4 * k, id[t])] : 0;
            const bool srch = a && mk[e] < 0;
            cnt[e] = srch ? m3_cnt(mk[e]) : 0;
            off[e] = srch ? m3_off(mk[e]) : 0;
            sc[e] = scale[t];
        }
#pragma unroll
        for (int m = 0; m < 4; ++m)
            coop_stage<4>(ws, xval + 4 * (4 * h + m), waux + 4 * (4 * h + m), m * 64 + lane_id());
        coop_search_m<8, iq3_ch<GRID>()>(cnt, off, sc, p.neigh, p.neigh_len, ws, EvalIq4{grid, p.npt}, gi);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int t = e >> 2, k = 4 * h + (e & 3);
            if (!live || !(t == 0 || two)) continue;
            if (mk[e] >= 0) og |= 1u << (8 * t + k);
            int g = mk[e];
            if (g < 0) {
                g = gi[e];
                if (g < 0) {
                    flag_err(p);
                    g = 0;
                }
            }
            P[t][k] = grid[g];
        }
    }
}

// the shared IQ3 32-weight search (every lane of the wave runs it: the neighbour searches are wave-wide); returns
// the sub-block scale, P = its 8 group points, live = not skipped
template <bool XXS, int GRID>
DEV float iq3_search(const float (&x)[32], const float (&qv)[32], float sigma2, const QParams &p, const uint8_t *lds,
                     Iq3WS2 &ws2, uint32_t (&P)[8], uint32_t (&bsg)[4], bool &live) {
    Iq3WS &ws = *(Iq3WS *)&ws2;
    const uint32_t *grid = Iq4Tab<GRID>::grid(lds);
    const int32_t *map = Iq4Tab<GRID>::map(lds);
    float weight[32], waux[32], xval[32];
#pragma unroll
    for (int i = 0; i < 32; ++i) weight[i] = qv[i] * sqrtf(sigma2 + x[i] * x[i]);
#pragma unroll
    for (int i = 0; i < 32; ++i) waux[i] = sqrtf(weight[i]);
#pragma unroll
    for (int k = 0; k < 4; ++k)
        bsg[k] = XXS ? signs_even8(x + 8 * k, weight + 8 * k, xval + 8 * k) : signs_plain8(x + 8 * k, xval + 8 * k);
    float mx = xval[0];
#pragma unroll
    for (int i = 1; i < 32; ++i) mx = fmax_sel(mx, xval[i]);
#pragma unroll
    for (int k = 0; k < 8; ++k) P[k] = 0x01010101u;          // L = 0
    live = XXS ? !(mx < EPS_IQ3XXS) : (mx != 0.f);
    float best = 0;
    float scale = live ? mx / 15 : 0.f;
    uint32_t on_grid = XXS ? 0xffu : 0u;                  // bit k: group k's point on the grid (IQ3_S starts from
                                                          // "not on the grid")
    constexpr int NT = XXS ? 15 : 9;
#pragma unroll 1
    for (int is = -NT; is <= NT; is += 2) {            // two trials a call (the last alone)
        const bool two = is + 1 <= NT;
        float id[2], this_scale[2];
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            id[t] = (15 + (t && two ? is + 1 : is) * 0.2f) / mx;
            this_scale[t] = 1 / id[t];
        }
        uint32_t Pa[2][8], og = 0;
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int k = 0; k < 8; ++k) Pa[t][k] = 0x01010101u;
        iq3_points2<GRID>(live, id, this_scale, two, xval, waux, map, grid, p, ws2, Pa, og);
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            if (t == 1 && !two) break;
            float sumqx, sumq2;
            sums_q<32>(weight, xval, Pa[t], sumqx, sumq2);
            if (live && sumq2 > 0 && sumqx * sumqx > best * sumq2) {
                scale = sumqx / sumq2;
                best = scale * sumqx;
#pragma unroll
                for (int k = 0; k < 8; ++k) P[k] = Pa[t][k];
                on_grid = (og >> (8 * t)) & 0xffu;
            }
        }
    }
    const bool any_off = on_grid != 0xffu;
    const bool fin = live && any_off && scale > 0;
    {
        const float id = 1 / scale;
        bool act[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) act[k] = fin && !(XXS && ((on_grid >> k) & 1u));   // (IQ3_S: every group)
        bool og[8];
        iq3_points<GRID>(act, id, scale, xval, waux, map, grid, p, ws, P, og);
        if (fin) {
            float sumqx, sumq2;
            sums_q<32>(weight, xval, P, sumqx, sumq2);
            if (sumq2 > 0) scale = sumqx / sumq2;
        }
    }
    if (scale < 0) {
        scale = -scale;
#pragma unroll
        for (int k = 0; k < 4; ++k) bsg[k] = XXS ? ((~bsg[k]) & 127) : ((~bsg[k]) & 255);
    }
    return scale;
}

// IQ3_XXS: block d qs[96] = 64 grid bytes, then 8 u32 signs-and-scales (98 bytes)
struct KIQ3XXS : Iq4Tab<256> {
    static constexpr int BS = QK, G = 8, N = 32, BB = 98, WS = coop_wsm_bytes<8, 8, true, 4, 2>(), WGW = 8;
    static constexpr bool QUEUE = true;         // (tiles of varying cost: the tile queue)
    static DEV void quant(const float (&x)[N], const float *qwp, int g, uint8_t *img, int boff, uint8_t *lds,
                          const QParams &p) {
        const int32_t *map = Iq4Tab<256>::map(lds);
        float qv[N], sq[N];
        load_qw<N>(qwp, qv);
#pragma unroll
        for (int i = 0; i < N; ++i) sq[i] = x[i] * x[i];
        const float sigma2 = 2 * grp_chain_sum<G, N>(sq, g) / QK;
        uint32_t P[8], bsg[4];
        bool live;
        const float scale =
            iq3_search<true, 256>(x, qv, sigma2, p, lds, *(Iq3WS2 *)wave_ws<KIQ3XXS>(img), P, bsg, live);
        const float max_scale = grp_max<G>(live ? scale : 0.f);
        if (!max_scale) return;                               // qs all zero, d = 0
        uint32_t q3lo = 0, q3hi = 0, sas = 0;
        if (live) {
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const int gi = map[key3_of_point(P[k])];
                if (gi < 0) flag_err(p);
                if (k < 4) q3lo |= (uint32_t)(gi & 255) << (8 * k);
                else q3hi |= (uint32_t)(gi & 255) << (8 * (k - 4));
            }
            sas = bsg[0] | (bsg[1] << 7) | (bsg[2] << 14) | (bsg[3] << 21);
        }
        const float d = max_scale / 31;
        if (g == 0) img_or16(img, boff, f2h(d * 1.0125f));
        const float id = 1 / d;
        const int l = imax(0, imin(15, nint(0.5f * (id * (live ? scale : 0.f) - 1))));
        sas |= (uint32_t)l << 28;
        img_or32(img, boff + 2 + 8 * g, q3lo);
        img_or32(img, boff + 6 + 8 * g, q3hi);
        img_or32(img, boff + 2 + 64 + 4 * g, sas);
    }
};

// IQ3_S: block d qs[64] qh[8] signs[32] scales[4] (110 bytes). A skipped (all-zero) sub-block does not advance the
// qs / signs cursors (ggml's quirk, kept by the reference): the next live sub-block takes its slot.
struct KIQ3S : Iq4Tab<512> {
    static constexpr int BS = QK, G = 8, N = 32, BB = 110, WS = coop_wsm_bytes<8, 8, true, 4, 2>(), WGW = 8;
    static constexpr bool QUEUE = true;         // (tiles of varying cost: the tile queue)
    static DEV void quant(const float (&x)[N], const float *qwp, int g, uint8_t *img, int boff, uint8_t *lds,
                          const QParams &p) {
        const int32_t *map = Iq4Tab<512>::map(lds);
        float qv[N], sq[N];
        load_qw<N>(qwp, qv);
#pragma unroll
        for (int i = 0; i < N; ++i) sq[i] = x[i] * x[i];
        const float sigma2 = 2 * grp_chain_sum<G, N>(sq, g) / QK;
        uint32_t P[8], bsg[4];
        bool live;
        const float scale =
            iq3_search<false, 512>(x, qv, sigma2, p, lds, *(Iq3WS2 *)wave_ws<KIQ3S>(img), P, bsg, live);
        // the slot of this sub-block: the number of live sub-blocks before it
        const uint64_t bal = __ballot(live);
        const int gbase = lane_id() & ~(G - 1);
        const uint32_t gm = (uint32_t)(bal >> gbase) & ((1u << G) - 1);
        const int pos = __popc(gm & ((1u << g) - 1));
        if (live) {
            uint32_t qlo = 0, qhi = 0, qh = 0;
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const int gi = map[key3_of_point(P[k])];
                if (gi < 0) flag_err(p);
                if (k < 4) qlo |= (uint32_t)(gi & 255) << (8 * k);
                else qhi |= (uint32_t)(gi & 255) << (8 * (k - 4));
                qh |= (uint32_t)((gi >> 8) & 1) << k;
            }
            img_or32(img, boff + 2 + 8 * pos, qlo);
            img_or32(img, boff + 6 + 8 * pos, qhi);
            img_or8(img, boff + 66 + g, qh);
            img_or32(img, boff + 74 + 4 * pos, bsg[0] | (bsg[1] << 8) | (bsg[2] << 16) | (bsg[3] << 24));
        }
        const float max_scale = grp_max<G>(live ? scale : 0.f);
        if (!max_scale) return;
        const float d = max_scale / 31;
        if (g == 0) img_or16(img, boff, f2h(d * 1.033f));
        const float id = 1 / d;
        const int l = imax(0, imin(15, nint(0.5f * (id * (live ? scale : 0.f) - 1))));
        img_or8(img, boff + 106 + g / 2, (uint32_t)(l << (4 * (g % 2))));
    }
};
