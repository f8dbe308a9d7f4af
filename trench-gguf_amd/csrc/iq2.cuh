// trench-gguf_amd/csrc/iq2.cuh - IQ2_XXS, IQ2_XS and IQ2_S on gfx950.
//
// Semantics: ggml's quantize_row_iq2_{xxs,xs,s}_impl as the reference restates them (gpuq/gpuq.hip:178-197,
// 245-387, 690-969). Per lane: one 32-weight (IQ2_XXS) or 16-weight (IQ2_XS / IQ2_S) sub-block, its trial scales run
// serially in ggml's order, including the non-transitive `sumqx^2 > best*sumq2` acceptance chain. The neighbour
// searches of a trial (off-grid keys) run wave-wide (coop.cuh), so every lane of the wave executes every trial.
//
// Tables in LDS (per workgroup): the grid points (uint64: byte i = 2l+1) and the key map re-indexed by the base-3
// key sum(l_i * 3^i) of the 3^8 level vectors the trial rounding can produce (levels 0..2), 6561 int32 instead of the
// 43692-entry 2-bit map. The map's meaning is unchanged (>= 0: grid index, < 0: neighbour list offset); neighbour
// lists stay in HBM (L2-resident).
//
// Groups as grid indices: every group's levels after a search are those of a grid point (the key's own point, or the
// chosen neighbour), so a trial's levels are held as its groups' grid indices and q = 2l+1 is read from the point's
// bytes. The reference's final encode looks the levels up again in the full map; for a grid point's levels that
// returns the point itself (the loader checks map[key(grid[g])] == g for every point), so the index is written as is.
#pragma once
#include <float.h>
#include "kquants.cuh"
#include "coop.cuh"
#include "filter.cuh"

#define EPS_IQ2S 1e-8f
#define NKEY3 6561

template <int GRID> struct Iq8Tab {
    static constexpr int GRIDB = GRID * 8;
    static constexpr int TAB = (GRIDB + NKEY3 * 4 + 15) & ~15;
    static DEV void stage(const QParams &p, uint8_t *lds) {
        const uint4 *gs = (const uint4 *)p.grid;
        uint4 *gd = (uint4 *)lds;
        for (int i = threadIdx.x; i < GRIDB / 16; i += blockDim.x) gd[i] = gs[i];
        int32_t *md = (int32_t *)(lds + GRIDB);
        for (int i = threadIdx.x; i < NKEY3; i += blockDim.x) md[i] = p.map3[i];
    }
    static DEV const uint64_t *grid(const uint8_t *lds) { return (const uint64_t *)lds; }
    static DEV const int32_t *map3(const uint8_t *lds) { return (const int32_t *)(lds + GRIDB); }
};

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

DEV void flag_err(const QParams &p) { atomicOr(p.err, 1); }

// iq2_find_best_neighbour's distance of one grid point (gpuq/gpuq.hip:186-191) for an owner's staged values
// (st[0..7] the x's, st[8..15] the weights), in the serial scan's operation order
struct EvalIq8 {
    const uint64_t *grid;
    DEV uint64_t point(int idx) const { return grid[idx]; }
    DEV float operator()(const float *st, float scale, uint64_t pt) const {
        const uint32_t lo = (uint32_t)pt, hi = (uint32_t)(pt >> 32);
        float d2 = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float q = (float)(((i < 4 ? lo : hi) >> (8 * (i % 4))) & 0xffu);
            const float diff = scale * q - st[i];
            d2 += st[8 + i] * diff * diff;
        }
        return d2;
    }
};

// Two groups' grid points on every lane of the wave (all lanes call it together), in one wave-wide search call: two
// lists a lane, each with its group's x's and weights staged in row k*64 + lane. An active lane whose key is on the
// grid takes that point (og), an active off-grid key the winner of its neighbour list, an inactive lane 0; a search
// that accepts nothing flags the error (the reference traps) and yields 0.
using Iq8WS2 = CoopWSM<2, 16, true>;
DEV void group_points2_w(bool active, const int (&k3)[2], const int32_t *map3, const QParams &p, const uint64_t *grid,
                         const float *x0, const float *w0, const float *x1, const float *w1, float scale, Iq8WS2 &ws,
                         int (&gi)[2], bool (&og)[2]) {
    int m[2], cnt[2], off[2], g[2];
    const float sc[2] = {scale, scale};
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        m[k] = active ? map3[k3[k]] : 0;
        og[k] = m[k] >= 0;
        const bool srch = active && m[k] < 0;
        off[k] = srch ? m3_off(m[k]) : 0;
        cnt[k] = srch ? m3_cnt(m[k]) : 0;
        coop_stage<8>(ws, k ? x1 : x0, k ? w1 : w0, k * 64 + lane_id());
    }
    coop_search_m<2, 4>(cnt, off, sc, p.neigh, p.neigh_len, ws, EvalIq8{grid}, g);
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        if (!(active && m[k] < 0)) {
            gi[k] = active ? m[k] : 0;
        } else if (g[k] < 0) {
            flag_err(p);
            gi[k] = 0;
        } else {
            gi[k] = g[k];
        }
    }
}

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

// rotate a sub-block's 32 values left by one group (four rotations restore the order): a rolled loop over the
// groups then always finds the current group at [0, 8) and never indexes registers with a variable
DEV void rot8(float (&v)[32]) {
    float t[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) t[i] = v[i];
#pragma unroll
    for (int i = 0; i < 24; ++i) v[i] = v[i + 8];
#pragma unroll
    for (int i = 0; i < 8; ++i) v[24 + i] = t[i];
}

// one group's terms of the sub-block sums of w*x*q and w*q*q (q = 2l+1 from the point's bytes), added in index order
DEV void sums_q8(const float *w, const float *xv, uint64_t pt, float &sumqx, float &sumq2) {
    const uint32_t lo = (uint32_t)pt, hi = (uint32_t)(pt >> 32);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float q = (float)(((i < 4 ? lo : hi) >> (8 * (i % 4))) & 0xffu);
        sumqx += w[i] * xv[i] * q;
        sumq2 += w[i] * q * q;
    }
}

// One group's trials of a window (every lane of the wave calls it together: the searches are wave-wide). xk, waux:
// the group's 8 values and search weights; trial m's inverse scale idv[m] and scale tsv[m]; valid: the trials that
// run (bit m; none for a lane that is not live). Trial m's key at idv[m]: on the grid its point; the runs of trials
// with one off-grid key are searched by one filtered walk of the key's list (filter.cuh), and a trial the filter leaves
// undecided goes through the exact search, up to 4 a lane a call (a search that accepts nothing flags the error, as
// the reference traps, and yields 0). gk[m]: trial m's grid index (0 for a trial that does not run); og: bit m set
// where trial m's key is on the grid (and for a trial that does not run). IB, NG: the grid indices' bits and the
// grid's size. The staged area of fws, ws and wsm is one (the caller's workspace). DEFER: the undecided trials are
// not searched here but returned in undec (bit m; their gk[m] is 0), for the caller to search with others at once.
template <int TW, int IB, int NG, bool DEFER = false>
DEV void window_group(const float (&xk)[8], const float (&waux)[8], const float (&idv)[TW], const float (&tsv)[TW],
                      unsigned valid, const int32_t *map3, const QParams &p, const uint64_t *grid, FiltWS<TW> &fws,
                      CoopWS &ws, CoopWSM<4> &wsm, int (&gk)[TW], unsigned &og, unsigned &undec) {
    float sw = 0.f, swx = 0.f, swxx = 0.f;      // the filter's bound: sums of w, w|x|, w x^2
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        sw += waux[i];
        swx = fmaf(waux[i], fabsf(xk[i]), swx);
        swxx = fmaf(waux[i] * xk[i], xk[i], swxx);
    }
    // the window's keys; a list a run of equal off-grid keys (cnt > 0 at the run's first trial)
    int mk[TW], cnt[TW], off[TW], ntr[TW];
    og = 0;
#pragma unroll
    for (int m = 0; m < TW; ++m) {
        mk[m] = (valid >> m) & 1 ? map3[group_key3(xk, idv[m])] : 0;
        if (mk[m] >= 0) og |= 1u << m;
    }
    {
        int run = 0;
#pragma unroll
        for (int m = TW - 1; m >= 0; --m) {
            run = mk[m] < 0 ? (m + 1 < TW && mk[m + 1] == mk[m] ? run + 1 : 1) : 0;
            const bool head = mk[m] < 0 && (m == 0 || mk[m - 1] != mk[m]);
            cnt[m] = head ? m3_cnt(mk[m]) : 0;
            off[m] = head ? m3_off(mk[m]) : 0;
            ntr[m] = head ? run : 0;
        }
    }
    unsigned k1[TW], k2[TW];
    coop_filter<TW, IB, NG>(cnt, off, ntr, tsv, xk, waux, p.neigh, p.neigh_len, fws, grid, k1, k2);
    unsigned amb = 0;
#pragma unroll
    for (int m = 0; m < TW; ++m) {
        gk[m] = mk[m] >= 0 ? mk[m] : filt_pick<IB>(k1[m], k2[m], tsv[m], sw, swx, swxx);
        if (gk[m] < 0) amb |= 1u << m;
    }
    undec = DEFER ? amb : 0u;
    if (DEFER) {
#pragma unroll
        for (int m = 0; m < TW; ++m) gk[m] = gk[m] < 0 ? 0 : gk[m];
        return;
    }
    if (__ballot(amb != 0)) coop_stage<8>(ws, xk, waux);
#pragma unroll 1
    while (__ballot(amb != 0)) {
        int em[4], ecnt[4], eoff[4], egi[4];
        float esc[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            em[i] = amb ? __builtin_ctz(amb) : -1;
            amb &= amb - 1;
            int mv = 0;
            esc[i] = tsv[0];
#pragma unroll
            for (int m = 0; m < TW; ++m) {
                if (m == em[i]) {
                    mv = mk[m];
                    esc[i] = tsv[m];
                }
            }
            ecnt[i] = em[i] >= 0 ? m3_cnt(mv) : 0;
            eoff[i] = em[i] >= 0 ? m3_off(mv) : 0;
        }
        coop_search_m<4>(ecnt, eoff, esc, p.neigh, p.neigh_len, wsm, EvalIq8{grid}, egi);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if (em[i] >= 0) {
                int gv = egi[i];
                if (gv < 0) {
                    flag_err(p);
                    gv = 0;
                }
#pragma unroll
                for (int m = 0; m < TW; ++m)
                    if (m == em[i]) gk[m] = gv;
            }
        }
    }
}

// ------------------------------------------------------------------ IQ2_XXS (gpuq/gpuq.hip:245-387)
// block: d qs[32] u16 (66 bytes); lane g = 32-weight sub-block g; q2[2g] at 2+8g, q2[2g+1] at 6+8g
struct KIQ2XXS : Iq8Tab<256> {
    static constexpr int BS = QK, G = 8, N = 32, BB = 66, NTRIAL = 13;
    static constexpr bool QUEUE = true;         // (tiles of varying cost: the tile queue)
    static constexpr int TW = 7;        // trials a window: windows 0..6 and 7..12 (the second of 6)
    // per-wave LDS: the search workspace, shared by the filtered, the 4-list, the 2-list and the 1-list searches and
    // their staged values; eight waves a workgroup share one copy of the tables (the workspace would not let two
    // four-wave workgroups share a CU's LDS)
    static constexpr int WS1 = coop_wsm_bytes<4>() > COOP_WS_BYTES ? coop_wsm_bytes<4>() : COOP_WS_BYTES;
    static constexpr int WS0 = coop_wsm_bytes<2, 16, true>() > WS1 ? coop_wsm_bytes<2, 16, true>() : WS1;
    static constexpr int WS = (((int)sizeof(FiltWS<TW>) > WS0 ? (int)sizeof(FiltWS<TW>) : WS0) + 15) & ~15;
    static constexpr int WGW = 8;
    static DEV void quant(const float (&x)[N], const float *qwp, int g, uint8_t *img, int boff, uint8_t *lds,
                          const QParams &p) {
        const uint64_t *grid = Iq8Tab<256>::grid(lds);
        const int32_t *map3 = Iq8Tab<256>::map3(lds);
        CoopWS &ws = *(CoopWS *)wave_ws<KIQ2XXS>(img);
        CoopWSM<4> &wsm = *(CoopWSM<4> *)wave_ws<KIQ2XXS>(img);
        Iq8WS2 &ws2 = *(Iq8WS2 *)wave_ws<KIQ2XXS>(img);
        FiltWS<TW> &fws = *(FiltWS<TW> *)wave_ws<KIQ2XXS>(img);
        float weight[N], xval[N];
        uint32_t bsg = 0;       // the 4 groups' 7-bit sign fields
        {
            float qv[N], sq[N];
            load_qw<N>(qwp, qv);
#pragma unroll
            for (int i = 0; i < N; ++i) sq[i] = x[i] * x[i];
            const float sigma2 = grp_chain_sum<G, N>(sq, g) / QK;
#pragma unroll
            for (int i = 0; i < N; ++i) weight[i] = qv[i] * sqrtf(sigma2 + sq[i]);
#pragma unroll
            for (int k = 0; k < 4; ++k) bsg |= signs_even8(x + 8 * k, weight + 8 * k, xval + 8 * k) << (7 * k);
        }
        float mx = xval[0];
#pragma unroll
        for (int i = 1; i < N; ++i) mx = fmax_sel(mx, xval[i]);
        float scale = 0.f, eff_max = 0.f;
        bool live = false;
        if (!(mx < EPS_GROUP)) {
            Lv<N> Lqp;
            scale = qp_levels<N>(4, xval, Lqp, weight);
            eff_max = scale * 3;
            if (eff_max <= 0) scale = 0.f;
            else live = true;
        }
        // The trials, a window of TW at a time (every lane runs them: the neighbour searches are wave-wide), group by
        // group: a group's values are staged once for the window, each trial's key on the grid is its point, and the
        // trials that share an off-grid key are searched by one filtered walk of its list (filter.cuh). A trial the
        // filter leaves undecided waits: after both windows the undecided searches of the whole tile go through the
        // exact search together (two a lane a call; an exact call costs about the same for one search as for many,
        // and a wave of 64 lanes has some undecided trial in about a third of its window-group calls). The trials'
        // grid indices are kept a byte a group (pk[t], group k at bits 8k); then the trials' sums of w*x*q and w*q*q
        // gather group by group in index order, and the acceptance chain runs over the 13 trials in ggml's order
        // (each trial's searches do not depend on another trial's outcome, so this order changes nothing). The
        // chain keeps the accepted trial (its number and scales), not its grid points.
        float best = 0;
        int tacc = -1;          // the last accepted trial (-1: none), its inverse scale and scale
        float acc_id = 0.f, acc_sc = 0.f;
        uint32_t pk[NTRIAL];
        uint64_t und = 0;       // undecided searches: group k, trial t at bit 13k + t
#pragma unroll
        for (int t = 0; t < NTRIAL; ++t) pk[t] = 0u;
        // trial t's inverse scale (as ggml forms it)
        auto trial_id = [&](int t) { return (5 + (t - 6) * 0.1f) / eff_max; };
        // (a window of W trials from trial W0: the first of TW, the second of the NTRIAL - TW left, so that no walk
        // evaluates a trial past the last)
        auto window = [&](auto wc, auto w0c) {
            constexpr int W = decltype(wc)::value, W0 = decltype(w0c)::value;
            FiltWS<W> &fw = *(FiltWS<W> *)&fws;
            float idv[W], tsv[W];
#pragma unroll
            for (int m = 0; m < W; ++m) {
                idv[m] = trial_id(W0 + m);
                tsv[m] = 1 / idv[m];
            }
            unsigned valid = 0;
#pragma unroll
            for (int m = 0; m < W; ++m)
                if (live && W0 + m < NTRIAL) valid |= 1u << m;
#pragma unroll 1
            for (int k = 0; k < 4; ++k) {       // (not unrolled: one copy of the search code, groups kept apart)
                float xk[8], waux[8];           // group k: rotated to the front (rot8 below)
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    xk[i] = xval[i];
                    waux[i] = sqrtf(weight[i]);
                }
                int gk[W];                     // the trials' grid indices of group k
                unsigned og, undec;
                window_group<W, 8, 256, true>(xk, waux, idv, tsv, valid, map3, p, grid, fw, ws, wsm, gk, og, undec);
#pragma unroll
                for (int m = 0; m < W; ++m) pk[W0 + m] |= (uint32_t)gk[m] << (8 * k);
                und |= (uint64_t)undec << (13 * k + W0);
                rot8(xval);
                rot8(weight);
            }
        };
        window(IntC<TW>{}, IntC<0>{});
        window(IntC<NTRIAL - TW>{}, IntC<TW>{});
        // the undecided searches, two a lane a call (each list with its group's values staged in its own row)
#pragma unroll 1
        while (__ballot(und != 0)) {
            int kk[2], tt[2], cnt[2], off[2], gi[2];
            float sc[2];
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int b = und ? __builtin_ctzll(und) : -1;
                und &= und - 1;
                kk[j] = b < 0 ? 0 : b / 13;
                tt[j] = b < 0 ? 0 : b - 13 * kk[j];
                float xs[8], wa[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    xs[i] = kk[j] == 0 ? xval[i] : kk[j] == 1 ? xval[8 + i] : kk[j] == 2 ? xval[16 + i] : xval[24 + i];
                    wa[i] = sqrtf(kk[j] == 0 ? weight[i] : kk[j] == 1 ? weight[8 + i] : kk[j] == 2 ? weight[16 + i]
                                                                                                  : weight[24 + i]);
                }
                const float id = trial_id(tt[j]);
                sc[j] = 1 / id;
                const int mv = b < 0 ? 0 : map3[group_key3(xs, id)];
                cnt[j] = b < 0 ? 0 : m3_cnt(mv);
                off[j] = b < 0 ? 0 : m3_off(mv);
                coop_stage<8>(ws2, xs, wa, j * 64 + lane_id());
            }
            coop_search_m<2, 4>(cnt, off, sc, p.neigh, p.neigh_len, ws2, EvalIq8{grid}, gi);
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                if (cnt[j] > 0) {
                    int gv = gi[j];
                    if (gv < 0) {
                        flag_err(p);
                        gv = 0;
                    }
#pragma unroll
                    for (int t = 0; t < NTRIAL; ++t)
                        if (t == tt[j]) pk[t] |= (uint32_t)gv << (8 * kk[j]);
                }
            }
        }
        {
            float sqx[NTRIAL], sq2[NTRIAL];
#pragma unroll
            for (int t = 0; t < NTRIAL; ++t) sqx[t] = sq2[t] = 0.f;
#pragma unroll 1
            for (int k = 0; k < 4; ++k) {       // group by group, in index order (group k rotated to the front)
#pragma unroll
                for (int t = 0; t < NTRIAL; ++t) sums_q8(weight, xval, grid[(pk[t] >> (8 * k)) & 255u], sqx[t], sq2[t]);
                rot8(xval);
                rot8(weight);
            }
            // the acceptance chain over the trials, in ggml's order
#pragma unroll
            for (int t = 0; t < NTRIAL; ++t) {
                if (live && sq2[t] > 0 && sqx[t] * sqx[t] > best * sq2[t]) {
                    scale = sqx[t] / sq2[t];
                    best = scale * sqx[t];
                    tacc = t;
                }
            }
        }
        if (tacc >= 0) {
            acc_id = trial_id(tacc);
            acc_sc = 1 / acc_id;
        }
        // The final pass at the chain's scale (after the trials scale > 0 unless the accepted trial's sum of w*x*q
        // was negative: either make_qp_quants' positive scale or an accepted one). A lane whose chain ended on a
        // negative scale keeps the accepted trial's grid points, found here again by the same searches at that
        // trial's scales (none accepted: the points stay 0).
        const bool fin = live && scale > 0;
        const bool alt = live && !fin && tacc >= 0;
        uint32_t P = 0;
        {
            const float id = fin ? 1 / scale : acc_id;
            const float fsc = fin ? scale : acc_sc;
            uint32_t Pf = 0;
            float sumqx = 0, sumq2 = 0;
#pragma unroll 1
            for (int h = 0; h < 2; ++h) {       // groups 2h and 2h+1 in one search call
                float wa0[8], wa1[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    wa0[i] = sqrtf(weight[i]);
                    wa1[i] = sqrtf(weight[8 + i]);
                }
                const int k3[2] = {group_key3(xval, id), group_key3(xval + 8, id)};
                int gi[2];
                bool og[2];
                group_points2_w(fin || alt, k3, map3, p, grid, xval, wa0, xval + 8, wa1, fsc, ws2, gi, og);
                Pf |= ((uint32_t)gi[0] | ((uint32_t)gi[1] << 8)) << (16 * h);
                sums_q8(weight, xval, grid[gi[0]], sumqx, sumq2);
                sums_q8(weight + 8, xval + 8, grid[gi[1]], sumqx, sumq2);
                rot8(xval);
                rot8(xval);
                rot8(weight);
                rot8(weight);
            }
            if (fin || alt) P = Pf;
            if (fin && sumq2 > 0) scale = sumqx / sumq2;
        }
        // a lane with no positive scale and no accepted trial (non-finite values or importances) keeps
        // make_qp_quants' levels (0..4), which ggml looks up in the full map: a key off the grid (or past the map)
        // is its abort, flagged here
        if (__ballot(live && !fin && tacc < 0)) {
            Lv<N> Lq;
            (void)qp_levels<N>(4, xval, Lq, weight);
            uint32_t Pq = 0;
            bool off = false;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                int u = 0;
#pragma unroll
                for (int i = 0; i < 8; ++i) u |= (int)Lq.get(8 * k + i) << (2 * i);
                int m = u < p.map_size ? p.map[u] : -1;
                if (m < 0) {
                    off = true;
                    m = 0;
                }
                Pq |= (uint32_t)m << (8 * k);
            }
            if (live && !fin && tacc < 0) {
                P = Pq;
                if (off) flag_err(p);
            }
        }
        uint32_t q2lo = 0, q2hi = 0;
        if (live) {
            if (scale < 0) {
                scale = -scale;
                bsg = (~bsg) & 0x0fffffffu;
            }
            q2lo = P;
            q2hi = bsg;
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
// The searches deal their lists in pieces of ch16 candidates: IQ2_S's one-shell lists hold 3.4 points on average
// (pieces of 2 measured 2% faster than 4, 11% faster than 8), IQ2_XS's two-shell lists more (4: 6% faster than 2)
template <int GRID> constexpr int ch16() { return GRID == 1024 ? 2 : 4; }
constexpr int IQ2XS_TW = 7;     // IQ2_XS's trial window (filtered search)
// the search workspace of the 16-weight types: T trial scales of the lane's two groups as 2T lists (list t*2 + k:
// trial t, group k), the two groups' values staged once (row k*64 + lane), one scale row a trial for T = 3
template <int T> using Iq16WST = CoopWSM<2 * T, 16, true, 2, (T == 2 ? 4 : T)>;
using Iq16WS = Iq16WST<2>;

// the two groups' grid indices of every lane at T scales (all lanes call it together): list m = t*2 + k with act[m]
// takes the grid point of group k's key at id[t] if the key is on the grid, else the winner of its neighbour list
// (the distances at scale[t]), one wave-wide call for the 2T lists (the groups' values staged beforehand). A search
// that accepts nothing flags the error (the reference traps) and yields index 0. Inactive lists get 0.
template <int GRID, int T = 2>
DEV void iq2_16_points(const bool (&act)[2 * T], const float (&id)[T], const float (&scale)[T],
                       const float (&xval)[16], const int32_t *map3, const QParams &p, const uint64_t *grid,
                       Iq16WST<T> &ws, int (&gi)[2 * T], bool (&og)[2 * T]) {
    constexpr int M = 2 * T;
    int mk[M], cnt[M], off[M], g[M];
    float sc[M];
#pragma unroll
    for (int m = 0; m < M; ++m) {
        mk[m] = act[m] ? map3[group_key3(xval + 8 * (m & 1), id[m >> 1])] : 0;
        og[m] = mk[m] >= 0;
        cnt[m] = act[m] && mk[m] < 0 ? m3_cnt(mk[m]) : 0;
        off[m] = act[m] && mk[m] < 0 ? m3_off(mk[m]) : 0;
        sc[m] = scale[m >> 1];
    }
    coop_search_m<M, ch16<GRID>()>(cnt, off, sc, p.neigh, p.neigh_len, ws, EvalIq8{grid}, g);
#pragma unroll
    for (int m = 0; m < M; ++m) {
        gi[m] = mk[m];
        if (act[m] && mk[m] < 0) {
            gi[m] = g[m];
            if (g[m] < 0) {
                flag_err(p);
                gi[m] = 0;
            }
        }
    }
}

// IQ2_S (GRID 1024) searches three trials a call (Iq16WST<3>), IQ2_XS two (Iq16WS)
template <int GRID> using Iq16WSOf = Iq16WST<GRID == 1024 ? 3 : 2>;
template <bool PARITY, int GRID>
DEV float iq2_16_search(const float (&x)[16], const float (&qv)[16], float sigma2, float eps, const QParams &p,
                        const uint8_t *lds, Iq16WSOf<GRID> &ws, int (&gidx)[2], uint32_t (&bsg)[2], bool &live) {
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
    // every lane runs the trials (the neighbour search is wave-wide); only live lanes use them
    float best = 0;
    float scale = mx / 5;
    int P[2] = {-1, -1};        // accepted trial's groups as grid indices; -1: all levels 0 (no trial accepted yet)
    bool on_grid[2] = {true, true};
    if constexpr (GRID == 512) {
        // IQ2_XS (two-shell lists, 12.9 points on average): the 19 trials in windows of TW, group by group, through
        // the filtered search (window_group; the trials it leaves undecided searched once a window, after both
        // groups' walks), and the acceptance chain over each window from the trials' sums; the chain keeps the
        // accepted trial (number, scales, which groups were on the grid), and the pass below finds its points again:
        // on the grid from their keys, off the grid by the same searches (IQ2_XXS's scheme, KIQ2XXS::quant)
        constexpr int TW = IQ2XS_TW, NT = 19;
        FiltWS<TW> &fws = *(FiltWS<TW> *)&ws;
        CoopWS &ws1 = *(CoopWS *)&ws;
        CoopWSM<4> &wsm = *(CoopWSM<4> *)&ws;
        int tacc = -1;
        float acc_id = 0.f, acc_sc = 0.f;
        unsigned acc_og = 3u;
        // (a window of W trials from trial w0: two of TW, then one of the NT - 2 TW left, so that no walk evaluates a
        // trial past the last)
        auto window = [&](auto wc, int w0) {
            constexpr int W = decltype(wc)::value;
            FiltWS<W> &fw = *(FiltWS<W> *)&fws;
            float idv[W], tsv[W], sqx[W], sq2[W];
            unsigned valid = 0;
#pragma unroll
            for (int m = 0; m < W; ++m) {
                idv[m] = (5 + (w0 + m - 9) * 0.1f) / mx;
                tsv[m] = 1 / idv[m];
                sqx[m] = sq2[m] = 0.f;
                if (live && w0 + m < NT) valid |= 1u << m;
            }
            // the window's grid indices, group k at bits 9k; the trials the filter leaves undecided (group k, trial
            // m at bit 8k + m) are searched after both groups' walks, four a lane a call (two of each group)
            unsigned ogk[2], und = 0;
            uint32_t pk[W];
#pragma unroll
            for (int m = 0; m < W; ++m) pk[m] = 0u;
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                float xk[8], wk[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    xk[i] = xval[8 * k + i];
                    wk[i] = waux[8 * k + i];
                }
                int gk[W];
                unsigned undec;
                window_group<W, 9, 512, true>(xk, wk, idv, tsv, valid, map3, p, grid, fw, ws1, wsm, gk, ogk[k],
                                              undec);
#pragma unroll
                for (int m = 0; m < W; ++m) pk[m] |= (uint32_t)gk[m] << (9 * k);
                und |= undec << (8 * k);
            }
            if (__ballot(und != 0)) {
#pragma unroll
                for (int k = 0; k < 2; ++k) coop_stage<8>(ws, xval + 8 * k, waux + 8 * k, k * 64 + lane_id());
            }
#pragma unroll 1
            while (__ballot(und != 0)) {
                int cnt[4], off[4], gi[4], tm[4];
                float sc[4];
#pragma unroll
                for (int j = 0; j < 4; ++j) {           // list j searches for group j & 1 (its staged row)
                    const int k = j & 1;
                    const unsigned u = (und >> (8 * k)) & 0xffu;
                    const int m = u ? __builtin_ctz(u) : -1;
                    if (m >= 0) und &= ~(1u << (8 * k + m));
                    tm[j] = m;
                    float id = idv[0];
                    sc[j] = tsv[0];
#pragma unroll
                    for (int mm = 0; mm < W; ++mm) {
                        if (mm == m) {
                            id = idv[mm];
                            sc[j] = tsv[mm];
                        }
                    }
                    const int mv = m < 0 ? 0 : map3[group_key3(xval + 8 * k, id)];
                    cnt[j] = m < 0 ? 0 : m3_cnt(mv);
                    off[j] = m < 0 ? 0 : m3_off(mv);
                }
                coop_search_m<4, ch16<GRID>()>(cnt, off, sc, p.neigh, p.neigh_len, ws, EvalIq8{grid}, gi);
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    if (cnt[j] > 0) {
                        int gv = gi[j];
                        if (gv < 0) {
                            flag_err(p);
                            gv = 0;
                        }
#pragma unroll
                        for (int mm = 0; mm < W; ++mm)
                            if (mm == tm[j]) pk[mm] |= (uint32_t)gv << (9 * (j & 1));
                    }
                }
            }
#pragma unroll
            for (int k = 0; k < 2; ++k) {
#pragma unroll
                for (int m = 0; m < W; ++m)
                    sums_q8(weight + 8 * k, xval + 8 * k, grid[(pk[m] >> (9 * k)) & 511u], sqx[m], sq2[m]);
            }
#pragma unroll
            for (int m = 0; m < W; ++m) {
                if (w0 + m < NT && live && sq2[m] > 0 && sqx[m] * sqx[m] > best * sq2[m]) {
                    scale = sqx[m] / sq2[m];
                    best = scale * sqx[m];
                    tacc = w0 + m;
                    acc_id = idv[m];
                    acc_sc = tsv[m];
                    acc_og = ((ogk[0] >> m) & 1u) | (((ogk[1] >> m) & 1u) << 1);
                }
            }
        };
        static_assert(NT > 2 * TW && NT <= 3 * TW, "windows: two of TW and the rest");
#pragma unroll 1
        for (int w0 = 0; w0 < 2 * TW; w0 += TW) window(IntC<TW>{}, w0);
        window(IntC<NT - 2 * TW>{}, 2 * TW);
        on_grid[0] = (acc_og & 1u) != 0;
        on_grid[1] = (acc_og & 2u) != 0;
        // (a group left at levels 0 is on the grid: on_grid stays true for it)
        const bool fin = live && (!on_grid[0] || !on_grid[1]) && scale > 0;
        const bool alt = live && !fin && tacc >= 0;        // the accepted trial's points, found again
#pragma unroll
        for (int k = 0; k < 2; ++k) coop_stage<8>(ws, xval + 8 * k, waux + 8 * k, k * 64 + lane_id());
        {
            const float idf = fin ? 1 / scale : acc_id, scf = fin ? scale : acc_sc;
            const float id[2] = {idf, idf}, fsc[2] = {scf, scf};
            const bool act[4] = {(fin || alt) && !on_grid[0], (fin || alt) && !on_grid[1], false, false};
            int gi[4];
            bool og[4];
            iq2_16_points<GRID>(act, id, fsc, xval, map3, p, grid, ws, gi, og);
            float sumqx = 0, sumq2 = 0;
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                if (act[k]) P[k] = gi[k];
                else if (tacc >= 0) P[k] = map3[group_key3(xval + 8 * k, acc_id)];   // (on the grid)
                sums_q8(weight + 8 * k, xval + 8 * k, grid[P[k] < 0 ? 0 : P[k]], sumqx, sumq2);
            }
            if (fin && sumq2 > 0) scale = sumqx / sumq2;
        }
    } else {
    // the two groups' values, staged once for all the trials and the final pass
#pragma unroll
    for (int k = 0; k < 2; ++k) coop_stage<8>(ws, xval + 8 * k, waux + 8 * k, k * 64 + lane_id());
    // the 19 trials three a call (the last call has one: a wave-wide call costs much the same for few lists as for
    // many), accepted in trial order
    constexpr int TC = 3;
#pragma unroll 1
    for (int is = -9; is <= 9; is += TC) {
        const int nt = 10 - is < TC ? 10 - is : TC;     // trials is .. is + nt - 1 (wave-uniform)
        float id[TC], tsc[TC];
        bool act[2 * TC];
#pragma unroll
        for (int t = 0; t < TC; ++t) {
            id[t] = (5 + (is + t) * 0.1f) / mx;
            tsc[t] = 1 / id[t];
            act[2 * t] = act[2 * t + 1] = live && t < nt;
        }
        int Pa[2 * TC];
        bool og[2 * TC];
        iq2_16_points<GRID, TC>(act, id, tsc, xval, map3, p, grid, ws, Pa, og);
#pragma unroll
        for (int t = 0; t < TC; ++t) {
            if (t >= nt) break;
            float sumqx = 0, sumq2 = 0;
#pragma unroll
            for (int k = 0; k < 2; ++k) sums_q8(weight + 8 * k, xval + 8 * k, grid[Pa[2 * t + k]], sumqx, sumq2);
            if (live && sumq2 > 0 && sumqx * sumqx > best * sumq2) {
                scale = sumqx / sumq2;
                best = scale * sumqx;
                P[0] = Pa[2 * t];
                P[1] = Pa[2 * t + 1];
                on_grid[0] = og[2 * t];
                on_grid[1] = og[2 * t + 1];
            }
        }
    }
    // (a group left at levels 0 is on the grid: on_grid stays true for it)
    const bool fin = live && (!on_grid[0] || !on_grid[1]) && scale > 0;
    {
        const float id[TC] = {1 / scale, 1 / scale, 1 / scale}, fsc[TC] = {scale, scale, scale};
        const bool act[2 * TC] = {fin && !on_grid[0], fin && !on_grid[1], false, false, false, false};
        int gi[2 * TC];
        bool og[2 * TC];
        iq2_16_points<GRID, TC>(act, id, fsc, xval, map3, p, grid, ws, gi, og);
        float sumqx = 0, sumq2 = 0;
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            if (act[k]) P[k] = gi[k];
            sums_q8(weight + 8 * k, xval + 8 * k, grid[P[k] < 0 ? 0 : P[k]], sumqx, sumq2);
        }
        if (fin && sumq2 > 0) scale = sumqx / sumq2;
    }
    }
    if (!live) return 0.f;
    if (scale < 0) {
        scale = -scale;
#pragma unroll
        for (int k = 0; k < 2; ++k) bsg[k] = PARITY ? ((~bsg[k]) & 127) : ((~bsg[k]) & 255);
    }
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        if (P[k] < 0) {                         // levels 0: the all-ones point's index from the full map
            P[k] = p.map[0];
            if (P[k] < 0) { flag_err(p); P[k] = 0; }
        }
        gidx[k] = P[k];
    }
    return scale;
}

// IQ2_S: block d qs[64] (32 grid bytes, 32 sign bytes) qh[8] scales[8] (82 bytes); lane g = 16-weight sub-block g
struct KIQ2S : Iq8Tab<1024> {
    static constexpr int BS = QK, G = 16, N = 16, BB = 82, WS = (int)sizeof(Iq16WSOf<1024>), WGW = 8;
    static constexpr bool QUEUE = true;         // (tiles of varying cost: the tile queue)
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
        const float scale = iq2_16_search<false, 1024>(x, qv, sigma2, EPS_IQ2S, p, lds,
                                                       *(Iq16WSOf<1024> *)wave_ws<KIQ2S>(img), gidx, bsg, live);
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
    static constexpr int WS0 = coop_wsm_bytes<4, 16, true, 2>();
    static constexpr bool QUEUE = true;         // (tiles of varying cost: the tile queue)
    static constexpr int BS = QK, G = 16, N = 16, BB = 74, WGW = 8,
                         WS = (((int)sizeof(FiltWS<IQ2XS_TW>) > WS0 ? (int)sizeof(FiltWS<IQ2XS_TW>) : WS0) + 15) & ~15;
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
        const float scale = iq2_16_search<true, 512>(x, qv, sigma2, EPS_GROUP, p, lds,
                                                     *(Iq16WS *)wave_ws<KIQ2XS>(img), gidx, bsg, live);
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
