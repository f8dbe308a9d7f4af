// trench-gguf_amd/csrc/iq1.cuh - IQ1_S and IQ1_M on gfx950.
//
// Semantics: ggml's quantize_row_iq1_s_impl / quantize_row_iq1_m_impl as the reference restates them
// (gpuq/gpuq.hip:199-232, 389-688). Per lane: one 32-weight (IQ1_S) or 16-weight (IQ1_M) block.
//  - The stable sort by value is computed as ranks, rank_i = #{j < i: x_j <= x_i} + #{j > i: x_j < x_i}, which is
//    the position of element i in glibc's stable order; the prefix sums then run in that order, serially, as ggml's.
//  - The (i1, i2) partition search runs every candidate in ggml's order on the lane, so its cross-multiplied
//    acceptance chain is ggml's exactly. Its loop indices are wave-uniform, so the prefix arrays are indexed through
//    uniform (M0-relative) register addressing. IQ1_M first ranks the candidates by an approximate score, without
//    branches; where the best stands clear of the rest by more than the rounding can move them, it is the chain's
//    last accept (iq1_rank_ok), and only the other lanes run the chain.
//  - IQ1_M's final least-squares d over all 256 weights is a lane-to-lane chain in ggml's index order.
//  - The neighbour searches of the final points run wave-wide (coop.cuh), so every lane takes part in them.
// Tables: the 2048-point IQ1 grid and its base-3 key map in LDS (the IQ1 levels are always 0..2), lists in HBM.
#pragma once
#include "iq2.cuh"

#define EPS_IQ1S 1e-12f
#define EPS_IQ1M 1e-7f
#define IQ1_DELTA 0.125f

// x_p = {-1+d, d, 1+d}, x_m = {-1-d, -d, 1-d}: the value of level l (0..2) for shift +1 / -1
DEV float iq1_val(int l, bool minus) {
    const float a = minus ? -1 - IQ1_DELTA : -1 + IQ1_DELTA;
    const float b = minus ? -IQ1_DELTA : IQ1_DELTA;
    const float c = minus ? 1 - IQ1_DELTA : 1 + IQ1_DELTA;
    return l == 0 ? a : (l == 1 ? b : c);
}

// iq1_find_best_neighbour2's distance of one grid point (gpuq/gpuq.hip:199-232) for an owner's staged values
// (st[0..7] the x's, st[8..15] the weights), in the serial scan's operation order. The owner's shift rides on the
// sign of its (positive) scale; a level's value (l - 1) +- 1/8 = b/2 - 3/2 +- 1/8 from the point byte b = 2l + 1 is
// exact in float, so it equals ggml's table entry. (A key with no finite distance makes the reference scan the whole
// grid with an out-of-block read; the caller reports it as an error.)
struct EvalIq1 {
    const uint64_t *grid;
    DEV uint64_t point(int idx) const { return grid[idx]; }
    DEV float operator()(const float *st, float ssc, uint64_t pt) const {
        const float scale = fabsf(ssc);
        const float c = ssc < 0 ? -1.5f - IQ1_DELTA : -1.5f + IQ1_DELTA;
        const uint32_t lo = (uint32_t)pt, hi = (uint32_t)(pt >> 32);
        float d2 = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float q = (float)(((i < 4 ? lo : hi) >> (8 * (i % 4))) & 0xffu) * 0.5f + c;
            const float diff = scale * q - st[i];
            d2 += st[8 + i] * diff * diff;
        }
        return d2;
    }
};

// Two groups' grid points on every lane of the wave (all lanes call it together; live as the caller has it): a key
// on the grid directly, else the cooperative search over its list, both groups' lists in one wave-wide call (two
// lists a lane, each with its group's staged values, row k*64 + lane). gi[k] is 0 for a lane that is not live; a
// search that accepts nothing is flagged and yields 0. og[k]: no search was needed.
using Iq1WS = CoopWSM<2, 16, true>;
static_assert(sizeof(Iq1WS) >= 17 * 64 * sizeof(float2), "the rank-order slots fit the search workspace");
DEV void iq1_group_points2(bool live, const int (&m)[2], const float *x0, const float *w0, const float *x1,
                           const float *w1, float scale, const bool (&minus)[2], const QParams &p,
                           const uint64_t *grid, Iq1WS &ws, int (&gi)[2], bool (&og)[2]) {
    int cnt[2], off[2], g[2];
    float ssc[2];
    bool neg = false;                   // (a negative importance: distances of any sign, see coop.cuh)
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const float *xk = k ? x1 : x0, *wk = k ? w1 : w0;
        const bool srch = live && m[k] < 0;
        og[k] = !srch;
        cnt[k] = srch ? m3_cnt(m[k]) : 0;
        off[k] = srch ? m3_off(m[k]) : 0;
        ssc[k] = minus[k] ? -scale : scale;
        if (srch) coop_stage<8>(ws, xk, wk, k * 64 + lane_id());
#pragma unroll
        for (int i = 0; i < 8; ++i) neg = neg || (srch && wk[i] < 0.f);
    }
    if (__ballot(neg)) coop_search_m<2, 4, true, true>(cnt, off, ssc, p.neigh, p.neigh_len, ws, EvalIq1{grid}, g);
    else coop_search_m<2, 4, false, true>(cnt, off, ssc, p.neigh, p.neigh_len, ws, EvalIq1{grid}, g);
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        gi[k] = 0;
        if (!live) continue;
        if (og[k]) {
            gi[k] = m[k];
        } else if (g[k] < 0) {
            flag_err(p);
        } else {
            gi[k] = g[k];
        }
    }
}

// Whether IQ1_S's partition scan may drop its `sumq2 > 0` test: a candidate's sumq2 is
// a_w x0^2 + (s2w - s1w) x1^2 + (totw - s2w) x2^2 over the weights' prefix sums, three terms >= 0 that split totw, so
// with every weight 0 or in [2^-100, 2^100] (no underflow or overflow on the way) it is > 0 exactly when the block's
// weights are not all 0, and a block of zero weights never accepts. The test is dropped when every scanning lane of
// the wave qualifies (wave-uniform: one scan variant a wave); a lane of zero weights then starts from best = +inf,
// which rejects every candidate as the test did (sumq2 = 0: inf * 0 is NaN). (IQ1_M keeps its single scan: the
// same change measured slower there, its loop's register allocation being the cost.)
template <bool B> struct ScanTest { static constexpr bool q2 = B; };
template <int N> DEV bool iq1_weights_plain(const float (&w)[N], bool &any) {
    bool ok = true;
    any = false;
#pragma unroll
    for (int i = 0; i < N; ++i) {
        ok = ok && (w[i] == 0.f || (w[i] >= 0x1p-100f && w[i] <= 0x1p100f));
        any = any || w[i] > 0.f;
    }
    return ok;
}

// Whether IQ1_M's ranking pass settles a lane's partition scan. ggml's chain accepts a candidate c when
// fl(sumqx_c^2) > fl(best * sumq2_c), best = fl(fl(sumqx_r / sumq2_r) * sumqx_r) of the last accepted r (at first
// -FLT_MAX); with T(c) = sumqx_c^2 / sumq2_c over the candidates' own float sums, that test reads
// T(c) (1 + e) > T(r) (1 + e1) (1 + e2) (1 + e3), |e*| <= u = 2^-24, while the products stay in the normal range.
// The ranking pass's score A(c) = fl(fl(sumqx_c^2) rcp(sumq2_c)) is T(c) within 4u (rcp: 1 ulp). If the largest
// score S1 exceeds the second S2 by the factor fl(1 + 2^-20) (at least 1 + 15u), its candidate c* has
// T(c*) > T(c) (1 + 6u) for every other c: the chain accepts c* when it reaches it (whatever record precedes it) and
// nothing after it, so c* is the last accept, and its scale is fl(sumqx* / sumq2*) as the chain computes it. The
// range conditions: weights 0 or in [2^-100, 2^100] with a total in [2^-40, 2^40] (every sumq2 is then >= 2^-47: each
// weight's q^2 is >= 1/64, the sums' rounding far below that, so every candidate has sumq2 > 0 as the chain requires),
// max|x| * total <= 2^50 (sumqx^2 <= 2^101 and best * sumq2 <= 81 sumqx*^2: no overflow), and S1 in [2^-60, 2^100]
// (the comparisons that accept c* or reject the candidates after it stay normal; a losing candidate's square may
// underflow, which only lowers it). A lane outside them, or whose top two are closer (near ties, exact ties from zero
// weights), replays the chain.
DEV bool iq1_rank_ok(bool wplain, float totw, float mx, float S1, float S2) {
    return wplain && totw >= 0x1p-40f && totw <= 0x1p40f && mx * totw <= 0x1p50f && S1 >= 0x1p-60f &&
           S1 <= 0x1p100f && S1 > S2 * (1.f + 0x1p-20f);
}

// position of element i in the stable ascending order of x
template <int N> DEV void stable_ranks(const float (&x)[N], Lv<N> &R) {
#pragma unroll
    for (int i = 0; i < N; ++i) {
        int r = 0;
#pragma unroll
        for (int j = 0; j < N; ++j) {
            if (j < i) r += x[j] <= x[i];
            else if (j > i) r += x[j] < x[i];
        }
        R.put(i, (uint32_t)r);
    }
}

// 2-sum chain over the group in lane (index) order
template <int G, int N> DEV void grp_chain_sum2(const float (&a)[N], const float (&b)[N], int g, float &sa, float &sb) {
    float acc_a = 0.f, acc_b = 0.f;
#pragma unroll
    for (int j = 0; j < G; ++j) {
        float ta = acc_a, tb = acc_b;
        if (g == j) {
#pragma unroll
            for (int i = 0; i < N; ++i) { ta += a[i]; tb += b[i]; }
        }
        acc_a = grp_bcast<G>(ta, j);
        acc_b = grp_bcast<G>(tb, j);
    }
    sa = acc_a;
    sb = acc_b;
}

// ------------------------------------------------------------------ IQ1_S (gpuq/gpuq.hip:389-514)
// block: d qs[32] qh[8] u16 (50 bytes); lane g = 32-weight block g
struct KIQ1S : Iq8Tab<2048> {
    static constexpr int BS = QK, G = 8, N = 32, BB = 50, WS = coop_wsm_bytes<2, 16, true>(), WGW = 8;
    static constexpr bool QUEUE = true;         // (tiles of varying cost: the tile queue)
    static DEV void quant(const float (&x)[N], const float *qwp, int g, uint8_t *img, int boff, uint8_t *lds,
                          const QParams &p) {
        const uint64_t *grid = Iq8Tab<2048>::grid(lds);
        const int32_t *map3 = Iq8Tab<2048>::map3(lds);
        const float xp0 = -1 + IQ1_DELTA, xp1 = IQ1_DELTA, xp2 = 1 + IQ1_DELTA;
        const float xm0 = -1 - IQ1_DELTA, xm1 = -IQ1_DELTA, xm2 = 1 - IQ1_DELTA;
        float qv[N], sq[N], weight[N];
        load_qw<N>(qwp, qv);
#pragma unroll
        for (int i = 0; i < N; ++i) sq[i] = x[i] * x[i];
        const float sigma2 = 2 * grp_chain_sum<G, N>(sq, g) / QK;
#pragma unroll
        for (int i = 0; i < N; ++i) weight[i] = qv[i] * sqrtf(sigma2 + sq[i]);
        float mx = fabsf(x[0]);
#pragma unroll
        for (int i = 1; i < N; ++i) mx = fmax_sel(mx, fabsf(x[i]));
        bool live = false, minus = false;
        float scale = 0.f;
        int gi4[4] = {0, 0, 0, 0}, m4[4] = {0, 0, 0, 0};
        Iq1WS &ws = *(Iq1WS *)wave_ws<KIQ1S>(img);
        bool wany;
        const bool wplain = iq1_weights_plain<N>(weight, wany);
        const bool q2pos = !__ballot(!(mx < EPS_IQ1S) && !wplain);     // (wave-uniform)
        if (!(mx < EPS_IQ1S)) {
            Lv<N> R;
            stable_ranks<N>(x, R);
            // prefix sums 0..N: entries 0..N-1 in 32-register arrays (their loop-uniform indexing stays in registers;
            // a 33-entry array would not) and entry N, the totals, apart
            float sumx[N], sumw[N], totx, totw;
            sumx[0] = sumw[0] = 0;
            {
                // the elements in rank order through LDS: each element's (w*x, w) goes to its rank's slot of this
                // lane's column of the wave's search workspace (unused until the searches below), then the slots are
                // read back in rank order; 16 ranks a pass, the other pass's elements written to a 17th slot
                float2 *slots = (float2 *)&ws;
                const int lane = lane_id();
#pragma unroll
                for (int h = 0; h < 2; ++h) {
#pragma unroll
                    for (int i = 0; i < N; ++i) {
                        const int r = (int)R.get(i) - 16 * h;
                        slots[((unsigned)r < 16u ? r : 16) * 64 + lane] = make_float2(weight[i] * x[i], weight[i]);
                    }
                    wave_sync();
#pragma unroll
                    for (int jj = 0; jj < 16; ++jj) {
                        const int j = 16 * h + jj;
                        const float2 v = slots[jj * 64 + lane];
                        if (j + 1 < N) {
                            sumx[j + 1] = sumx[j] + v.x;
                            sumw[j + 1] = sumw[j] + v.y;
                        } else {
                            totx = sumx[j] + v.x;
                            totw = sumw[j] + v.y;
                        }
                    }
                    wave_sync();
                }
            }
            scale = mx;
            int bidx = -1;            // the accepted candidate: i1 << 8 | i2 << 1 | (shift -1)
            auto scan = [&](auto tst) {
                constexpr bool TQ2 = decltype(tst)::q2;
                float best_score = TQ2 || wany ? -FLT_MAX : __builtin_inff();
                for (int i1 = 0; i1 <= N; ++i1) {
                    const float s1x = i1 < N ? sumx[i1 & (N - 1)] : totx, s1w = i1 < N ? sumw[i1 & (N - 1)] : totw;
                    const float a_x = s1x - sumx[0], a_w = s1w - sumw[0];
                    for (int i2 = i1; i2 <= N; ++i2) {
                        const float s2x = i2 < N ? sumx[i2 & (N - 1)] : totx;
                        const float s2w = i2 < N ? sumw[i2 & (N - 1)] : totw;
                        const int id = (i1 << 8) | (i2 << 1);
                        float sumqx = a_x * xp0 + (s2x - s1x) * xp1 + (totx - s2x) * xp2;
                        float sumq2 = a_w * xp0 * xp0 + (s2w - s1w) * xp1 * xp1 + (totw - s2w) * xp2 * xp2;
                        if ((!TQ2 || sumq2 > 0) & (sumqx * sumqx > best_score * sumq2)) {   // (one branch, both tests)
                            scale = sumqx / sumq2;
                            best_score = scale * sumqx;
                            bidx = id;
                        }
                        sumqx = a_x * xm0 + (s2x - s1x) * xm1 + (totx - s2x) * xm2;
                        sumq2 = a_w * xm0 * xm0 + (s2w - s1w) * xm1 * xm1 + (totw - s2w) * xm2 * xm2;
                        if ((!TQ2 || sumq2 > 0) & (sumqx * sumqx > best_score * sumq2)) {
                            scale = sumqx / sumq2;
                            best_score = scale * sumqx;
                            bidx = id | 1;
                        }
                    }
                }
            };
            if (q2pos) scan(ScanTest<false>{});
            else scan(ScanTest<true>{});
            if (bidx < 0) {
                scale = 0.f;
            } else {
                const int besti1 = bidx >> 8, besti2 = (bidx >> 1) & 127;
                int best_shift = bidx & 1 ? -1 : 1;
                live = true;
                const bool flip = scale < 0;
                if (flip) { scale = -scale; best_shift = -best_shift; }
                minus = best_shift != 1;
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    int k3 = 0, p3 = 1;
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        const int r = (int)R.get(8 * k + j);
                        int l = r < besti1 ? 0 : (r < besti2 ? 1 : 2);
                        if (flip) l = 2 - l;
                        k3 += l * p3;
                        p3 *= 3;
                    }
                    m4[k] = map3[k3];
                }
            }
        }
        // the groups' points (every lane: the neighbour search is wave-wide), two groups a call
        bool all_on_grid = true;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int mk[2] = {m4[2 * h], m4[2 * h + 1]};
            const bool mn[2] = {minus, minus};
            int gi[2];
            bool og[2];
            iq1_group_points2(live, mk, x + 16 * h, weight + 16 * h, x + 16 * h + 8, weight + 16 * h + 8, scale, mn, p,
                              grid, ws, gi, og);
            gi4[2 * h] = gi[0];
            gi4[2 * h + 1] = gi[1];
            all_on_grid = all_on_grid && og[0] && og[1];
        }
        if (live) {
            {
                if (!all_on_grid) {
                    float sumqx = 0, sumq2 = 0;
#pragma unroll
                    for (int k = 0; k < 4; ++k) {
                        const uint64_t pt = grid[gi4[k]];
#pragma unroll
                        for (int j = 0; j < 8; ++j) {
                            const int b = (int)((pt >> (8 * j)) & 0xffu);
                            const float w = weight[8 * k + j];
                            const float q = iq1_val((b - 1) / 2, minus);
                            sumqx += w * q * x[8 * k + j];
                            sumq2 += w * q * q;
                        }
                    }
                    if (sumqx > 0 && sumq2 > 0) scale = sumqx / sumq2;
                }
            }
        }
        uint32_t h = 0;
        if (live) {
            img_or32(img, boff + 2 + 4 * g, (uint32_t)(gi4[0] & 255) | ((uint32_t)(gi4[1] & 255) << 8) |
                                               ((uint32_t)(gi4[2] & 255) << 16) | ((uint32_t)(gi4[3] & 255) << 24));
#pragma unroll
            for (int k = 0; k < 4; ++k) h |= (uint32_t)(gi4[k] >> 8) << (3 * k);
        }
        const float max_scale = grp_max<G>(scale);
        if (max_scale) {
            const float d = max_scale / 15;
            if (g == 0) img_or16(img, boff, f2h(d * 1.125f));
            const float id = 1 / d;
            int l = imax(0, imin(7, nint(0.5f * (id * scale - 1))));
            if (live && minus) l |= 8;
            h |= (uint32_t)l << 12;
        }
        img_or16(img, boff + 34 + 2 * g, h & 0xffffu);
    }
};

// ------------------------------------------------------------------ IQ1_M (gpuq/gpuq.hip:516-688)
// The sums of one (i1, i2) candidate of IQ1_M's partition scan for its four shift combinations k (bit 1: the first
// half's shift is -1, bit 0: the second half's), from the halves' prefix sums at i1 (a*) and i2 (b*) and their totals
// (t*), in the operation order of gpuq/gpuq.hip:579-604
DEV void iq1m_sums(float a0x, float a1x, float a0w, float a1w, float b0x, float b1x, float b0w, float b1w, float txs0,
                   float txs1, float tws0, float tws1, float (&sumqx)[4], float (&sumq2)[4]) {
    const float xp0 = -1 + IQ1_DELTA, xp1 = IQ1_DELTA, xp2 = 1 + IQ1_DELTA;
    const float xm0 = -1 - IQ1_DELTA, xm1 = -IQ1_DELTA, xm2 = 1 - IQ1_DELTA;
    const float p2 = xp2, m2 = xm2;
    const float cp1 = xp0 * xp0 - xp1 * xp1, cp2 = xp1 * xp1 - xp2 * xp2;
    const float cm1 = xm0 * xm0 - xm1 * xm1, cm2 = xm1 * xm1 - xm2 * xm2;
    float qx_p[2], qx_m[2], q2_p[2], q2_m[2];
    {
        const float sx = a0x + b0x;
        qx_p[0] = txs0 * p2 - sx;
        qx_m[0] = txs0 * m2 - sx;
        q2_p[0] = tws0 * p2 * p2 + a0w * cp1 + b0w * cp2;
        q2_m[0] = tws0 * m2 * m2 + a0w * cm1 + b0w * cm2;
    }
    {
        const float sx = a1x + b1x;
        qx_p[1] = txs1 * p2 - sx;
        qx_m[1] = txs1 * m2 - sx;
        q2_p[1] = tws1 * p2 * p2 + a1w * cp1 + b1w * cp2;
        q2_m[1] = tws1 * m2 * m2 + a1w * cm1 + b1w * cm2;
    }
    sumqx[0] = qx_p[0] + qx_p[1];
    sumqx[1] = qx_p[0] + qx_m[1];
    sumqx[2] = qx_m[0] + qx_p[1];
    sumqx[3] = qx_m[0] + qx_m[1];
    sumq2[0] = q2_p[0] + q2_p[1];
    sumq2[1] = q2_p[0] + q2_m[1];
    sumq2[2] = q2_m[0] + q2_p[1];
    sumq2[3] = q2_m[0] + q2_m[1];
}

// block: qs[32] qh[16] scales[8] (56 bytes); lane g = 16-weight block g
struct KIQ1M : Iq8Tab<2048> {
    static constexpr int BS = QK, G = 16, N = 16, BB = 56, WS = coop_wsm_bytes<2, 16, true>(), WGW = 8;
    static constexpr bool QUEUE = true;         // (tiles of varying cost: the tile queue)
    static DEV void quant(const float (&x)[N], const float *qwp, int g, uint8_t *img, int boff, uint8_t *lds,
                          const QParams &p) {
        const uint64_t *grid = Iq8Tab<2048>::grid(lds);
        const int32_t *map3 = Iq8Tab<2048>::map3(lds);
        float qv[N], sq[N], weight[N];
        load_qw<N>(qwp, qv);
#pragma unroll
        for (int i = 0; i < N; ++i) sq[i] = x[i] * x[i];
        const float sigma2 = 2 * grp_chain_sum<G, N>(sq, g) / QK;
#pragma unroll
        for (int i = 0; i < N; ++i) weight[i] = qv[i] * sqrtf(sigma2 + sq[i]);
        float mx = fabsf(x[0]);
#pragma unroll
        for (int i = 1; i < N; ++i) mx = fmax_sel(mx, fabsf(x[i]));
        bool live = false;
        int best_k = 0;       // the shift combination (0 for a skipped block, masks[0] = 0)
        float scale = 0.f;
        int gi2[2] = {0, 0}, mk2[2] = {0, 0};
        Iq1WS &ws = *(Iq1WS *)wave_ws<KIQ1M>(img);
        if (!(mx < EPS_IQ1M)) {
            Lv<N> R;
            stable_ranks<N>(x, R);
            float px0[N + 1], px1[N + 1], pw0[N + 1], pw1[N + 1];
            px0[0] = px1[0] = 0;
            pw0[0] = pw1[0] = 0;
            {
                // the elements in rank order through LDS (as IQ1_S's prefix sums), with a mask of the ranks whose
                // element lies in the second half
                float2 *slots = (float2 *)&ws;
                const int lane = lane_id();
                uint32_t hm = 0;
#pragma unroll
                for (int i = 0; i < N; ++i) {
                    const uint32_t r = R.get(i);
                    slots[r * 64 + lane] = make_float2(weight[i] * x[i], weight[i]);
                    if (i >= N / 2) hm |= 1u << r;
                }
                wave_sync();
#pragma unroll
                for (int j = 0; j < N; ++j) {
                    const float2 v = slots[j * 64 + lane];
                    const int hsel = (int)((hm >> j) & 1u);
                    px0[j + 1] = hsel == 0 ? px0[j] + v.x : px0[j];
                    px1[j + 1] = hsel == 1 ? px1[j] + v.x : px1[j];
                    pw0[j + 1] = hsel == 0 ? pw0[j] + v.y : pw0[j];
                    pw1[j + 1] = hsel == 1 ? pw1[j] + v.y : pw1[j];
                }
                wave_sync();
            }
            const float txs0 = px0[N], txs1 = px1[N], tws0 = pw0[N], tws1 = pw1[N];
            scale = mx;
            int besti1 = -1, besti2 = -1, bk = -1;
            // The ranking pass (see iq1_rank_ok): every candidate's score sumqx^2 / sumq2 approximated without a
            // branch, the two largest kept with the largest's candidate; a lane whose largest stands clear of the
            // second takes it as the chain's last accept, the others replay the chain below.
            bool ok;
            {
                bool wany;
                const bool wplain = iq1_weights_plain<N>(weight, wany);
                const float totw = tws0 + tws1;
                // the largest's candidate: its i1 (set when an i1 iteration raised the largest) and its i2 (set when
                // the pair's four candidates raised it); its k is found after the pass, as the first of the pair's
                // four scores, formed again, that equals the largest (the first to reach it is the last raise)
                float S1 = -1.f, S2 = -1.f;
                int si1 = 0, si2 = 0;
                for (int i1 = 0; i1 <= N; ++i1) {
                    const float a0x = px0[i1], a1x = px1[i1], a0w = pw0[i1], a1w = pw1[i1];
                    const float S1in = S1;
#pragma unroll
                    for (int i2 = 0; i2 <= N; ++i2) {
                        if (i2 < i1) continue;
                        float sumqx[4], sumq2[4];
                        iq1m_sums(a0x, a1x, a0w, a1w, px0[i2], px1[i2], pw0[i2], pw1[i2], txs0, txs1, tws0, tws1,
                                  sumqx, sumq2);
                        const float S1p = S1;
#pragma unroll
                        for (int k = 0; k < 4; ++k) {
                            const float A = sumqx[k] * sumqx[k] * __builtin_amdgcn_rcpf(sumq2[k]);
                            S2 = __builtin_amdgcn_fmed3f(S1, S2, A);      // (S1 >= S2: the second of the three)
                            S1 = fmaxf(S1, A);                            // (no NaN where the result is used)
                        }
                        si2 = S1 > S1p ? i2 : si2;
                    }
                    si1 = S1 > S1in ? i1 : si1;
                }
                ok = iq1_rank_ok(wplain, totw, mx, S1, S2);
                if (ok) {
                    besti1 = si1;
                    besti2 = si2;
                    // the winner's sums again (the same operations on the same prefix values), its shift pair k and
                    // its scale as the chain computes it
                    float a[4] = {0.f, 0.f, 0.f, 0.f}, b[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                    for (int j = 0; j <= N; ++j) {
                        if (j == besti1) { a[0] = px0[j]; a[1] = px1[j]; a[2] = pw0[j]; a[3] = pw1[j]; }
                        if (j == besti2) { b[0] = px0[j]; b[1] = px1[j]; b[2] = pw0[j]; b[3] = pw1[j]; }
                    }
                    float sumqx[4], sumq2[4];
                    iq1m_sums(a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3], txs0, txs1, tws0, tws1, sumqx, sumq2);
                    bk = 3;
#pragma unroll
                    for (int k = 2; k >= 0; --k)
                        if (sumqx[k] * sumqx[k] * __builtin_amdgcn_rcpf(sumq2[k]) == S1) bk = k;
                    float bx = sumqx[0], b2 = sumq2[0];
#pragma unroll
                    for (int k = 1; k < 4; ++k) {
                        if (k == bk) { bx = sumqx[k]; b2 = sumq2[k]; }
                    }
                    scale = bx / b2;
                }
            }
            // ggml's acceptance chain for the lanes the ranking could not settle: i1 rolled (its prefix values read
            // once an iteration), i2 unrolled with a uniform skip below i1: every prefix read in the inner body is a
            // fixed register
            if (__ballot(!ok)) {
                float best_score = ok ? __builtin_inff() : -FLT_MAX;     // (a settled lane accepts nothing here)
                for (int i1 = 0; i1 <= N; ++i1) {
                    const float a0x = px0[i1], a1x = px1[i1], a0w = pw0[i1], a1w = pw1[i1];
#pragma unroll
                    for (int i2 = 0; i2 <= N; ++i2) {
                        if (i2 < i1) continue;
                        float sumqx[4], sumq2[4];
                        iq1m_sums(a0x, a1x, a0w, a1w, px0[i2], px1[i2], pw0[i2], pw1[i2], txs0, txs1, tws0, tws1,
                                  sumqx, sumq2);
#pragma unroll
                        for (int k = 0; k < 4; ++k) {
                            // (both tests evaluated: one branch instead of two nested ones; the second has no effects)
                            if ((sumq2[k] > 0) & (sumqx[k] * sumqx[k] > best_score * sumq2[k])) {
                                scale = sumqx[k] / sumq2[k];
                                best_score = scale * sumqx[k];
                                besti1 = i1; besti2 = i2; bk = k;
                            }
                        }
                    }
                }
            }
            if (besti1 < 0 || besti2 < 0 || bk < 0) {
                scale = 0.f;
            } else {
                live = true;
                const bool flip = scale < 0;
                if (flip) { scale = -scale; bk = 3 - bk; }
                best_k = bk;
#pragma unroll
                for (int k = 0; k < 2; ++k) {
                    int k3 = 0, p3 = 1;
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        const int r = (int)R.get(8 * k + j);
                        int l = r < besti1 ? 0 : (r < besti2 ? 1 : 2);
                        if (flip) l = 2 - l;
                        k3 += l * p3;
                        p3 *= 3;
                    }
                    mk2[k] = map3[k3];
                }
            }
        }
        // the groups' points (every lane: the neighbour search is wave-wide), both groups in one call
        bool all_on_grid;
        {
            const bool mn[2] = {!(best_k < 2), !(best_k % 2 == 0)};
            bool og[2];
            iq1_group_points2(live, mk2, x, weight, x + 8, weight + 8, scale, mn, p, grid, ws, gi2, og);
            all_on_grid = og[0] && og[1];
        }
        if (live) {
            {
                const int bk = best_k;
                if (!all_on_grid) {
                    float sqx = 0, sq2 = 0;
#pragma unroll
                    for (int k = 0; k < 2; ++k) {
                        const bool minus = k == 0 ? !(bk < 2) : !(bk % 2 == 0);
                        const uint64_t pt = grid[gi2[k]];
#pragma unroll
                        for (int j = 0; j < 8; ++j) {
                            const int b = (int)((pt >> (8 * j)) & 0xffu);
                            const float w = weight[8 * k + j];
                            const float q = iq1_val((b - 1) / 2, minus);
                            sqx += w * q * x[8 * k + j];
                            sq2 += w * q * q;
                        }
                    }
                    if (sqx > 0 && sq2 > 0) scale = sqx / sq2;
                }
            }
        }
        uint32_t qh = 0;
        if (live) {
            img_or16(img, boff + 2 * g, (uint32_t)(gi2[0] & 255) | ((uint32_t)(gi2[1] & 255) << 8));
            qh = (uint32_t)((gi2[0] >> 8) | ((gi2[1] >> 8) << 4));
        }
        const float max_scale = grp_max<G>(scale);
        if (!max_scale) {
            img_or8(img, boff + 32 + g, qh);
            return;
        }
        float d = max_scale / 15;
        const float id = 1 / d;
        const int l = imax(0, imin(7, nint(0.5f * (id * scale - 1))));
        const uint32_t masks = best_k == 0 ? 0x00u : best_k == 1 ? 0x80u : best_k == 2 ? 0x08u : 0x88u;
        qh |= masks;
        img_or8(img, boff + 32 + g, qh);
        // ggml's least-squares d over all 256 weights, with each block's stored point (grid[0] for a skipped one)
        float tqx[16], tq2[16];
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const bool minus = k == 0 ? !(best_k < 2) : !(best_k % 2 == 0);
            const uint64_t pt = grid[live ? gi2[k] : 0];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int b = (int)((pt >> (8 * j)) & 0xffu);
                const float w = weight[8 * k + j];
                const float q = iq1_val((b - 1) / 2, minus) * (2 * l + 1);
                tqx[8 * k + j] = w * q * x[8 * k + j];
                tq2[8 * k + j] = w * q * q;
            }
        }
        float sumqx_f, sumq2_f;
        grp_chain_sum2<G, 16>(tqx, tq2, g, sumqx_f, sumq2_f);
        if (sumq2_f > 0) d = sumqx_f / sumq2_f;
        const uint32_t s = f2h(d * 1.1125f);
        // scales: 4 u16 words, block ib's 3 bits at word ib/4, bits 3*(ib%4); the fp16 nibbles at bits 12..15
        img_or16(img, boff + 48 + 2 * (g / 4), (uint32_t)(l << (3 * (g % 4))));
        if (g < 4) {
            const uint32_t nib = (s >> (4 * g)) & 0xfu;
            img_or16(img, boff + 48 + 2 * g, nib << 12);
        }
    }
};
