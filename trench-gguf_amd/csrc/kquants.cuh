// trench-gguf_amd/csrc/kquants.cuh - Q2_K .. Q6_K, Q8_0, IQ4_NL and IQ4_XS on gfx950.
//
// Semantics: ggml's quantize_row_*_impl (with an imatrix) and *_ref (without), as the reference restates them in
// gpuq/gpuq.hip:1403-1838 and 1285-1398. Each lane runs its sub-block's search (affine trial scales, symmetric trial
// scales, coordinate descent) in ggml's serial order; super-block steps over all sub-blocks (sigma2, make_qp_quants
// of the sub-block scales, the max-|scale| pick) run on gathered values in every lane of the group.
#pragma once
#include "frame.cuh"

#define EPS_GROUP 1e-15f

// N levels packed four to a dword (byte i of the sub-block at bits 8*(i%4) of word i/4). Indices are compile-time
// constants after unrolling, so the words stay in VGPRs.
template <int N> struct Lv {
    uint32_t w[(N + 3) / 4];
    DEV void clear() {
#pragma unroll
        for (int k = 0; k < (N + 3) / 4; ++k) w[k] = 0u;
    }
    DEV uint32_t get(int i) const { return (w[i / 4] >> (8 * (i % 4))) & 0xffu; }
    DEV int gets(int i) const { return (int)(int8_t)get(i); }
    DEV void put(int i, uint32_t v) {
        const int s = 8 * (i % 4);
        w[i / 4] = (w[i / 4] & ~(0xffu << s)) | ((v & 0xffu) << s);
    }
};

// the lowest lane index of the group holding the largest a (a >= 0, not NaN): ggml's `if (a > amax)` scan in order
template <int G> DEV int grp_argmax_first(float a, int g) {
    float best = a;
    int bi = g;
#pragma unroll
    for (int o = 1; o < G; o <<= 1) {
        const float oa = __shfl_xor(best, o, 64);
        const int oi = __shfl_xor(bi, o, 64);
        if (oa > best || (oa == best && oi < bi)) { best = oa; bi = oi; }
    }
    return bi;
}

template <int G, int N> DEV void grp_gather(float v, float (&out)[N]) {
#pragma unroll
    for (int j = 0; j < N; ++j) out[j] = grp_bcast<G>(v, j);
}

// ------------------------------------------------------------------ searches (one lane, one sub-block)
// make_qp_quants: levels 0..nmax for non-negative x (gpuq/gpuq.hip:114-176); uint8 stores as ggml's.
// qp_start: the first scale, the eight trial scales, and the best one's levels and sums (sum w x l, sum w l^2); false
// for a group whose largest value is below EPS_GROUP (levels 0, scale 0, no refinement)
template <int N>
DEV bool qp_start(int nmax, const float (&x)[N], Lv<N> &L, const float (&qw)[N], float &sumlx, float &suml2) {
    float mx = 0;
#pragma unroll
    for (int i = 0; i < N; ++i) mx = fmax_sel(mx, x[i]);
    if (mx < EPS_GROUP) {
        L.clear();
        return false;
    }
    float iscale = nmax / mx;
#pragma unroll
    for (int i = 0; i < N; ++i) L.put(i, (uint32_t)nint(iscale * x[i]));
    const float scale = 1 / iscale;
    float best_mse = 0;
#pragma unroll
    for (int i = 0; i < N; ++i) {
        const float diff = x[i] - scale * (float)L.get(i);
        best_mse += qw[i] * diff * diff;
    }
    for (int is = -4; is <= 4; ++is) {
        if (is == 0) continue;
        const float iscale_is = (0.1f * is + nmax) / mx;
        const float scale_is = 1 / iscale_is;
        float mse = 0;
#pragma unroll
        for (int i = 0; i < N; ++i) {
            const int l = imin(nmax, nint(iscale_is * x[i]));
            const float diff = x[i] - scale_is * l;
            mse += qw[i] * diff * diff;
        }
        if (mse < best_mse) { best_mse = mse; iscale = iscale_is; }
    }
    sumlx = 0;
    suml2 = 0;
#pragma unroll
    for (int i = 0; i < N; ++i) {
        const int l = imin(nmax, nint(iscale * x[i]));
        L.put(i, (uint32_t)l);
        sumlx += qw[i] * x[i] * l;
        suml2 += qw[i] * l * l;
    }
    return true;
}

// one element of a refinement pass: element (x, w) at level li against the running sums; true when the pass changes
// it, to level nl with the sums (nslx, nsl2)
DEV bool qp_step(int nmax, float x, float w, int li, float sumlx, float suml2, int &nl, float &nslx, float &nsl2) {
    float slx = sumlx - w * x * li;
    float sl2 = suml2 - w * li * li;
    if (slx > 0 && sl2 > 0) {
        nl = imin(nmax, nint(x * sl2 / slx));
        if (nl != li) {
            slx += w * x * nl;
            sl2 += w * nl * nl;
            nslx = slx;
            nsl2 = sl2;
            return slx * slx * suml2 > sumlx * sumlx * sl2;
        }
    }
    return false;
}

// one refinement pass over the group in index order; the number of levels it changed
template <int N>
DEV int qp_pass(int nmax, const float (&x)[N], Lv<N> &L, const float (&qw)[N], float &sumlx, float &suml2) {
    int changed = 0;
#pragma unroll
    for (int i = 0; i < N; ++i) {
        int nl = 0;
        float a = 0.f, b = 0.f;
        if (qp_step(nmax, x[i], qw[i], (int)L.get(i), sumlx, suml2, nl, a, b)) {
            L.put(i, (uint32_t)nl);
            sumlx = a;
            suml2 = b;
            ++changed;
        }
    }
    return changed;
}

template <int N> DEV float qp_levels(int nmax, const float (&x)[N], Lv<N> &L, const float (&qw)[N]) {
    float sumlx, suml2;
    if (!qp_start<N>(nmax, x, L, qw, sumlx, suml2)) return 0.f;
    for (int pass = 0; pass < 5; ++pass)
        if (!qp_pass<N>(nmax, x, L, qw, sumlx, suml2)) break;
    return suml2 > 0.0f ? sumlx / suml2 : 0.0f;
}

// qp_levels over a group's G values that every lane of the group holds (the k-quants' sub-block scales and mins):
// the 9 first-scale evaluations (the first iscale, then is = -4..-1, 1..4) are dealt over the lanes, each computed as
// the serial loop computes it, and every lane replays the strict-less minimum over them in trial order; the levels
// and the refinement passes that follow run on every lane as in qp_levels.
template <int G> DEV float qp_levels_grp(int nmax, const float (&x)[G], Lv<G> &L, const float (&qw)[G], int g) {
    float mx = 0;
#pragma unroll
    for (int i = 0; i < G; ++i) mx = fmax_sel(mx, x[i]);
    if (mx < EPS_GROUP) {
        L.clear();
        return 0.f;
    }
    constexpr int NE = 9, NR = (NE + G - 1) / G;
    auto iscale_of = [&](int e) -> float {
        if (e == 0) return nmax / mx;
        const int is = e <= 4 ? e - 5 : e - 4;
        return (0.1f * is + nmax) / mx;
    };
    float mse_r[NR];
#pragma unroll
    for (int r = 0; r < NR; ++r) {
        const int e = r * G + g < NE ? r * G + g : NE - 1;
        const float iscale_e = iscale_of(e);
        const float scale_e = 1 / iscale_e;
        float mse = 0;
#pragma unroll
        for (int i = 0; i < G; ++i) {
            const int lr = nint(iscale_e * x[i]);
            // (the first evaluation takes the level unclamped, through its uint8 store; the trials clamp it)
            const float lf = e == 0 ? (float)(uint32_t)lr : (float)imin(nmax, lr);
            const float diff = x[i] - scale_e * lf;
            mse += qw[i] * diff * diff;
        }
        mse_r[r] = mse;
    }
    float best = grp_bcast<G>(mse_r[0], 0);
    int win = 0;
#pragma unroll
    for (int e = 1; e < NE; ++e) {
        const float m = grp_bcast<G>(mse_r[e / G], e % G);
        win = m < best ? e : win;
        best = m < best ? m : best;
    }
    const float iscale = iscale_of(win);
    float sumlx = 0, suml2 = 0;
#pragma unroll
    for (int i = 0; i < G; ++i) {
        const int l = imin(nmax, nint(iscale * x[i]));
        L.put(i, (uint32_t)l);
        sumlx += qw[i] * x[i] * l;
        suml2 += qw[i] * l * l;
    }
    for (int pass = 0; pass < 5; ++pass)
        if (!qp_pass<G>(nmax, x, L, qw, sumlx, suml2)) break;
    return suml2 > 0.0f ? sumlx / suml2 : 0.0f;
}

// symmetric levels (l + nmax) in [0, 2 nmax), best of 19 trial scales, wv = the importance (qw, or x^2)
// (gpuq/gpuq.hip:1427-1466)
template <int N> DEV float sym_levels(int nmax, const float (&x)[N], Lv<N> &L, const float (&wv)[N]) {
    float amax = 0, mx = 0;
#pragma unroll
    for (int i = 0; i < N; ++i) {
        const float ax = fabsf(x[i]);
        if (ax > amax) { amax = ax; mx = x[i]; }
    }
    if (amax < EPS_GROUP) {
        L.clear();
        return 0.f;
    }
    float iscale = -nmax / mx;
    float sumlx = 0, suml2 = 0;
#pragma unroll
    for (int i = 0; i < N; ++i) {
        const int l = imax(-nmax, imin(nmax - 1, nint(iscale * x[i])));
        L.put(i, (uint32_t)(l + nmax));
        sumlx += wv[i] * x[i] * l;
        suml2 += wv[i] * l * l;
    }
    float scale = suml2 ? sumlx / suml2 : 0.0f;
    float best = scale * sumlx;
    // A wave whose values are all finite forms the trials' levels in float: |iscale * x| <= nmax + 0.9 (mx has the
    // largest magnitude), and for |v| <= 2^21 nint(v) is (v + 1.5*2^23) - 1.5*2^23, so clamping v to the integer
    // bounds first gives the clamped level exactly (two-clock adds in place of the integer extraction and
    // conversion); the accepted trial's levels are formed again after the loop. (A NaN or infinite value, whose level
    // ggml's integer rounding takes from its bits, keeps the integer loop below.)
    bool fin = true;
#pragma unroll
    for (int i = 0; i < N; ++i) fin = fin && __builtin_isfinite(x[i]);
    if (!__ballot(!fin)) {
        constexpr float RND = 12582912.f;
        const float lo = (float)-nmax, hi = (float)(nmax - 1);
        float acc_is = 0.f;
        bool acc = false;
        for (int is = -9; is <= 9; ++is) {
            if (is == 0) continue;
            iscale = -(nmax + 0.1f * is) / mx;
            sumlx = suml2 = 0;
#pragma unroll
            for (int i = 0; i < N; ++i) {
                const float lf = (fminf(fmaxf(iscale * x[i], lo), hi) + RND) - RND;
                sumlx += wv[i] * x[i] * lf;
                suml2 += wv[i] * lf * lf;
            }
            if (suml2 > 0 && sumlx * sumlx > best * suml2) {
                acc = true;
                acc_is = iscale;
                scale = sumlx / suml2;
                best = scale * sumlx;
            }
        }
        if (acc) {
#pragma unroll
            for (int i = 0; i < N; ++i) L.put(i, (uint32_t)(imax(-nmax, imin(nmax - 1, nint(acc_is * x[i]))) + nmax));
        }
        return scale;
    }
    for (int is = -9; is <= 9; ++is) {
        if (is == 0) continue;
        iscale = -(nmax + 0.1f * is) / mx;
        sumlx = suml2 = 0;
        Lv<N> La;
#pragma unroll
        for (int i = 0; i < N; ++i) {
            const int l = imax(-nmax, imin(nmax - 1, nint(iscale * x[i])));
            if (i % 4 == 0) La.w[i / 4] = 0u;
            La.w[i / 4] |= (uint32_t)(l + nmax) << (8 * (i % 4));
            sumlx += wv[i] * x[i] * l;
            suml2 += wv[i] * l * l;
        }
        if (suml2 > 0 && sumlx * sumlx > best * suml2) {
            L = La;
            scale = sumlx / suml2;
            best = scale * sumlx;
        }
    }
    return scale;
}

// sym_levels over a group's G values that every lane of the group holds (Q3_K's 16 sub-block scales): the 19
// evaluations (the first iscale, then the trials is = -9..-1, 1..9) are dealt one a lane (lanes 0-2 take a second),
// each computed exactly as the serial loop computes it; every lane then replays ggml's acceptance chain over them in
// trial order from the owners' sums. Returns the scale; lvl = the level (0 .. 2 nmax - 1) of value g (own = x[g]), or
// 0 when the values are all negligible (make_qx_quants, gpuq/gpuq.hip:75-112).
template <int G>
DEV float sym_levels_grp(int nmax, const float (&x)[G], const float (&wv)[G], float own, int g, int &lvl) {
    float amax = 0, mx = 0;
#pragma unroll
    for (int i = 0; i < G; ++i) {
        const float ax = fabsf(x[i]);
        if (ax > amax) { amax = ax; mx = x[i]; }
    }
    lvl = 0;
    if (amax < EPS_GROUP) return 0.f;
    constexpr int NE = 19;                      // evaluation e: 0 the first iscale, then is = e - 10 (e <= 9) or e - 9
    auto iscale_of = [&](int e) -> float {
        if (e == 0) return -nmax / mx;
        const int is = e <= 9 ? e - 10 : e - 9;
        return -(nmax + 0.1f * is) / mx;
    };
    auto eval = [&](int e, float &sumlx, float &suml2) {
        const float iscale = iscale_of(e);
        sumlx = 0;
        suml2 = 0;
#pragma unroll
        for (int i = 0; i < G; ++i) {
            const int l = imax(-nmax, imin(nmax - 1, nint(iscale * x[i])));
            sumlx += wv[i] * x[i] * l;
            suml2 += wv[i] * l * l;
        }
    };
    // pass 0: evaluation g; pass 1: evaluation G + g (lanes g < NE - G; the others repeat evaluation G)
    float sx0, s20, sx1, s21;
    eval(g, sx0, s20);
    eval(G + (g < NE - G ? g : 0), sx1, s21);
    // an evaluation's scale and best as the chain would set them on accepting it (the first: unconditionally)
    const float sc0 = g == 0 ? (s20 ? sx0 / s20 : 0.0f) : sx0 / s20, bt0 = sc0 * sx0;
    const float sc1 = sx1 / s21, bt1 = sc1 * sx1;
    float best = grp_bcast<G>(bt0, 0);
    int win = 0;
#pragma unroll
    for (int e = 1; e < NE; ++e) {
        const int src = e < G ? e : e - G;
        const float sumlx = grp_bcast<G>(e < G ? sx0 : sx1, src);
        const float suml2 = grp_bcast<G>(e < G ? s20 : s21, src);
        const float bt = grp_bcast<G>(e < G ? bt0 : bt1, src);
        const bool acc = suml2 > 0 && sumlx * sumlx > best * suml2;
        best = acc ? bt : best;
        win = acc ? e : win;
    }
    const float scw0 = grp_bcast<G>(sc0, win < G ? win : 0), scw1 = grp_bcast<G>(sc1, win < G ? 0 : win - G);
    lvl = imax(-nmax, imin(nmax - 1, nint(iscale_of(win) * own))) + nmax;
    return win < G ? scw0 : scw1;
}

// Q3_K without an imatrix: 3-bit levels then coordinate descent on x^2 weights (gpuq/gpuq.hip:1468-1508)
template <int N> DEV float sym3_levels(int nmax, const float (&x)[N], Lv<N> &L) {
    float amax = 0, mx = 0;
#pragma unroll
    for (int i = 0; i < N; ++i) {
        const float ax = fabsf(x[i]);
        if (ax > amax) { amax = ax; mx = x[i]; }
    }
    if (amax < EPS_GROUP) {
        L.clear();
        return 0.f;
    }
    const float iscale = -nmax / mx;
    float sumlx = 0, suml2 = 0;
#pragma unroll
    for (int i = 0; i < N; ++i) {
        const int l = imax(-nmax, imin(nmax - 1, nint(iscale * x[i])));
        L.put(i, (uint32_t)l);
        const float w = x[i] * x[i];
        sumlx += w * x[i] * l;
        suml2 += w * l * l;
    }
    for (int pass = 0; pass < 5; ++pass) {
        int changed = 0;
#pragma unroll
        for (int i = 0; i < N; ++i) {
            const float w = x[i] * x[i];
            const int Li = L.gets(i);
            float slx = sumlx - w * x[i] * Li;
            if (!(slx > 0)) continue;
            float sl2 = suml2 - w * Li * Li;
            const int nl = imax(-nmax, imin(nmax - 1, nint(x[i] * sl2 / slx)));
            if (nl == Li) continue;
            slx += w * x[i] * nl;
            sl2 += w * nl * nl;
            if (sl2 > 0 && slx * slx * suml2 > sumlx * sumlx * sl2) {
                L.put(i, (uint32_t)nl);
                sumlx = slx;
                suml2 = sl2;
                ++changed;
            }
        }
        if (!changed) break;
    }
#pragma unroll
    for (int i = 0; i < N; ++i) L.put(i, (uint32_t)(L.gets(i) + nmax));
    return suml2 > 0.0f ? sumlx / suml2 : 0.0f;
}

// affine levels in [0, nmax] (x ~ scale*L - the_min) over nstep+1 trial scales; WI: ggml's imatrix variant
// (make_qkx3), else the plain one (make_qkx2). Trial is reads the min that earlier accepted trials left
// (gpuq/gpuq.hip:1510-1587).
template <bool WI, int N>
DEV float affine_levels(int nmax, const float (&x)[N], const float (&w)[N], Lv<N> &L, float &the_min, float rmin,
                        float rdelta, int nstep, bool use_mad) {
    float mn = x[0], mx = x[0];
    float sum_w = w[0];
    float sum_x = sum_w * x[0];
#pragma unroll
    for (int i = 1; i < N; ++i) {
        if (x[i] < mn) mn = x[i];
        if (x[i] > mx) mx = x[i];
        sum_w += w[i];
        sum_x += w[i] * x[i];
    }
    if (mn > 0) mn = 0;
    if (WI ? mx <= mn : mx == mn) {
        L.clear();
        the_min = -mn;
        return 0.f;
    }
    float iscale = nmax / (mx - mn);
    float scale = 1 / iscale;
    float best = 0;
#pragma unroll
    for (int i = 0; i < N; ++i) {
        const int l = imax(0, imin(nmax, nint(iscale * (x[i] - mn))));
        L.put(i, (uint32_t)l);
        float diff = scale * l + mn - x[i];
        diff = use_mad ? fabsf(diff) : diff * diff;
        best += w[i] * diff;
    }
    // The trials keep their levels as floats; the accepted trial's (iscale, min) are kept and its levels formed again
    // after the loop (the same operations on the same values), instead of packing every trial's levels. With the
    // imatrix the level is formed in float: ggml's `v > 0 ? nint(v < nmax ? v : nmax) : 0` is nint(c) for
    // c = min(max(v, 0), nmax) (IEEE max and min: v <= 0, -inf and NaN give 0, +inf gives nmax), and with 0 <= c <= nmax
    // nint(c) is the integer that c + 1.5*2^23 rounds to, so (c + 1.5*2^23) - 1.5*2^23 is its exact value: one clamp
    // and two two-clock adds in place of the compare, select, integer extraction and conversion.
    constexpr float RND = 12582912.f;
    float acc_is = 0.f, acc_mn = 0.f;
    bool acc = false;
    for (int is = 0; is <= nstep; ++is) {
        iscale = (rmin + rdelta * is + nmax) / (mx - mn);
        float sum_l = 0, sum_l2 = 0, sum_xl = 0;
        float lf[N];
#pragma unroll
        for (int i = 0; i < N; ++i) {
            if (WI) {
                lf[i] = (fminf(fmaxf(iscale * (x[i] - mn), 0.f), (float)nmax) + RND) - RND;
            } else {
                lf[i] = (float)imax(0, imin(nmax, nint(iscale * (x[i] - mn))));
            }
            sum_l += w[i] * lf[i];
            sum_l2 += w[i] * lf[i] * lf[i];
            sum_xl += w[i] * lf[i] * x[i];
        }
        const float D = sum_w * sum_l2 - sum_l * sum_l;
        if (!(D > 0)) continue;
        float this_scale = (sum_w * sum_xl - sum_x * sum_l) / D;
        float this_min = (sum_l2 * sum_x - sum_l * sum_xl) / D;
        if (this_min > 0) {
            this_min = 0;
            this_scale = sum_xl / sum_l2;
        }
        float err = 0;
#pragma unroll
        for (int i = 0; i < N; ++i) {
            float diff = this_scale * lf[i] + this_min - x[i];
            diff = use_mad ? fabsf(diff) : diff * diff;
            err += w[i] * diff;
        }
        if (err < best) {
            acc = true;
            acc_is = iscale;
            acc_mn = mn;
            best = err;
            scale = this_scale;
            mn = this_min;
        }
    }
    if (acc) {
#pragma unroll
        for (int i = 0; i < N; ++i) {
            int l;
            if (WI) {
                const float v = acc_is * (x[i] - acc_mn);
                l = v > 0 ? nint(v < nmax ? v : (float)nmax) : 0;
            } else {
                l = imax(0, imin(nmax, nint(acc_is * (x[i] - acc_mn))));
            }
            L.put(i, (uint32_t)l);
        }
    }
    the_min = -mn;
    return scale;
}

// OR four packed level bytes (shifted) into the image at a dword-aligned-in-block position
DEV void img_or_words(uint8_t *img, int off, const uint32_t *wv, int nw) {
    for (int k = 0; k < nw; ++k) img_or32(img, off + 4 * k, wv[k]);
}

// ------------------------------------------------------------------ Q2_K (gpuq/gpuq.hip:1621-1668)
// block: scales[16] qs[64] d dmin (84 bytes); lane g = 16-weight sub-block g
struct KQ2K {
    static constexpr int BS = QK, G = 16, N = 16, BB = 84, TAB = 0;
    static DEV void stage(const QParams &, uint8_t *) {}
    static DEV void quant(const float (&x)[N], const float *qwp, int g, uint8_t *img, int boff, uint8_t *,
                          const QParams &) {
        Lv<N> L;
        float w[N], mn;
        uint32_t scb;
        uint16_t d16, m16;
        if (!qwp) {
#pragma unroll
            for (int i = 0; i < N; ++i) w[i] = fabsf(x[i]);
            const float scale = affine_levels<false, N>(3, x, w, L, mn, -0.5f, 0.1f, 15, true);
            const float max_scale = grp_max<G>(scale > 0 ? scale : 0.f);
            const float max_min = grp_max<G>(mn > 0 ? mn : 0.f);
            scb = 0;
            if (max_scale > 0) {
                const float is = 15.f / max_scale;
                scb = (uint32_t)nint(is * scale) & 0xffu;
                d16 = f2h(max_scale / 15.f);
            } else {
                d16 = f2h(0.f);
            }
            if (max_min > 0) {
                const float im = 15.f / max_min;
                scb = (scb | ((uint32_t)nint(im * mn) << 4)) & 0xffu;
                m16 = f2h(max_min / 15.f);
            } else {
                m16 = f2h(0.f);
            }
        } else {
            float qv[N], sq[N];
            load_qw<N>(qwp, qv);
#pragma unroll
            for (int i = 0; i < N; ++i) sq[i] = x[i] * x[i];
            const float sigma2 = grp_chain_sum<G, N>(sq, g) / QK;
            float sw = 0;
#pragma unroll
            for (int i = 0; i < N; ++i) w[i] = qv[i] * sqrtf(sigma2 + sq[i]);
#pragma unroll
            for (int i = 0; i < N; ++i) sw += w[i];
            const float scale = affine_levels<true, N>(3, x, w, L, mn, -0.9f, 0.05f, 36, false);
            float sc_all[G], mn_all[G], sw_all[G];
            grp_gather<G>(scale, sc_all);
            grp_gather<G>(mn, mn_all);
            grp_gather<G>(sw, sw_all);
            Lv<G> Ls, Lm;
            const float dm = qp_levels_grp<G>(15, sc_all, Ls, sw_all, g);
            const float mm = qp_levels_grp<G>(15, mn_all, Lm, sw_all, g);
            d16 = f2h(dm);
            m16 = f2h(mm);
            scb = 0;
#pragma unroll
            for (int j = 0; j < G; ++j)
                if (j == g) scb = (Ls.get(j) | (Lm.get(j) << 4)) & 0xffu;
        }
        const uint32_t sc = scb & 0xF, mq = scb >> 4;
        const float dj = h2f(d16) * sc;
        if (dj) {
            const float mj = h2f(m16) * mq;
#pragma unroll
            for (int i = 0; i < N; ++i) L.put(i, (uint32_t)imax(0, imin(3, nint((x[i] + mj) / dj))));
        }
        img_or8(img, boff + g, scb);
        if (g == 0) img_or32(img, boff + 80, (uint32_t)d16 | ((uint32_t)m16 << 16));
        // qs: weight j = 16g + i sits in byte 32*(j/128) + (j%32), bits 2*((j%128)/32)
        uint32_t wv[4];
        const int sh = 2 * ((g % 8) / 2);
#pragma unroll
        for (int k = 0; k < 4; ++k) wv[k] = L.w[k] << sh;
        img_or_words(img, boff + 16 + 32 * (g / 8) + 16 * (g % 2), wv, 4);
    }
};

// ------------------------------------------------------------------ Q3_K (gpuq/gpuq.hip:1670-1724)
// block: hmask[32] qs[64] scales[12] d (110 bytes)
struct KQ3K {
    static constexpr int BS = QK, G = 16, N = 16, BB = 110, TAB = 0;
    static constexpr int WPE = 3;    // three waves a SIMD (168 VGPRs, 28 bytes a lane of spill): 13% faster than two
    static DEV void stage(const QParams &, uint8_t *) {}
    static DEV void quant(const float (&x)[N], const float *qwp, int g, uint8_t *img, int boff, uint8_t *,
                          const QParams &) {
        Lv<N> L;
        int Ls;              // this sub-block's 6-bit scale, -1: no scale bits written
        uint16_t d16;
        if (!qwp) {
            const float scale = sym3_levels<N>(4, x, L);
            const int jm = grp_argmax_first<G>(fabsf(scale), g);
            const float max_scale = grp_bcast<G>(scale, jm);
            if (max_scale) {
                const float iscale = -32.f / max_scale;
                const int8_t l = (int8_t)nint(iscale * scale);
                Ls = imax(-32, imin(31, l)) + 32;
                d16 = f2h(1 / iscale);
            } else {
                Ls = -1;
                d16 = f2h(0.f);
            }
        } else {
            float qv[N], sq[N], w[N];
            load_qw<N>(qwp, qv);
#pragma unroll
            for (int i = 0; i < N; ++i) sq[i] = x[i] * x[i];
            const float sigma2 = 2 * grp_chain_sum<G, N>(sq, g) / QK;
#pragma unroll
            for (int i = 0; i < N; ++i) w[i] = qv[i] * sqrtf(sigma2 + sq[i]);
            float s = 0;
#pragma unroll
            for (int i = 0; i < N; ++i) s += w[i];
            const float scale = sym_levels<N>(4, x, L, w);
            float sc_all[G], sw_all[G];
            grp_gather<G>(scale, sc_all);
            grp_gather<G>(s, sw_all);
            d16 = f2h(sym_levels_grp<G>(32, sc_all, sw_all, scale, g, Ls));
        }
        if (Ls >= 0) {
            if (g < 8) img_or8(img, boff + 96 + g, (uint32_t)(Ls & 0xF));
            else img_or8(img, boff + 96 + g - 8, (uint32_t)((Ls & 0xF) << 4));
            img_or8(img, boff + 96 + 8 + g % 4, (uint32_t)((Ls >> 4) << (2 * (g / 4))));
        }
        const float d = h2f(d16);
        const int sc = (Ls >= 0 ? Ls : 0) - 32;
        const float dj = d * sc;
        if (dj) {
#pragma unroll
            for (int i = 0; i < N; ++i) L.put(i, (uint32_t)(imax(-4, imin(3, nint(x[i] / dj))) + 4));
        }
        // hmask: weight j = 16g + i: byte j % 32, bit j / 32; the level loses its bit 2
        uint32_t hm[4], lo[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            hm[k] = 0;
            lo[k] = 0;
        }
#pragma unroll
        for (int i = 0; i < N; ++i) {
            const uint32_t l = L.get(i);
            hm[i / 4] |= (uint32_t)(l > 3) << (8 * (i % 4) + g / 2);
            lo[i / 4] |= (l > 3 ? l - 4 : l) << (8 * (i % 4));
        }
        img_or_words(img, boff + 16 * (g % 2), hm, 4);
        const int sh = 2 * ((g % 8) / 2);
#pragma unroll
        for (int k = 0; k < 4; ++k) lo[k] <<= sh;
        img_or_words(img, boff + 32 + 32 * (g / 8) + 16 * (g % 2), lo, 4);
        if (g == 0) img_or16(img, boff + 108, d16);
    }
};

// ------------------------------------------------------------------ Q4_K / Q5_K (gpuq/gpuq.hip:1726-1794)
// block: d dmin scales[12] then Q4_K qs[128] (144 bytes) / Q5_K qh[32] qs[128] (176 bytes); lane g = 32 weights
template <int NMAX> struct KQ45K {
    static constexpr int BS = QK, G = 8, N = 32, BB = NMAX == 15 ? 144 : 176, TAB = 0;
    static DEV void stage(const QParams &, uint8_t *) {}
    static DEV void quant(const float (&x)[N], const float *qwp, int g, uint8_t *img, int boff, uint8_t *,
                          const QParams &) {
        Lv<N> L;
        float w[N], mn;
        uint32_t ls[G], lm[G];
        uint16_t d16, m16;
        if (!qwp) {
            float s2 = 0;
#pragma unroll
            for (int i = 0; i < N; ++i) s2 += x[i] * x[i];
            const float av = sqrtf(s2 / 32);
#pragma unroll
            for (int i = 0; i < N; ++i) w[i] = av + fabsf(x[i]);
            const float scale = NMAX == 15 ? affine_levels<false, N>(NMAX, x, w, L, mn, -1.f, 0.1f, 20, false)
                                           : affine_levels<false, N>(NMAX, x, w, L, mn, -0.5f, 0.1f, 15, false);
            const float max_scale = grp_max<G>(scale > 0 ? scale : 0.f);
            const float max_min = grp_max<G>(mn > 0 ? mn : 0.f);
            const float is = max_scale > 0 ? 63.f / max_scale : 0.f;
            const float im = max_min > 0 ? 63.f / max_min : 0.f;
            const uint32_t a = (uint32_t)nint(is * scale) & 0xffu, b = (uint32_t)nint(im * mn) & 0xffu;
            const int la = a < 63u ? (int)a : 63, lb = b < 63u ? (int)b : 63;
#pragma unroll
            for (int j = 0; j < G; ++j) {
                ls[j] = (uint32_t)grp_bcast_i<G>(la, j);
                lm[j] = (uint32_t)grp_bcast_i<G>(lb, j);
            }
            d16 = f2h(max_scale / 63.f);
            m16 = f2h(max_min / 63.f);
        } else {
            float qv[N], sq[N];
            load_qw<N>(qwp, qv);
#pragma unroll
            for (int i = 0; i < N; ++i) sq[i] = x[i] * x[i];
            const float sigma2 = 2 * grp_chain_sum<G, N>(sq, g) / QK;
#pragma unroll
            for (int i = 0; i < N; ++i) w[i] = qv[i] * sqrtf(sigma2 + sq[i]);
            float s = 0;
#pragma unroll
            for (int i = 0; i < N; ++i) s += w[i];
            const float scale = affine_levels<true, N>(NMAX, x, w, L, mn, -0.9f, 0.05f, 36, false);
            float sc_all[G], mn_all[G], sw_all[G];
            grp_gather<G>(scale, sc_all);
            grp_gather<G>(mn, mn_all);
            grp_gather<G>(s, sw_all);
            Lv<G> Lsv, Lmv;
            const float db = qp_levels_grp<G>(63, sc_all, Lsv, sw_all, g);
            const float mb = qp_levels_grp<G>(63, mn_all, Lmv, sw_all, g);
#pragma unroll
            for (int j = 0; j < G; ++j) {
                ls[j] = Lsv.get(j);
                lm[j] = Lmv.get(j);
                if (NMAX == 31) { ls[j] = ls[j] < 63u ? ls[j] : 63u; lm[j] = lm[j] < 63u ? lm[j] : 63u; }
            }
            d16 = f2h(db);
            m16 = f2h(mb);
        }
        // the 12 scale bytes (pack_scales_k4), then this sub-block's (scale, min) read back from them
        uint32_t s8[12];
#pragma unroll
        for (int j = 0; j < 4; ++j) { s8[j] = ls[j] & 0xffu; s8[j + 4] = lm[j] & 0xffu; }
#pragma unroll
        for (int j = 4; j < 8; ++j) {
            s8[j + 4] = ((ls[j] & 0xF) | ((lm[j] & 0xF) << 4)) & 0xffu;
            s8[j - 4] = (s8[j - 4] | ((ls[j] >> 4) << 6)) & 0xffu;
            s8[j] = (s8[j] | ((lm[j] >> 4) << 6)) & 0xffu;
        }
        uint32_t sc = 0, mq = 0;
#pragma unroll
        for (int j = 0; j < G; ++j) {
            if (j == g) {
                if (j < 4) { sc = s8[j] & 63; mq = s8[j + 4] & 63; }
                else { sc = (s8[j + 4] & 0xF) | ((s8[j - 4] >> 6) << 4); mq = (s8[j + 4] >> 4) | ((s8[j] >> 6) << 4); }
            }
        }
        const float dj = h2f(d16) * sc;
        if (dj) {
            const float mj = h2f(m16) * mq;
#pragma unroll
            for (int i = 0; i < N; ++i) L.put(i, (uint32_t)imax(0, imin(NMAX, nint((x[i] + mj) / dj))));
        }
        if (g == 0) img_or32(img, boff, (uint32_t)d16 | ((uint32_t)m16 << 16));
        if (g < 3) img_or32(img, boff + 4 + 4 * g, s8[4 * g] | (s8[4 * g + 1] << 8) | (s8[4 * g + 2] << 16) | (s8[4 * g + 3] << 24));
        // qs: sub-blocks 2p and 2p+1 share 32 bytes (low / high nibble); Q5_K: bit 4 of each level goes to qh
        const int qso = NMAX == 15 ? 16 : 48;
        uint32_t wv[8];
        if (NMAX == 31) {
            uint32_t qh[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) qh[k] = 0;
#pragma unroll
            for (int i = 0; i < N; ++i) qh[i / 4] |= ((L.get(i) >> 4) & 1u) << (8 * (i % 4) + g);
            img_or_words(img, boff + 16, qh, 8);
        }
#pragma unroll
        for (int k = 0; k < 8; ++k) wv[k] = (L.w[k] & 0x0f0f0f0fu) << (4 * (g % 2));
        img_or_words(img, boff + qso + 32 * (g / 2), wv, 8);
    }
};

// ------------------------------------------------------------------ Q6_K (gpuq/gpuq.hip:1796-1829)
// block: ql[128] qh[64] scales[16] d (210 bytes)
struct KQ6K {
    static constexpr int BS = QK, G = 16, N = 16, BB = 210, TAB = 0;
    static DEV void stage(const QParams &, uint8_t *) {}
    static DEV void quant(const float (&x)[N], const float *qwp, int g, uint8_t *img, int boff, uint8_t *,
                          const QParams &) {
        float wv[N];
        if (qwp) load_qw<N>(qwp, wv);
        else {
#pragma unroll
            for (int i = 0; i < N; ++i) wv[i] = x[i] * x[i];
        }
        Lv<N> L;
        const float scale = sym_levels<N>(32, x, L, wv);
        const float a = fabsf(scale);
        const int jm = grp_argmax_first<G>(a, g);
        const float amax = grp_bcast<G>(a, jm);
        const float max_scale = grp_bcast<G>(scale, jm);
        if (amax < EPS_GROUP) return;              // an all-zero block (the image is zero)
        const float iscale = -128.f / max_scale;
        const uint16_t d16 = f2h(1 / iscale);
        const int8_t sc = (int8_t)imin(127, nint(iscale * scale));
        const float dj = h2f(d16) * sc;
        if (dj) {
#pragma unroll
            for (int i = 0; i < N; ++i) L.put(i, (uint32_t)(imax(-32, imin(31, nint(x[i] / dj))) + 32));
        }
        img_or8(img, boff + 192 + g, (uint32_t)(uint8_t)sc);
        if (g == 0) img_or16(img, boff + 208, d16);
        // weight p = 16*(g%8) + i of half h = g/8: ql byte 64h + p%64 (high nibble for p >= 64),
        // qh byte 32h + p%32, bits 2*(p/32)
        const int p0 = 16 * (g % 8), h = g / 8;
        uint32_t ql[4], qh[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            ql[k] = (L.w[k] & 0x0f0f0f0fu) << (p0 >= 64 ? 4 : 0);
            qh[k] = ((L.w[k] >> 4) & 0x03030303u) << (2 * (p0 / 32));
        }
        img_or_words(img, boff + 64 * h + p0 % 64, ql, 4);
        img_or_words(img, boff + 128 + 32 * h + p0 % 32, qh, 4);
    }
};

// ------------------------------------------------------------------ Q8_0 (gpuq/gpuq.hip:1831-1838)
// block: d qs[32] (34 bytes). Streaming sources (F32 / F16 / BF16): every lane loads 16 contiguous bytes a step, so
// a wave reads 1 KB contiguous per load instruction; 32/E lanes share a block's amax through xor shuffles. The
// source is read once: nontemporal loads.
DEV uint4 nt_load16(const uint8_t *p) {
    const v4u32 v = __builtin_nontemporal_load((const v4u32 *)p);
    return make_uint4(v.x, v.y, v.z, v.w);
}
template <int SRC> __global__ __launch_bounds__(WG_THREADS) void k_q8_0_stream(const uint8_t *src, uint8_t *dst,
                                                                               int64_t nblk) {
    constexpr int E = SRC == T_F32 ? 4 : 8;          // values a lane loads a step
    constexpr int LPB = 32 / E;                      // lanes a block
    constexpr int BPS = 64 / LPB;                    // blocks a wave step
    constexpr int U = 4;                             // steps a tile
    constexpr int TB = BPS * U;                      // blocks a tile
    constexpr int IMG = (TB * 34 + 15) & ~15;
    __shared__ __align__(16) uint8_t lds[WG_WAVES * IMG];
    const int wave = (int)(threadIdx.x >> 6), lane = lane_id();
    uint8_t *img = lds + wave * IMG;
    const int part = lane % LPB, bl = lane / LPB;
    const int64_t nwaves = (int64_t)gridDim.x * WG_WAVES;
    for (int64_t t = (int64_t)blockIdx.x * WG_WAVES + wave; t * TB < nblk; t += nwaves) {
        const int64_t b0 = t * TB;
        const int nact = (int)(nblk - b0 < TB ? nblk - b0 : TB);
        uint4 raw[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t blk = b0 + u * BPS + bl;
            raw[u] = blk < nblk ? nt_load16(src + (blk * 32 + part * E) * (SRC == T_F32 ? 4 : 2))
                                : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            float v[E];
            const uint32_t w4[4] = {raw[u].x, raw[u].y, raw[u].z, raw[u].w};
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                if (SRC == T_F32) v[k % E] = ffrom(w4[k]);
                else if (SRC == T_BF16) { v[(2 * k) % E] = ffrom(w4[k] << 16); v[(2 * k + 1) % E] = ffrom(w4[k] & 0xffff0000u); }
                else { v[(2 * k) % E] = h2f(w4[k] & 0xffffu); v[(2 * k + 1) % E] = h2f(w4[k] >> 16); }
            }
            float amax = 0.0f;
#pragma unroll
            for (int j = 0; j < E; ++j) amax = fmax_sel(amax, fabsf(v[j]));
#pragma unroll
            for (int o = 1; o < LPB; o <<= 1) amax = fmax_sel(amax, __shfl_xor(amax, o, 64));
            const float d = amax / 127;
            const float id = d ? 1.0f / d : 0.0f;
            const int off = (u * BPS + bl) * 34;
            if (part == 0) *(uint16_t *)(img + off) = f2h(d);
#pragma unroll
            for (int j = 0; j < E; j += 2) {
                const uint32_t q0 = (uint32_t)(int)roundf(v[j] * id) & 0xffu;
                const uint32_t q1 = (uint32_t)(int)roundf(v[j + 1] * id) & 0xffu;
                *(uint16_t *)(img + off + 2 + part * E + j) = (uint16_t)(q0 | (q1 << 8));
            }
        }
        wave_sync();
        img_store<true>(dst + b0 * 34, img, nact * 34);
        wave_sync();
    }
}

// Q8_0 from block-encoded sources (Q8_0 / MXFP4): one lane a 32-block through the frame
struct KQ80 {
    static constexpr int BS = 32, G = 1, N = 32, BB = 34, TAB = 0;
    static DEV void stage(const QParams &, uint8_t *) {}
    static DEV void quant(const float (&x)[N], const float *, int, uint8_t *img, int boff, uint8_t *, const QParams &) {
        float amax = 0.0f;
#pragma unroll
        for (int j = 0; j < 32; ++j) amax = fmax_sel(amax, fabsf(x[j]));
        const float d = amax / 127;
        const float id = d ? 1.0f / d : 0.0f;
        img_or16(img, boff, f2h(d));
#pragma unroll
        for (int j = 0; j < 32; j += 2) {
            const uint32_t q0 = (uint32_t)(int)roundf(x[j] * id) & 0xffu;
            const uint32_t q1 = (uint32_t)(int)roundf(x[j + 1] * id) & 0xffu;
            img_or16(img, boff + 2 + j, q0 | (q1 << 8));
        }
    }
};

// ------------------------------------------------------------------ IQ4_NL / IQ4_XS (gpuq/gpuq.hip:1285-1398)
__constant__ float k_iq4f[16] = {-127.f, -104.f, -83.f, -65.f, -49.f, -35.f, -22.f, -10.f,
                                 1.f,    13.f,   25.f,  38.f,  53.f,  69.f,  89.f,  113.f};

// best_index_int8 over the IQ4 codebook (gpuq/gpuq.hip:1286-1295). For strictly increasing values the reference's
// binary search always ends at the interval kv[ml] <= x < kv[ml+1] (ml = 15 for x >= kv[15] and for NaN, which its
// false x < kv[mav] tests move up; ml = 0 for x < kv[1]); then the nearer end with the reference's tie rule. The
// codebook values are integers, so kv[j] <= x exactly when kv[j] <= floor(x): the interval is a table entry indexed
// by floor(x) clamped to [-128, 113] (NaN read as 113), one LDS read instead of the search's chain of dependent
// reads (tests/test_iq4_table.py: equal to the reference's search on a dense sample of all floats, every float within
// 4096 ulps of each codebook value and midpoint, and the special values).
struct Iq4Ent {
    float lo;       // kv[ml]
    int mh;         // ml + 256 kv[min(ml + 1, 15)]: the upper end (an integer) is exactly (mh - ml) / 256
};
constexpr int IQ4_T0 = -128, IQ4_TN = 113 - IQ4_T0 + 1;    // table entries: floor(x) = -128 .. 113
DEV int iq4_index(float x, const Iq4Ent *tab, float &q) {
    const float f = fminf(fmaxf(floorf(x), (float)IQ4_T0), 113.f);
    const int fi = x != x ? IQ4_TN - 1 : (int)f - IQ4_T0;
    const Iq4Ent e = tab[fi];
    const int ml = e.mh & 15;
    const float hi = (float)((e.mh - ml) / 256);
    const bool down = ml == 15 || x - e.lo < hi - x;
    q = down ? e.lo : hi;
    return down ? ml : ml + 1;
}
// The trial scales' codebook value alone (their levels are not kept), for finite x with floor(x) in [-135, 134]
// (a trial's |id x| <= 134: |id| <= 134 / max|x|): a second table, indexed by floor(x) + 135, holds the interval's two
// ends as floats, the upper one equal to the lower for the last interval (x >= kv[15], where the search keeps kv[15],
// and below kv[0] the first interval's ends); the nearer end by the same test x - lo < hi - x, which for equal ends
// gives that end.
constexpr int IQ4_Q0 = -135, IQ4_QN = 134 - IQ4_Q0 + 1;
// (int)floorf(x) in one instruction (v_floor_f32 and v_cvt_i32_f32 are two four-clock ones) for finite x in the
// int range. A subnormal x floors to -1 or 0, depending on the denormal mode: both index the interval [-10, 1) of
// the codebook, so the value is the same either way.
DEV int floor_i32(float x) {
    int r;
    asm("v_cvt_flr_i32_f32 %0, %1" : "=v"(r) : "v"(x));
    return r;
}
DEV float iq4_value(float x, const float2 *tq) {
    const float2 e = tq[floor_i32(x) - IQ4_Q0];
    return x - e.x < e.y - x ? e.x : e.y;
}
// the tables (and the 16 codebook values before them), staged by a workgroup's threads
DEV void iq4_stage(uint8_t *lds) {
    float *kv = (float *)lds;
    if (threadIdx.x < 16) kv[threadIdx.x] = k_iq4f[threadIdx.x];
    Iq4Ent *tab = (Iq4Ent *)(lds + 64);
    for (int i = threadIdx.x; i < IQ4_TN; i += blockDim.x) {
        const float v = (float)(i + IQ4_T0);
        int ml = 0;
#pragma unroll
        for (int j = 1; j < 16; ++j) ml = k_iq4f[j] <= v ? j : ml;
        tab[i] = Iq4Ent{k_iq4f[ml], ml + 256 * (int)k_iq4f[ml < 15 ? ml + 1 : 15]};
    }
    float2 *tq = (float2 *)(lds + 64 + IQ4_TN * (int)sizeof(Iq4Ent));
    for (int i = threadIdx.x; i < IQ4_QN; i += blockDim.x) {
        const float v = (float)(i + IQ4_Q0);
        int ml = 0;
#pragma unroll
        for (int j = 1; j < 16; ++j) ml = k_iq4f[j] <= v ? j : ml;
        tq[i] = make_float2(k_iq4f[ml], k_iq4f[ml < 15 ? ml + 1 : 15]);
    }
}
constexpr int IQ4_TAB = 64 + IQ4_TN * (int)sizeof(Iq4Ent) + IQ4_QN * 8;
DEV const Iq4Ent *iq4_tab(const uint8_t *lds) { return (const Iq4Ent *)(lds + 64); }
DEV const float2 *iq4_qtab(const uint8_t *lds) { return (const float2 *)(lds + 64 + IQ4_TN * (int)sizeof(Iq4Ent)); }

// one 32-weight sub-block's scale search; fills Lb, returns the scale (0 for a negligible block)
DEV float iq4_block(const float (&xb)[32], const float (&weight)[32], Lv<32> &Lb, const float *kv,
                    const Iq4Ent *tab, const float2 *tq) {
    float amax = 0, mx = 0;
#pragma unroll
    for (int j = 0; j < 32; ++j) {
        const float ax = fabsf(xb[j]);
        if (ax > amax) { amax = ax; mx = xb[j]; }
    }
    if (amax < EPS_GROUP) return 0.f;
    float d = -mx / kv[0];
    float id = 1 / d;
    float sumqx = 0, sumq2 = 0;
#pragma unroll
    for (int j = 0; j < 32; ++j) {
        const float al = id * xb[j];
        float q;
        const int l = iq4_index(al, tab, q);
        Lb.put(j, (uint32_t)l);
        const float w = weight[j];
        sumqx += w * q * xb[j];
        sumq2 += w * q * q;
    }
    d = sumq2 > 0 ? sumqx / sumq2 : 0.f;
    float best = d * sumqx;
    bool fin = true;
#pragma unroll
    for (int j = 0; j < 32; ++j) fin = fin && __builtin_isfinite(xb[j]);
    if (fin) {
        for (int itry = -7; itry <= 7; ++itry) {
            id = (float)(itry + (-127)) / mx;
            sumqx = sumq2 = 0;
#pragma unroll
            for (int j = 0; j < 32; ++j) {
                const float q = iq4_value(id * xb[j], tq);
                const float w = weight[j];
                sumqx += w * q * xb[j];
                sumq2 += w * q * q;
            }
            if (sumq2 > 0 && sumqx * sumqx > best * sumq2) {
                d = sumqx / sumq2;
                best = d * sumqx;
            }
        }
        return d;
    }
    for (int itry = -7; itry <= 7; ++itry) {            // (a non-finite value: the clamped lookup)
        id = (float)(itry + (-127)) / mx;
        sumqx = sumq2 = 0;
#pragma unroll
        for (int j = 0; j < 32; ++j) {
            const float al = id * xb[j];
            float q;
            (void)iq4_index(al, tab, q);
            const float w = weight[j];
            sumqx += w * q * xb[j];
            sumq2 += w * q * q;
        }
        if (sumq2 > 0 && sumqx * sumqx > best * sumq2) {
            d = sumqx / sumq2;
            best = d * sumqx;
        }
    }
    return d;
}

// IQ4_XS: block d scales_h scales_l[4] qs[128] (136 bytes); lane g = sub-block g
struct KIQ4XS {
    static constexpr int BS = QK, G = 8, N = 32, BB = 136, TAB = IQ4_TAB;
    static constexpr int WPE = 3;    // three waves a SIMD (at most 168 VGPRs, no spill with the 8-byte table entries)
    static DEV void stage(const QParams &, uint8_t *lds) { iq4_stage(lds); }
    static DEV void quant(const float (&x)[N], const float *qwp, int g, uint8_t *img, int boff, uint8_t *lds,
                          const QParams &) {
        const float *kv = (const float *)lds;
        float sq[N], weight[N];
#pragma unroll
        for (int i = 0; i < N; ++i) sq[i] = x[i] * x[i];
        float sigma2 = grp_chain_sum<G, N>(sq, g);
        sigma2 *= 2.f / QK;
        if (qwp) {
            float qv[N];
            load_qw<N>(qwp, qv);
#pragma unroll
            for (int j = 0; j < N; ++j) weight[j] = qv[j] * sqrtf(sigma2 + sq[j]);
        } else {
#pragma unroll
            for (int j = 0; j < N; ++j) weight[j] = sq[j];
        }
        Lv<32> Lb;
        Lb.clear();
        const float sd = iq4_block(x, weight, Lb, kv, iq4_tab(lds), iq4_qtab(lds));
        const int jm = grp_argmax_first<G>(fabsf(sd), g);
        const float amax_scale = grp_bcast<G>(fabsf(sd), jm);
        const float max_scale = amax_scale > 0 ? grp_bcast<G>(sd, jm) : 0.f;   // (+0 when no |d| beat 0)
        const float d = -max_scale / 32;
        const uint16_t d16 = f2h(d);
        const float id = d ? 1 / d : 0.f;
        int l = nint(id * sd);
        l = imax(-32, imin(31, l));
        const float dl = d * l;
        const float idl = dl ? 1 / dl : 0.f;
#pragma unroll
        for (int j = 0; j < 32; ++j) { float q; Lb.put(j, (uint32_t)iq4_index(idl * x[j], iq4_tab(lds), q)); }
        l += 32;
        if (g == 0) img_or16(img, boff, d16);
        img_or16(img, boff + 2, (uint32_t)((l >> 4) << (2 * g)));
        img_or8(img, boff + 4 + g / 2, (uint32_t)((l & 0xf) << (4 * (g % 2))));
        uint32_t wv[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) wv[k] = Lb.w[k] | (Lb.w[k + 4] << 4);
        img_or_words(img, boff + 8 + 16 * g, wv, 4);
    }
};

// IQ4_NL: block d qs[16] (18 bytes), one lane a 32-block
struct KIQ4NL {
    static constexpr int BS = 32, G = 1, N = 32, BB = 18, TAB = IQ4_TAB;
    static DEV void stage(const QParams &, uint8_t *lds) { iq4_stage(lds); }
    static DEV void quant(const float (&x)[N], const float *qwp, int, uint8_t *img, int boff, uint8_t *lds,
                          const QParams &) {
        const float *kv = (const float *)lds;
        float sq[N], weight[N];
        float sigma2 = 0;
#pragma unroll
        for (int j = 0; j < N; ++j) { sq[j] = x[j] * x[j]; sigma2 += sq[j]; }
        sigma2 *= 2.f / 32;
        if (qwp) {
            float qv[N];
            load_qw<N>(qwp, qv);
#pragma unroll
            for (int j = 0; j < N; ++j) weight[j] = qv[j] * sqrtf(sigma2 + sq[j]);
        } else {
#pragma unroll
            for (int j = 0; j < N; ++j) weight[j] = sq[j];
        }
        Lv<32> Lb;
        Lb.clear();
        const float s = iq4_block(x, weight, Lb, kv, iq4_tab(lds), iq4_qtab(lds));
        img_or16(img, boff, f2h(s));
        const float id = s ? 1 / s : 0;
#pragma unroll
        for (int j = 0; j < 32; ++j) { float q; Lb.put(j, (uint32_t)iq4_index(id * x[j], iq4_tab(lds), q)); }
        uint32_t wv[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) wv[k] = Lb.w[k] | (Lb.w[k + 4] << 4);
        img_or_words(img, boff + 2, wv, 4);
    }
};
