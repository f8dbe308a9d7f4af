// trench-gguf_amd/csrc/filter.cuh - the filtered neighbour search of IQ2_XXS / IQ2_XS: one walk of a neighbour list
// serves every trial scale whose key (and so whose list) is the same.
//
// The trial scales of a group mostly round to the same key: over IQ2_XXS's 13 trials a group's key changes about
// twice, so ggml's serial scan (gpuq/gpuq.hip:178-197) walks the same list about five times at different scales.
// Here a list is walked once for all the consecutive trials of a window that share it. A candidate's distance at
// scale s, d2(s) = sum_i w_i (s q_i - x_i)^2, is split as s^2 A - 2 s B + C with A = sum w q^2, B = sum (w x) q (once
// a candidate) and C = sum (w x) x (once a list), and evaluated as D = fma(s, fma(s, A, B'), C) with B' the fma chain
// of the products of -2 (w x) and q (the factor -2 is exact), two operations a trial instead of ggml's 40. That value
// only approximates the distance ggml computes (its own operation order, fp32 roundings); the search uses it to rule
// candidates out, never to pick one that ggml would not:
//
//   with w >= 0, s > 0, q in 1..7 and S = sum w (s q + |x|)^2, ggml's d2 lies within 13.3 u S of the exact sum
//   (u = 2^-24; its products and sums in fp32) and so does D (the fma chains of A, B' and C are within 8u, 9u and
//   9u of their terms' magnitudes, and the two fmas of the trial add u each: at most 11 u S to first order, 11.1 u S
//   in all; intermediates below the normal range add at most 2^-149 each, which the lower limit on Smax below makes
//   negligible), and S <= Smax = s^2 49 sum(w) + 14 s sum(w |x|) + sum(w x^2) for every candidate; so with
//   delta = 2^-19 Smax >= 24.4 u S / 0.76 (the slack covers Smax's own rounding), the candidate of least D is ggml's
//   pick whenever every other candidate's D exceeds it by more than 2 delta: each of their ggml distances is then
//   larger than its ggml distance, so the strict-< first-wins scan cannot choose another. A negative D (rounding
//   near 0) is read as |D|, which is as close to ggml's non-negative d2.
//
// Each walker keeps, per trial, the two least keys (bits(|D|) with the low IB bits replaced by the grid index: the
// truncation lowers the value by less than 2^IB units in the last place, which the test allows for), and merges them
// into the list's pair with one returning LDS atomic min (the displaced value goes to the second slot). The caller
// applies the test; a trial that fails it (near ties, out-of-range values, non-finite input) goes through the exact
// cooperative search (coop.cuh), which repeats ggml's scan order.
#pragma once
#include <float.h>
#include "coop.cuh"

// per-wave workspace of the search over windows of W trials. List m of lane L (id e = m*64 + L) is the run of the
// lane's trials m .. m+ntr-1 that share one key. Each lane stages what a walker needs of its lists, as planes of
// float4 (the 64 lanes' writes of one plane are consecutive): -2 w*x (2 planes), w (2), then C = sum (w x) x and the
// trials' scales s (W).
template <int W> struct FiltWS {
    static_assert(W >= 1 && W <= 7, "trials a window: 1..7 (list ids < 512, run lengths < 8)");
    static constexpr int NPL = 4 + (1 + W + 3) / 4;
    float4 own[NPL][64];
    int2 ent[64 * W];               // first point's offset | length << 21, next list with candidates | e << 9 | ntr << 18
    unsigned k1[W][64], k2[W][64];  // per trial and lane: the least and the second-least key of the trial's list
    int mark[64];                   // walker lane: the list of its first piece | piece in that list << 9
};

// the median of three (the compiler's v_med3_u32)
DEV unsigned umed3(unsigned a, unsigned b, unsigned c) {
    const unsigned lo = a < b ? a : b, hi = a < b ? b : a;
    const unsigned m = hi < c ? hi : c;
    return lo > m ? lo : m;
}

// All 64 lanes call it together. Lane L's list m (cnt[m] candidates from neigh[off[m] + 1]; cnt[m] = 0: none)
// serves its trials m .. m + ntr[m] - 1 (the lists of one lane cover disjoint trials), searched at the scales s[t]
// for the lane's values xv (8) and weights wv (8). k1[t], k2[t]: the least and second-least key of trial t over its
// list (~0u: none, or trial t in no list). NG: the grid's size (a power of two).
//
// The deal: each list is cut into pieces of CH consecutive candidates, the wave's pieces are concatenated lane by
// lane, list by list (a wave prefix sum), and walker L takes the contiguous run of R = ceil(pieces / 64) pieces from
// L*R, one a round. A walker changes lists only between rounds, so the walkers' list changes (merge the running
// keys, read the new owner's values) come once a round rather than at any position, and within a round every walker
// evaluates CH candidates of one list (positions past the list's end are masked). The next piece's list entries are
// read while the current piece is evaluated.
template <int W, int IB, int NG, int CH = 4>
DEV void coop_filter(const int (&cnt)[W], const int (&off)[W], const int (&ntr)[W], const float (&s)[W],
                     const float (&xv)[8], const float (&wv)[8], const uint16_t *neigh, int neigh_len, FiltWS<W> &ws,
                     const uint64_t *grid, unsigned (&k1)[W], unsigned (&k2)[W]) {
    static_assert(CH == 1 || CH == 2 || CH == 4 || CH == 8, "piece size: a power of two");
    static_assert(NG >= 1 && (NG & (NG - 1)) == 0 && NG <= (1 << IB), "grid indices within a key's low bits");
    constexpr int CSH = CH == 1 ? 0 : CH == 2 ? 1 : CH == 4 ? 2 : 3;
    constexpr int OFF_MASK = (1 << 21) - 1;
    constexpr unsigned KHI = 0x7fffffffu & ~((1u << IB) - 1);   // a key's distance bits (the sign cleared)
    constexpr int NPL = FiltWS<W>::NPL;
    const __amdgpu_buffer_rsrc_t nrs = __builtin_amdgcn_make_buffer_rsrc((void *)neigh, 0, neigh_len * 2, 0x00020000);
    const int lane = lane_id();
    int tot = 0;
#pragma unroll
    for (int m = 0; m < W; ++m) tot += (cnt[m] + CH - 1) >> CSH;
    const int incl = wave_incl_scan(tot);
    const int total = __builtin_amdgcn_readlane(incl, 63);
#pragma unroll
    for (int t = 0; t < W; ++t) k1[t] = k2[t] = ~0u;
    if (total == 0) return;                             // wave-uniform
    // the lane's values for its walkers
    {
        float v[NPL * 4];
        float C = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float wx = wv[i] * xv[i];
            v[i] = -2.f * wx;
            v[8 + i] = wv[i];
            C = fmaf(wx, xv[i], C);
        }
        v[16] = C;
#pragma unroll
        for (int t = 0; t < W; ++t) v[17 + t] = s[t];
#pragma unroll
        for (int i = 17 + W; i < NPL * 4; ++i) v[i] = 0.f;
#pragma unroll
        for (int pl = 0; pl < NPL; ++pl)
            ws.own[pl][lane] = make_float4(v[4 * pl], v[4 * pl + 1], v[4 * pl + 2], v[4 * pl + 3]);
    }
    const unsigned long long has = __ballot(tot > 0);
    // the lane's first and last lists with candidates; the first list of the next lane with candidates
    int first = -1, last = -1;
#pragma unroll
    for (int m = W - 1; m >= 0; --m)
        if (cnt[m] > 0) first = m * 64 + lane;
#pragma unroll
    for (int m = 0; m < W; ++m)
        if (cnt[m] > 0) last = m * 64 + lane;
    const unsigned long long after = has & ~((2ull << lane) - 1);
    const int nfirst = __shfl(first, after ? __ffsll((long long)after) - 1 : lane);
    const int wlast = __builtin_amdgcn_readlane(last, 63 - __clzll(has));
    {
        int carry = after ? nfirst : -1;                // (the wave's last list links to itself)
#pragma unroll
        for (int m = W - 1; m >= 0; --m) {
            const int e = m * 64 + lane;
            ws.ent[e] = make_int2((off[m] + 1) | (cnt[m] << 21), (carry < 0 ? e : carry) | (e << 9) | (ntr[m] << 18));
            ws.k1[m][lane] = ~0u;
            ws.k2[m][lane] = ~0u;
            if (cnt[m] > 0) carry = e;
        }
    }
    const int R = (total + 63) >> 6;                    // pieces a walker
    {
        int np[W];
#pragma unroll
        for (int m = 0; m < W; ++m) np[m] = (cnt[m] + CH - 1) >> CSH;
        deal_marks<W, 9, true>(ws.mark, np, incl - tot, R);
    }
    wave_sync();
    const int p0 = (int)__umul24((unsigned)lane, (unsigned)R);   // this walker's first piece
    // walk state: the piece's list, its piece number, the list's length and first entry, the next list's entry
    int o, j;
    if (p0 < total) {
        const int mk = ws.mark[lane];
        o = mk & 511;
        j = mk >> 9;
    } else {                                            // (a walker with no pieces starts on the last list)
        o = wlast;
        j = 0;
    }
    int2 nx;
    int ocnt, ol, on;
    {
        const int2 oe = ws.ent[o];
        ocnt = oe.x >> 21;
        ol = oe.x & OFF_MASK;
        on = oe.y >> 18;
        nx = ws.ent[oe.y & 511];
    }
    // evaluation state: the list (id, first trial, trials), its owner's values, the walker's two least keys a trial
    int cur = -1, cm = 0, cn = 0;
    float nwx[8], w[8], C, sc[W];
    unsigned r1[W], r2[W];
#pragma unroll
    for (int t = 0; t < W; ++t) r1[t] = r2[t] = ~0u;
    // the walker's pairs into the list's pairs, for the list's trials (a trial outside them offers ~0u, which changes
    // nothing): the first slots' atomics all issued, then the second slots' (no branch a trial, so the atomics of the
    // trials overlap instead of waiting one after another)
    auto flush = [&]() {
        unsigned o[W];
#pragma unroll
        for (int t = 0; t < W; ++t)
            o[t] = atomicMin(&ws.k1[t][cur & 63], (unsigned)(t - cm) < (unsigned)cn ? r1[t] : ~0u);
#pragma unroll
        for (int t = 0; t < W; ++t)   // (the second least of the slot's old key and the walker's two)
            atomicMin(&ws.k2[t][cur & 63], (unsigned)(t - cm) < (unsigned)cn ? umed3(o[t], r1[t], r2[t]) : ~0u);
    };
    int idx[CH];
#pragma unroll
    for (int r = 0; r < CH; ++r) idx[r] = __builtin_amdgcn_raw_buffer_load_b16(nrs, (ol + (j << CSH) + r) * 2, 0, 0);
    for (int rd = 0; rd < R; ++rd) {
        // the next piece: the list's next, or the next list's first; its list entries read now
        int o2 = o, j2 = j + 1, ocnt2 = ocnt, ol2 = ol, on2 = on;
        int2 nx2 = nx;
        if ((j2 << CSH) >= ocnt) {
            o2 = (nx.y >> 9) & 511;
            ocnt2 = nx.x >> 21;
            ol2 = nx.x & OFF_MASK;
            on2 = nx.y >> 18;
            j2 = 0;
            nx2 = ws.ent[nx.y & 511];
        }
        int idx2[CH];
        if (rd + 1 < R) {                               // (wave-uniform)
#pragma unroll
            for (int r = 0; r < CH; ++r)
                idx2[r] = __builtin_amdgcn_raw_buffer_load_b16(nrs, (ol2 + (j2 << CSH) + r) * 2, 0, 0);
        }
        // a new list: merge the pairs of the last one, read the owner's values
        if (o != cur) {
            if (cur >= 0) flush();
            cur = o;
            cm = o >> 6;
            cn = on;
            const int ow = o & 63;
#pragma unroll
            for (int pl = 0; pl < 2; ++pl) {
                const float4 a = ws.own[pl][ow], b = ws.own[2 + pl][ow];
                nwx[4 * pl] = a.x; nwx[4 * pl + 1] = a.y; nwx[4 * pl + 2] = a.z; nwx[4 * pl + 3] = a.w;
                w[4 * pl] = b.x; w[4 * pl + 1] = b.y; w[4 * pl + 2] = b.z; w[4 * pl + 3] = b.w;
            }
            float v[NPL * 4 - 16];
#pragma unroll
            for (int pl = 4; pl < NPL; ++pl) {
                const float4 a = ws.own[pl][ow];
                v[4 * (pl - 4)] = a.x; v[4 * (pl - 4) + 1] = a.y; v[4 * (pl - 4) + 2] = a.z; v[4 * (pl - 4) + 3] = a.w;
            }
            C = v[0];
#pragma unroll
            for (int t = 0; t < W; ++t) {
                sc[t] = v[1 + t];
                r1[t] = r2[t] = ~0u;
            }
        }
        // this piece's candidates (positions past the list's end or pieces past the wave's total: no key)
        const bool pv = p0 + rd < total;
        uint64_t pt[CH];
        unsigned low[CH];
#pragma unroll
        for (int r = 0; r < CH; ++r) {
            const bool v = pv && (j << CSH) + r < ocnt;
            low[r] = v ? (unsigned)idx[r] : ~0u;
            pt[r] = grid[idx[r] & (NG - 1)];
        }
#pragma unroll
        for (int r = 0; r < CH; ++r) {
            const uint32_t lo = (uint32_t)pt[r], hi = (uint32_t)(pt[r] >> 32);
            // (B: -2 sum (w x) q. The first terms are products: an fma with a zero addend rounds the same, up to the
            // sign of a zero, which the key clears)
            float A = 0.f, B = 0.f;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float q = small_int_f((float)(((i < 4 ? lo : hi) >> (8 * (i % 4))) & 0xffu));
                A = i ? fmaf(w[i], q * q, A) : w[0] * (q * q);
                B = i ? fmaf(nwx[i], q, B) : nwx[0] * q;
            }
#pragma unroll
            for (int t = 0; t < W; ++t) {
                const float D = fmaf(sc[t], fmaf(sc[t], A, B), C);
                const unsigned key = (__float_as_uint(D) & KHI) | low[r];
                r2[t] = umed3(r1[t], r2[t], key);   // (r1 <= r2: the second least of the three)
                r1[t] = r1[t] < key ? r1[t] : key;
            }
        }
        o = o2; j = j2; ocnt = ocnt2; ol = ol2; on = on2; nx = nx2;
#pragma unroll
        for (int r = 0; r < CH; ++r) idx[r] = idx2[r];
    }
    flush();
    wave_sync();
#pragma unroll
    for (int t = 0; t < W; ++t) {
        k1[t] = ws.k1[t][lane];
        k2[t] = ws.k2[t][lane];
    }
}

// The test on a trial's key pair (see the top of this file): the grid index of ggml's pick, or -1 when the filter
// cannot decide it (the exact search must). sw = sum w, swx = sum w |x|, swxx = sum w x^2 of the group, s the trial
// scale.
template <int IB> DEV int filt_pick(unsigned k1, unsigned k2, float s, float sw, float swx, float swxx) {
    constexpr unsigned KM = (1u << IB) - 1;
    const float smax = fmaf(s * s, 49.f * sw, fmaf(14.f * s, swx, swxx));
    const float delta = smax * 0x1p-19f;
    bool ok = smax >= 0x1p-60f && smax <= 0x1p100f && k1 != ~0u;
    const float up1 = __uint_as_float((k1 & ~KM) + KM + 1);
    ok = ok && up1 + delta < FLT_MAX;
    ok = ok && (k2 == ~0u || __uint_as_float(k2 & ~KM) - up1 > 2.002f * delta);
    return ok ? (int)(k1 & KM) : -1;
}
