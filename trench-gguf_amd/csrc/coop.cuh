// trench-gguf_amd/csrc/coop.cuh - the wave-cooperative neighbour search of the i-quants.
//
// The reference scans a key's neighbour list serially on the thread that owns the key (gpuq/gpuq.hip:178-197,
// 199-232, 971-992). Lists are 1 to ~190 points long, so a wave scanning its lanes' lists side by side runs as long
// as its longest list while most lanes idle. Here the lists of the wave's 64 lanes are concatenated in lane order and
// dealt out 64 candidates a round, one a lane, so every lane does useful work until the wave's total is exhausted.
//
// A candidate's distance is computed from the owner's values exactly as the serial scan computes it (same operands,
// same operation order), and each list's winner is the minimum of (distance bits, list position) over its
// candidates, taken with LDS atomic mins. A distance is a sum of w*diff*diff terms from +0; with w >= 0 (or NaN
// weights) it is never negative and never -0, so the unsigned order of its bits is the float order, with NaN above
// +inf. Negative weights (ggml takes any importance) make negative distances, which the serial scan accepts like any
// other: the searches of a wave with a negative staged weight (SIGNED) map each distance to an order-preserving key
// instead (-0 read as +0, NaN above everything). The smallest position among equal distances is the serial scan's
// first-wins rule (it replaces only on a strictly smaller distance), and a minimum at or above FLT_MAX is the serial
// scan accepting nothing (best starts at FLT_MAX, strict <; NaN is never accepted): the reference traps there, the
// caller flags it.
//
// The deal: the wave's lists occupy consecutive ranges of one concatenation (a wave prefix sum). With
// R = ceil(total / 64) rounds, lane L takes the contiguous run of positions [L*R, L*R + R): mostly one list's
// consecutive candidates, so the lane keeps that list's owner values in registers, keeps a running minimum, and issues
// one atomic min per list it visits rather than one per candidate (many lanes of one list hitting one LDS address in
// the same instruction serialize). A lane finds the list of its first position from a table the owners fill (each
// owner marks the lanes whose first position falls in its list), then walks on to the next list with candidates when
// the current one ends.
#pragma once
#include "frame.cuh"

// per-wave LDS workspace of the search with M lists a lane. List m of lane L has the id e = m*64 + L (the search
// order is lane by lane, list by list; the ids are laid out list-major so that the 64 lanes' writes of one list's
// fields hit consecutive addresses). The owner values are staged in NP rows a lane, row e mod 64 NP for list e:
// NP = 1 (PL = false) when the lane's M lists search for one group (row L), NP = M (PL = true) for M groups of the
// lane (row e), or a divisor of M for M/NP searches of NP groups each (list m uses group m mod NP). A row holds SW
// floats: NV x's then NV weights (SW = 2 NV), stored as SW/4 planes of float4 so that the lanes' staging writes are
// consecutive too. The lists' scales are kept in ES rows a lane: ES = M (one a list), or a divisor of M when the
// lists come in runs of M/ES with one scale (list m's scale row: m / (M / ES)). List ids take LB bits (8 up to 4 lists
// a lane, 9 up to 8).
template <int M, int SW = 16, bool PL = false, int NP = (PL ? M : 1), int ES = M> struct CoopWSM {
    static_assert(M == 1 || M == 2 || M == 4 || M == 6 || M == 8, "lists a lane: 1, 2, 4, 6 or 8");
    static_assert(NP >= 1 && NP <= M && M % NP == 0, "staged rows a lane: a divisor of M");
    static_assert(ES >= 1 && ES <= M && M % ES == 0, "scale rows a lane: a divisor of M");
    static_assert(SW == 8 || SW == 16, "staged values: 4 or 8 x's and weights");
    static constexpr int sw = SW;
    static constexpr int np = NP;
    static constexpr int es = ES;
    static constexpr int LB = M <= 4 ? 8 : 9;
    float4 stage[SW / 4][64 * NP];
    int2 ent[64 * M];               // list e: first point's offset | length << 21, next list with candidates | e << LB
    float esc[64 * ES];             // scale row r: its lists' scale
    unsigned long long key[64 * M]; // list e: min of (distance bits << 32 | list position << 12 | grid index)
    int mark[64];                   // walker lane: the list of its first position | position in that list << LB
};
template <int M, int SW = 16, bool PL = false, int NP = (PL ? M : 1), int ES = M> constexpr int coop_wsm_bytes() {
    return (int)sizeof(CoopWSM<M, SW, PL, NP, ES>);
}
using CoopWS = CoopWSM<1>;
static constexpr int COOP_WS_BYTES = (int)sizeof(CoopWS);

// write this lane's values for the search: n values and n weights (slot: the lane, or with several staged rows a
// lane the row m*64 + lane of the lane's group m)
template <int NV, class W> DEV void coop_stage(W &ws, const float *xv, const float *wv, int slot = -1) {
    static_assert(2 * NV <= W::sw, "staged row too small");
    const int row = slot < 0 ? lane_id() : slot;
#pragma unroll
    for (int i = 0; i < NV / 4; ++i) {
        ws.stage[i][row] = make_float4(xv[4 * i], xv[4 * i + 1], xv[4 * i + 2], xv[4 * i + 3]);
        ws.stage[NV / 4 + i][row] = make_float4(wv[4 * i], wv[4 * i + 1], wv[4 * i + 2], wv[4 * i + 3]);
    }
}

// an owner's staged values into registers
template <class W> DEV void coop_fetch(const W &ws, int owner, float (&st)[16]) {
#pragma unroll
    for (int i = 0; i < W::sw / 4; ++i) {
        const float4 v = ws.stage[i][owner];
        st[4 * i] = v.x; st[4 * i + 1] = v.y; st[4 * i + 2] = v.z; st[4 * i + 3] = v.w;
    }
}

// a / b for 0 <= a < 2^20, 1 <= b < 2^12: a float quotient (hardware reciprocal, within 1 of the floor), corrected
// to the floor; the products stay below 2^32 with 24-bit operands (full-rate multiplies)
DEV int div_small(int a, int b) {
    int q = (int)((float)a * __builtin_amdgcn_rcpf((float)b));
    q += (int)__umul24((unsigned)(q + 1), (unsigned)b) <= a;
    q -= (int)__umul24((unsigned)q, (unsigned)b) > a;
    return q;
}

// The deal's mark table: walker L's first piece is L*R; this lane's lists hold pieces [s0, s0 + sum np) of the wave's
// concatenation, list m the np[m] pieces after those of lists 0..m-1. For each walker whose first piece falls in
// them (at most a few: the lane's pieces over R), mark[L] = (m*64 + lane) | (the piece's number in list m << SH).
// INC: list by list, the walkers starting in it R pieces apart (a few instructions a walker, a loop a list: for many
// lists a lane or many walkers a lane); else walker by walker, each finding its list among the M (fewer loops).
template <int M, int SH, bool INC = M >= 6>
DEV void deal_marks(int *mark, const int (&np)[M], int s0, int R) {
    const int lane = lane_id();
    if (INC) {
        int L = div_small(s0 + R - 1, R);               // the first walker starting among the lane's pieces
        int j = (int)__umul24((unsigned)L, (unsigned)R) - s0;   // its first piece, counted from list m's first
#pragma unroll
        for (int m = 0; m < M; ++m) {
            while (j < np[m] && L < 64) {
                mark[L] = (m * 64 + lane) | (j << SH);
                ++L;
                j += R;
            }
            j -= np[m];
        }
        return;
    }
    int tot = 0;
#pragma unroll
    for (int m = 0; m < M; ++m) tot += np[m];
    const int lf = div_small(s0 + R - 1, R);
    const int ll = div_small(s0 + tot - 1, R);          // (no pieces: ll < lf)
    for (int L = lf; L <= ll && L < 64; ++L) {
        int j = (int)__umul24((unsigned)L, (unsigned)R) - s0;   // the walker's first piece among the lane's
        int m = M - 1;
        bool found = false;
#pragma unroll
        for (int i = 0; i < M; ++i) {                    // the list holding it (lists of no pieces skipped)
            const bool hit = !found && j < np[i];
            m = hit ? i : m;
            j = found || hit ? j : j - np[i];
            found = found || hit;
        }
        mark[L] = (m * 64 + lane) | (j << SH);
    }
}

// inclusive prefix sum over the wave's 64 lanes (DPP: shifts within rows of 16, then the row broadcasts)
DEV int wave_incl_scan(int v) {
    v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xf, 0xf, true);      // row_shr:1 (lanes shifted in read 0)
    v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xf, 0xf, true);      // row_shr:2
    v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, true);      // row_shr:4
    v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xf, true);      // row_shr:8
    v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xa, 0xf, false);     // row_bcast:15 into rows 1 and 3
    v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xc, 0xf, false);     // row_bcast:31 into rows 2 and 3
    return v;
}

// All 64 lanes call this together (wave-uniform control flow), each with M lists of its own: cnt[m] the length of
// list m (0: no search), off[m] its offset in neigh (count at neigh[off], points from neigh[off + 1]; off + 1 < 2^21,
// cnt < 2^10), scale[m] its scale. The lane's values (shared by its M lists) must have been staged (coop_stage) when
// any cnt[m] > 0. gi[m]: the winning grid index (-1: no candidate accepted; -2: cnt[m] == 0).
// ev.point(idx): grid point idx (< 4096) as stored; ev(st, scale, pt): its distance for the owner's staged values st
// (16 floats).
//
// The deal: each list is cut into pieces of CH consecutive candidates; the wave's pieces are concatenated lane by
// lane, list by list (ids m*64 + lane, so M searches of every lane share one set-up and one last, partly filled
// round), and walker L takes the contiguous run of R = ceil(pieces / 64) pieces from L*R, one a round. A walker
// changes lists only between rounds, so the list changes (merge the running minimum, read the new owner's values and
// scale) come once a round for the wave rather than at any position; within a round every walker evaluates the CH
// candidates of one piece (positions past the list's end are masked). The next piece's list entries are read while
// the current piece is evaluated. Along a walker's run a list's positions come in increasing order, so a strictly
// smaller distance alone keeps the first of equal ones; the (distance, position) minimum across walkers is taken once
// per list visited.
// a distance's key in float order for any sign: -0 as +0, negatives below +0 in reverse bit order, NaN above all
DEV unsigned signed_key(float d) {
    const unsigned b = d == 0.f ? 0u : __float_as_uint(d);
    const unsigned k = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    return d != d ? ~0u : k;
}

// An Eval with LIST_POINTS = true reads its candidates' grid points from ev.npt, an array beside the lists with the
// same offsets, in the same load as the list entry (no grid read a candidate); the winner's grid index is then read
// from the list at its position, once a list.
template <class E, class = void> struct list_points { static constexpr bool value = false; };
template <class E> struct list_points<E, decltype((void)E::LIST_POINTS)> { static constexpr bool value = E::LIST_POINTS; };

// FIRST_WAIT: wait for the first round's list entries before the rounds start. The compiler otherwise merges the
// loop's entry (those loads pending) with its back edge and waits for each round's prefetched entries at the start
// of that round; with the wait its waits move to the round's end. It pays for IQ1's long lists (IQ1_M 0.7% faster)
// and costs the shorter searches 1% (the other wave of the SIMD already covers the latency there).
template <int M, int CH = 4, bool SIGNED = false, bool FIRST_WAIT = false, class Eval, int SW, bool PL, int NP,
          int ES>
DEV void coop_search_m(const int (&cnt)[M], const int (&off)[M], const float (&scale)[M], const uint16_t *neigh,
                       int neigh_len, CoopWSM<M, SW, PL, NP, ES> &ws, const Eval &ev, int (&gi)[M]) {
    static_assert(CH == 1 || CH == 2 || CH == 4 || CH == 8, "piece size: a power of two");
    constexpr int CSH = CH == 1 ? 0 : CH == 2 ? 1 : CH == 4 ? 2 : 3;
    constexpr int ROWS = 64 * NP - 1;                   // list e's staged row: e & ROWS
    constexpr int OFF_MASK = (1 << 21) - 1;
    constexpr int LB = CoopWSM<M, SW, PL, NP, ES>::LB, IDM = (1 << LB) - 1;
    constexpr int SR = M / ES;                          // lists a scale row
    auto srow = [](int e) { return SR == 1 ? e : ((e >> 6) / SR) * 64 + (e & 63); };
    // the lists (or their points) through a buffer resource: 32-bit offsets, and reads past the table return 0
    // instead of faulting
    constexpr bool LP = list_points<Eval>::value;
    const void *lbase = neigh;
    if constexpr (LP) lbase = ev.npt;
    const __amdgpu_buffer_rsrc_t nrs =
        __builtin_amdgcn_make_buffer_rsrc((void *)lbase, 0, neigh_len * (LP ? 4 : 2), 0x00020000);
    auto entry = [&](int e) -> int {    // list element e: its grid index, or (LP) its point's bits
        if constexpr (LP) return (int)__builtin_amdgcn_raw_buffer_load_b32(nrs, e * 4, 0, 0);
        else return __builtin_amdgcn_raw_buffer_load_b16(nrs, e * 2, 0, 0);
    };
    const int lane = lane_id();
    int tot = 0;
#pragma unroll
    for (int m = 0; m < M; ++m) tot += (cnt[m] + CH - 1) >> CSH;
    const int incl = wave_incl_scan(tot);
    const int total = __builtin_amdgcn_readlane(incl, 63);
#pragma unroll
    for (int m = 0; m < M; ++m) gi[m] = -2;
    if (total == 0) return;                             // wave-uniform
    const unsigned long long has = __ballot(tot > 0);
    // the lane's first and last lists with candidates; the first list of the next lane with candidates
    int first = -1, last = -1;
#pragma unroll
    for (int m = M - 1; m >= 0; --m)
        if (cnt[m] > 0) first = m * 64 + lane;
#pragma unroll
    for (int m = 0; m < M; ++m)
        if (cnt[m] > 0) last = m * 64 + lane;
    const unsigned long long after = has & ~((2ull << lane) - 1);
    const int nfirst = __shfl(first, after ? __ffsll((long long)after) - 1 : lane);
    // the wave's last list (read here, in wave-uniform control flow: a lane read inside a branch may not have been
    // computed there)
    const int wlast = __builtin_amdgcn_readlane(last, 63 - __clzll(has));
    {
        int carry = after ? nfirst : -1;                // (the wave's last list links to itself)
#pragma unroll
        for (int m = M - 1; m >= 0; --m) {
            const int e = m * 64 + lane;
            ws.ent[e] = make_int2((off[m] + 1) | (cnt[m] << 21), (carry < 0 ? e : carry) | (e << LB));
            if (SR == 1 || m % SR == 0) ws.esc[srow(e)] = scale[m];
            ws.key[e] = ~0ull;
            if (cnt[m] > 0) carry = e;
        }
    }
    const int R = (total + 63) >> 6;                    // pieces a walker
    {
        int np[M];
#pragma unroll
        for (int m = 0; m < M; ++m) np[m] = (cnt[m] + CH - 1) >> CSH;
        deal_marks<M, LB>(ws.mark, np, incl - tot, R);
    }
    wave_sync();
    const int p0 = (int)__umul24((unsigned)lane, (unsigned)R);   // this walker's first piece
    // walk state: the piece's list, its piece number, the list's length and first entry, the next list's entry
    int o, j;
    if (p0 < total) {
        const int mk = ws.mark[lane];
        o = mk & IDM;
        j = mk >> LB;
    } else {                                            // (a walker with no pieces starts on the last list)
        o = wlast;
        j = 0;
    }
    int2 nx;
    int ocnt, ol;
    {
        const int2 oe = ws.ent[o];
        ocnt = oe.x >> 21;
        ol = oe.x & OFF_MASK;
        nx = ws.ent[oe.y & IDM];
    }
    // evaluation state: the list being evaluated, its owner's values and scale, the best distance bits and position
    int cur = -1;
    float st[16], sc = 0.f;
    unsigned bbits = ~0u;
    int bpos = 0, bidx = 0;
    int idx[CH];
#pragma unroll
    for (int r = 0; r < CH; ++r) idx[r] = entry(ol + (j << CSH) + r);
    if (FIRST_WAIT) __builtin_amdgcn_s_waitcnt(0xF70);  // vmcnt(0), expcnt and lgkmcnt unconstrained
    for (int rd = 0; rd < R; ++rd) {
        // the next piece: the list's next, or the next list's first; its list entries read now
        int o2 = o, j2 = j + 1, ocnt2 = ocnt, ol2 = ol;
        int2 nx2 = nx;
        if ((j2 << CSH) >= ocnt) {
            o2 = nx.y >> LB;
            ocnt2 = nx.x >> 21;
            ol2 = nx.x & OFF_MASK;
            j2 = 0;
            nx2 = ws.ent[nx.y & IDM];
        }
        int idx2[CH];
        if (rd + 1 < R) {                               // (wave-uniform)
#pragma unroll
            for (int r = 0; r < CH; ++r)
                idx2[r] = entry(ol2 + (j2 << CSH) + r);
        }
        // a new list: merge the minimum of the last one, read the owner's values and scale
        if (o != cur) {
            if (cur >= 0) atomicMin(&ws.key[cur], ((unsigned long long)bbits << 32) | (unsigned)(bpos << 12 | bidx));
            if (NP == M || cur < 0 || ((o ^ cur) & ROWS)) coop_fetch(ws, o & ROWS, st);
            sc = ws.esc[srow(o)];
            cur = o;
            bbits = ~0u;
        }
        // this piece's candidates (positions past the list's end or pieces past the wave's total: no distance)
        const bool pv = p0 + rd < total;
        decltype(ev.point(0)) pt[CH];
        bool v[CH];
#pragma unroll
        for (int r = 0; r < CH; ++r) {
            v[r] = pv && (j << CSH) + r < ocnt;
            if constexpr (LP) pt[r] = (decltype(ev.point(0)))(unsigned)idx[r];   // (a masked position: any point)
            else pt[r] = ev.point(v[r] ? idx[r] : 0);   // (a masked position reads point 0)
        }
#pragma unroll
        for (int r = 0; r < CH; ++r) {
            const int pos = (j << CSH) + r;
            const float dv = ev(st, sc, pt[r]);
            const unsigned b = v[r] ? (SIGNED ? signed_key(dv) : __float_as_uint(dv)) : ~0u;
            const bool lt = b < bbits;                  // (selects, not a branch)
            bbits = lt ? b : bbits;
            bpos = lt ? pos : bpos;
            if constexpr (!LP) bidx = lt ? idx[r] : bidx;
        }
        o = o2; j = j2; ocnt = ocnt2; ol = ol2; nx = nx2;
#pragma unroll
        for (int r = 0; r < CH; ++r) idx[r] = idx2[r];
    }
    atomicMin(&ws.key[cur], ((unsigned long long)bbits << 32) | (unsigned)(bpos << 12 | bidx));
    wave_sync();
    // the winners: a minimum at or above FLT_MAX (or NaN) is nothing accepted
    constexpr unsigned KMAX = SIGNED ? 0xff7fffffu : 0x7f7fffffu;   // FLT_MAX's key
#pragma unroll
    for (int m = 0; m < M; ++m) {
        if (cnt[m] > 0) {
            const unsigned long long k = ws.key[m * 64 + lane];
            if constexpr (LP)   // the winner's index from the list, at its position
                gi[m] = (unsigned)(k >> 32) >= KMAX ? -1 : (int)neigh[off[m] + 1 + (int)((k >> 12) & 0xfffffu)];
            else
                gi[m] = (unsigned)(k >> 32) >= KMAX ? -1 : (int)(k & 0xfffu);
        }
    }
}

// the search with one list a lane: returns gi (see coop_search_m)
template <int CH = 4, bool SIGNED = false, class Eval>
DEV int coop_search(int cnt, int off, float scale, const uint16_t *neigh, int neigh_len, CoopWS &ws,
                    const Eval &ev) {
    const int c[1] = {cnt}, o[1] = {off};
    const float s[1] = {scale};
    int g[1];
    coop_search_m<1, CH, SIGNED>(c, o, s, neigh, neigh_len, ws, ev, g);
    return g[0];
}
