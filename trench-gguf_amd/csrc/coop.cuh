// trench-gguf_amd/csrc/coop.cuh - the wave-cooperative neighbour search of the i-quants.
//
// The reference scans a key's neighbour list serially on the thread that owns the key (gpuq/gpuq.hip:178-197,
// 199-232, 971-992). Lists are 1 to ~190 points long, so a wave scanning its lanes' lists side by side runs as long
// as its longest list while most lanes idle. Here the lists of the wave's 64 lanes are concatenated in lane order and
// dealt out 64 candidates a round, one a lane, so every lane does useful work until the wave's total is exhausted.
//
// A candidate's distance is computed from the owner's values exactly as the serial scan computes it (same operands,
// same operation order), and each owner's winner is the minimum of (distance bits, list position) over its
// candidates, taken with LDS atomic mins. A distance is a sum of w*diff*diff terms from +0 with w >= 0 (or NaN
// weights), so it is never negative and never -0: the unsigned order of its bits is the float order, with NaN above
// +inf. The smallest position among equal distances is the serial scan's first-wins rule (it replaces only on a
// strictly smaller distance), and a minimum at or above FLT_MAX is the serial scan accepting nothing (best starts at
// FLT_MAX, strict <): the reference traps there, the caller flags it.
//
// The deal: lane L's list occupies positions [excl_L, incl_L) of the concatenation (a wave prefix sum). With
// R = ceil(total / 64) rounds, lane L takes the contiguous run of positions [L*R, L*R + R): mostly one owner's
// consecutive candidates, so the lane keeps that owner's values in registers, keeps a running minimum, and issues one
// atomic min per owner it visits rather than one per candidate (many lanes of one owner hitting one LDS address in
// the same instruction serialize). A lane finds the owner of its first position from a byte table the owners fill
// (each owner marks the lanes whose first position falls in its range), then walks on to the next lane with a list
// when the current owner's list ends.
#pragma once
#include "frame.cuh"

// per-wave LDS workspace of the search
struct CoopWS {
    float stage[64][16];        // an owner's values: 8 (or 4) x's then 8 (or 4) weights
    int4 info[64];              // owner: list offset, first position, scale bits, list length | next owner << 16
    int2 nxt[64];               // owner: its next owner's list offset, list length | the one after it << 16
    unsigned long long key[64]; // owner: min of (distance bits << 32 | list position << 12 | grid index)
    uint8_t mark[64];           // lane: the owner of its first position
};
static constexpr int COOP_WS_BYTES = (int)sizeof(CoopWS);

// write this lane's values for the search: n values and n weights
template <int NV, class W> DEV void coop_stage(W &ws, const float *xv, const float *wv) {
    float4 *s = (float4 *)ws.stage[lane_id()];
#pragma unroll
    for (int i = 0; i < NV / 4; ++i) {
        s[i] = make_float4(xv[4 * i], xv[4 * i + 1], xv[4 * i + 2], xv[4 * i + 3]);
        s[NV / 4 + i] = make_float4(wv[4 * i], wv[4 * i + 1], wv[4 * i + 2], wv[4 * i + 3]);
    }
}

// an owner's staged values into registers
template <class W> DEV void coop_fetch(const W &ws, int owner, float (&st)[16]) {
    const float4 *sp = (const float4 *)ws.stage[owner];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float4 v = sp[i];
        st[4 * i] = v.x; st[4 * i + 1] = v.y; st[4 * i + 2] = v.z; st[4 * i + 3] = v.w;
    }
}

// a / b for 0 <= a < 2^20, 1 <= b < 2^12: a float quotient (hardware reciprocal, within 1 of the floor), corrected
// to the floor
DEV int div_small(int a, int b) {
    int q = (int)((float)a * __builtin_amdgcn_rcpf((float)b));
    q += (q + 1) * b <= a;
    q -= q * b > a;
    return q;
}

// inclusive prefix sum over the wave's 64 lanes (DPP: shifts within rows of 16, then the row broadcasts)
DEV int wave_incl_scan(int v) {
    v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xf, 0xf, false);     // row_shr:1
    v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xf, 0xf, false);     // row_shr:2
    v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, false);     // row_shr:4
    v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xf, false);     // row_shr:8
    v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xa, 0xf, false);     // row_bcast:15 into rows 1 and 3
    v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xc, 0xf, false);     // row_bcast:31 into rows 2 and 3
    return v;
}

// All 64 lanes call this together (wave-uniform control flow). cnt: the lane's list length (0: no search), off: the
// list's offset in neigh (count at neigh[off], points from neigh[off + 1]), scale: the owner's scale. The lane's
// values must have been staged (coop_stage) when cnt > 0.
// Returns, for cnt > 0, the winning grid index (-1: no candidate accepted); for cnt == 0, -2.
// ev.point(idx): grid point idx (< 4096) as stored; ev(st, scale, pt): its distance for the owner's staged values st
// (16 floats).
//
// Rounds run in chunks of up to 8: a first pass walks the chunk's positions (owner, list position) and issues their
// list reads, a second reads their grid points, a third evaluates them, so a chunk's reads are in flight together.
template <class Eval>
DEV int coop_search(int cnt, int off, float scale, const uint16_t *neigh, int neigh_len, CoopWS &ws,
                    const Eval &ev) {
    // the lists through a buffer resource: 32-bit offsets, and reads past the table return 0 instead of faulting
    const __amdgpu_buffer_rsrc_t nrs = __builtin_amdgcn_make_buffer_rsrc((void *)neigh, 0, neigh_len * 2, 0x00020000);
    const int lane = lane_id();
    const int incl = wave_incl_scan(cnt);
    const int total = __builtin_amdgcn_readlane(incl, 63);
    if (total == 0) return -2;                          // wave-uniform
    const int excl = incl - cnt;
    const unsigned long long has = __ballot(cnt > 0);
    const unsigned long long after = has & ~((2ull << lane) - 1);
    const int next = after ? __ffsll((long long)after) - 1 : lane;     // the next lane with a list
    ws.info[lane] = make_int4(off, excl, __float_as_int(scale), cnt | (next << 16));
    {
        const int noff = __shfl(off, next), ncnt = __shfl(cnt, next), nnext = __shfl(next, next);
        ws.nxt[lane] = make_int2(noff, ncnt | (nnext << 16));
    }
    ws.key[lane] = ~0ull;
    const int R = (total + 63) >> 6;                    // positions a lane
    if (cnt > 0) {                                      // lanes L with excl <= L*R < incl start in this list
        const int lf = div_small(excl + R - 1, R);
        const int ll = div_small(incl - 1, R);
        for (int L = lf; L <= ll && L < 64; ++L) ws.mark[L] = (uint8_t)lane;
    }
    wave_sync();
    const int p0 = lane * R;
    const int np = total - p0 < R ? (total - p0 > 0 ? total - p0 : 0) : R;   // this lane's positions
    // walk state: owner, list position, the owner's list length and its first entry
    int o = ws.mark[lane] & 63;
    if (np == 0) o = 63 - __clzll(has);                 // (idle lane: repeats the last owner's candidates)
    const int4 oi = ws.info[o];
    int ocnt = oi.w & 0xffff;
    int ol = oi.x + 1;                                  // the owner's first list entry
    int onext = oi.w >> 16;                             // the owner after it, and that owner's list (read ahead)
    int2 nx = ws.nxt[o];
    int j = np ? p0 - oi.y : 0;
    // evaluation state: the owner whose values are in registers, and the running minimum over its candidates
    int cur = o;
    float st[16], sc = __int_as_float(oi.z);
    unsigned long long kmin = ~0ull;
    coop_fetch(ws, o, st);
    for (int r0 = 0; r0 < R; r0 += 8) {
        const int rend = R - r0 < 8 ? R - r0 : 8;
        int own_j[8], idx[8];           // owner | list position << 6; the candidate's grid index
        uint64_t pt[8];                 // the candidate's grid point
        // walk: past this lane's positions the walk stays in the owner it is in (list position clamped), so every
        // slot holds a valid candidate of that owner and repeats change no minimum
#pragma unroll
        for (int r = 0; r < 8; ++r) {
            if (r < rend) {
                if (j >= ocnt && r0 + r < np) {         // the owner's list ends: on to the next lane with a list
                    o = onext;
                    ol = nx.x + 1;
                    ocnt = nx.y & 0xffff;
                    onext = nx.y >> 16;
                    j = 0;
                    nx = ws.nxt[o];                     // (needed at the next change of owner only)
                }
                const int jc = j < ocnt ? j : ocnt - 1;
                own_j[r] = o | (jc << 6);
                idx[r] = __builtin_amdgcn_raw_buffer_load_b16(nrs, (ol + jc) * 2, 0, 0);
                ++j;
            }
        }
#pragma unroll
        for (int r = 0; r < 8; ++r)
            if (r < rend) pt[r] = ev.point(idx[r]);
#pragma unroll
        for (int r = 0; r < 8; ++r) {
            if (r < rend) {
                const int owner = own_j[r] & 63;
                if (owner != cur) {
                    atomicMin(&ws.key[cur], kmin);
                    cur = owner;
                    kmin = ~0ull;
                    coop_fetch(ws, owner, st);
                    sc = __int_as_float(ws.info[owner].z);
                }
                const float d2 = ev(st, sc, pt[r]);
                const unsigned long long key = ((unsigned long long)__float_as_uint(d2) << 32) |
                                               (((unsigned)(own_j[r] >> 6) << 12) | (unsigned)idx[r]);
                kmin = key < kmin ? key : kmin;
            }
        }
    }
    atomicMin(&ws.key[cur], kmin);
    wave_sync();
    if (cnt <= 0) return -2;
    const unsigned long long k = ws.key[lane];
    if ((unsigned)(k >> 32) >= 0x7f7fffffu) return -1;  // min distance >= FLT_MAX (or NaN): nothing accepted
    return (int)(k & 0xfffu);
}

// ------------------------------------------------------------------ several lists a lane
// The same search over M lists a lane (M = 2 or 4; the lane's values, staged once, and a scale per list): the wave's
// 64*M lists are concatenated lane by lane, list by list (list e = lane*M + m), and dealt out as above. One call then
// covers M searches of every lane, so the set-up and the last, partly filled round are paid once for the M.
// The stage sits at the start, as in CoopWS, so both searches can share one workspace and its staged values.
template <int M> struct CoopWSM {
    static_assert(M == 2 || M == 4, "lists a lane: 2 or 4");
    float stage[64][16];            // a lane's values: 8 x's then 8 weights
    int2 ent[64 * M];               // list e: offset | length << 21, the next list with candidates | e << 8
    float esc[64 * M];              // list e: its scale
    unsigned long long key[64 * M]; // list e: min of (distance bits << 32 | list position << 12 | grid index)
    int mark[64];                   // walker lane: the list of its first position | position in that list << 8
};
template <int M> constexpr int coop_wsm_bytes() { return (int)sizeof(CoopWSM<M>); }

// cnt[m]: the length of the lane's list m (0: no search), off[m]: its offset in neigh (packed as off | cnt << 21 must
// fit 31 bits: off < 2^21, cnt < 2^10), scale[m]: its scale. gi[m]: the winner (-1: none accepted; -2: cnt[m] == 0).
template <int M, class Eval>
DEV void coop_search_m(const int (&cnt)[M], const int (&off)[M], const float (&scale)[M], const uint16_t *neigh,
                       int neigh_len, CoopWSM<M> &ws, const Eval &ev, int (&gi)[M]) {
    constexpr int LM = M == 4 ? 2 : 1;
    const __amdgpu_buffer_rsrc_t nrs = __builtin_amdgcn_make_buffer_rsrc((void *)neigh, 0, neigh_len * 2, 0x00020000);
    const int lane = lane_id();
    int tot = 0;
#pragma unroll
    for (int m = 0; m < M; ++m) tot += cnt[m];
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
        if (cnt[m] > 0) first = lane * M + m;
#pragma unroll
    for (int m = 0; m < M; ++m)
        if (cnt[m] > 0) last = lane * M + m;
    const unsigned long long after = has & ~((2ull << lane) - 1);
    const int nfirst = __shfl(first, after ? __ffsll((long long)after) - 1 : lane);
    // the wave's last list (read here, in wave-uniform control flow: a lane read inside a branch may not have been
    // computed there)
    const int wlast = __builtin_amdgcn_readlane(last, 63 - __clzll(has));
    {
        int carry = after ? nfirst : -1;                // (the wave's last list links to itself)
#pragma unroll
        for (int m = M - 1; m >= 0; --m) {
            const int e = lane * M + m;
            ws.ent[e] = make_int2(off[m] | (cnt[m] << 21), (carry < 0 ? e : carry) | (e << 8));
            ws.esc[e] = scale[m];
            ws.key[e] = ~0ull;
            if (cnt[m] > 0) carry = e;
        }
    }
    const int R = (total + 63) >> 6;                    // positions a lane
    {
        int start = incl - tot;                         // the list's first position
#pragma unroll
        for (int m = 0; m < M; ++m) {
            if (cnt[m] > 0) {                           // walkers L with start <= L*R < start + cnt begin in list m
                const int lf = div_small(start + R - 1, R);
                const int ll = div_small(start + cnt[m] - 1, R);
                for (int L = lf; L <= ll && L < 64; ++L) ws.mark[L] = (lane * M + m) | ((L * R - start) << 8);
            }
            start += cnt[m];
        }
    }
    wave_sync();
    const int p0 = lane * R;
    const int np = total - p0 < R ? (total - p0 > 0 ? total - p0 : 0) : R;
    int o, j;
    if (np) {
        const int mk = ws.mark[lane];
        o = mk & 255;
        j = mk >> 8;
    } else {                                            // (idle lane: repeats the wave's last list's first candidate)
        o = wlast;
        j = 0;
    }
    const int2 oe = ws.ent[o];
    int ocnt = oe.x >> 21;
    int ol = (oe.x & ((1 << 21) - 1)) + 1;              // the list's first entry
    int2 nx = ws.ent[oe.y & 255];                       // the entry of the list after it (read ahead)
    int cur = o;
    float st[16], sc = ws.esc[o];
    unsigned long long kmin = ~0ull;
    coop_fetch(ws, o >> LM, st);
    for (int r0 = 0; r0 < R; r0 += 8) {
        const int rend = R - r0 < 8 ? R - r0 : 8;
        int own_j[8], idx[8];           // list | list position << 8; the candidate's grid index
        uint64_t pt[8];
#pragma unroll
        for (int r = 0; r < 8; ++r) {
            if (r < rend) {
                if (j >= ocnt && r0 + r < np) {
                    o = nx.y >> 8;
                    ol = (nx.x & ((1 << 21) - 1)) + 1;
                    ocnt = nx.x >> 21;
                    j = 0;
                    nx = ws.ent[nx.y & 255];
                }
                const int jc = j < ocnt ? j : ocnt - 1;
                own_j[r] = o | (jc << 8);
                idx[r] = __builtin_amdgcn_raw_buffer_load_b16(nrs, (ol + jc) * 2, 0, 0);
                ++j;
            }
        }
#pragma unroll
        for (int r = 0; r < 8; ++r)
            if (r < rend) pt[r] = ev.point(idx[r]);
#pragma unroll
        for (int r = 0; r < 8; ++r) {
            if (r < rend) {
                const int e = own_j[r] & 255;
                if (e != cur) {
                    atomicMin(&ws.key[cur], kmin);
                    if ((e ^ cur) >> LM) coop_fetch(ws, e >> LM, st);
                    cur = e;
                    kmin = ~0ull;
                    sc = ws.esc[e];
                }
                const float d2 = ev(st, sc, pt[r]);
                const unsigned long long key = ((unsigned long long)__float_as_uint(d2) << 32) |
                                               (((unsigned)(own_j[r] >> 8) << 12) | (unsigned)idx[r]);
                kmin = key < kmin ? key : kmin;
            }
        }
    }
    atomicMin(&ws.key[cur], kmin);
    wave_sync();
#pragma unroll
    for (int m = 0; m < M; ++m) {
        if (cnt[m] > 0) {
            const unsigned long long k = ws.key[lane * M + m];
            gi[m] = (unsigned)(k >> 32) >= 0x7f7fffffu ? -1 : (int)(k & 0xfffu);
        }
    }
}
