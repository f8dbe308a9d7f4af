/* oracle/gq_oracle.c - CPU oracle for the GGUF quantizer path. TEST INFRASTRUCTURE ONLY (see gq_oracle.h).
 *
 * A plain-C restatement of ggml's quantize_row_*_impl / *_ref searches and to_float, written from the reference's
 * executable statement of them, gpuq/gpuq.hip, which the reference documents as ggml-quants.c (llama.cpp bed0a8566,
 * re-checked on ac8e1694d) line for line (gpuq/gpuq.hip:1-17, README.md:513-524). Each function cites the lines it
 * follows. The arithmetic contract (the reference's exactness rules):
 *   - every float expression keeps the reference's operand order, evaluated left to right, with no contraction;
 *   - every accumulation runs in index order;
 *   - "/" and sqrtf are IEEE (SSE scalar), fp32 subnormals are kept;
 *   - nearest_int is the 12582912.f magic-number rounding (gpuq/gpuq.hip:108-112);
 *   - fp32 -> fp16 is ggml's bit-trick round-to-nearest-even (gpuq/gpuq.hip:91-106);
 *   - the stable sort orders by key with ties in index order (gpuq/gpuq.hip:234-243);
 *   - integer narrowing (int -> int8_t / uint8_t stores) is C's, as ggml's.
 * Where the reference would trap (a search with no candidate, gpuq/gpuq.hip:82-86) the oracle flags an error and the
 * call returns 0 bytes.
 */
#include "gq_oracle.h"

#include <float.h>
#include <math.h>
#include <pthread.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#define QK 256
#define EPS_GROUP 1e-15f
#define EPS_IQ2S 1e-8f
#define EPS_IQ1M 1e-7f
#define EPS_IQ1S 1e-12f
#define EPS_IQ3XXS 1e-8f
#define DELTA_IQ1 0.125f
#define NGRID_IQ1 2048
/* ggml's MAX / MIN (a > b ? a : b) with each argument evaluated once */
#define GMAX(a, b) ({ __typeof__(a) ga_ = (a); __typeof__(b) gb_ = (b); ga_ > gb_ ? ga_ : gb_; })
#define GMIN(a, b) ({ __typeof__(a) ga_ = (a); __typeof__(b) gb_ = (b); ga_ < gb_ ? ga_ : gb_; })

#ifdef GQO_COUNT_OPS
static __thread uint64_t t_ops;
static uint64_t g_ops;
static pthread_mutex_t g_ops_mu = PTHREAD_MUTEX_INITIALIZER;
#define OPS(n) (t_ops += (uint64_t)(n))
static void ops_flush(void) { pthread_mutex_lock(&g_ops_mu); g_ops += t_ops; t_ops = 0; pthread_mutex_unlock(&g_ops_mu); }
uint64_t gqo_ops_read_reset(void) { ops_flush(); pthread_mutex_lock(&g_ops_mu); uint64_t v = g_ops; g_ops = 0; pthread_mutex_unlock(&g_ops_mu); return v; }
#else
#define OPS(n) ((void)0)
static void ops_flush(void) {}
uint64_t gqo_ops_read_reset(void) { return 0; }
#endif
/* cost of one sqrtf / fp32 division in the op count: the length of a correctly rounded VALU expansion */
#define C_SQRT 8
#define C_DIV 10

static __thread int t_err;   /* a reference trap condition was hit in this thread */

/* path counters: how often a quantization reached a case the GPU treats apart (see gq_oracle.h); counted per
 * thread (a shared counter would serialise the threads on one cache line) and added up at the end of every chunk */
static uint64_t g_stat[GQO_NSTAT];
static __thread uint64_t t_stat[GQO_NSTAT];
#define STAT(i) (++t_stat[i])
static void stat_flush(void) {
    for (int i = 0; i < GQO_NSTAT; ++i) {
        if (t_stat[i]) __atomic_fetch_add(&g_stat[i], t_stat[i], __ATOMIC_RELAXED);
        t_stat[i] = 0;
    }
}
uint64_t gqo_stat_read_reset(int which) {
    if (which < 0 || which >= GQO_NSTAT) return 0;
    stat_flush();
    return __atomic_exchange_n(&g_stat[which], 0, __ATOMIC_RELAXED);
}

/* ------------------------------------------------------------------ scalar helpers (gpuq/gpuq.hip:88-112, 2108-2121) */
static inline uint32_t bits_of(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float float_of(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* ggml_compute_fp32_to_fp16: scale the magnitude so the fp32 adder rounds it to a half's precision (RNE), then
 * extract the half's exponent and mantissa bits; NaN -> 0x7E00 (gpuq/gpuq.hip:91-106) */
static uint16_t f32_to_f16(float f) {
    float base = (fabsf(f) * 0x1.0p+112f) * 0x1.0p-110f;
    const uint32_t w = bits_of(f);
    const uint32_t w2 = w + w;
    const uint32_t sgn = w & 0x80000000u;
    uint32_t bias = w2 & 0xFF000000u;
    if (bias < 0x71000000u) bias = 0x71000000u;
    base = float_of((bias >> 1) + 0x07800000u) + base;
    const uint32_t b = bits_of(base);
    const uint32_t nonsign = ((b >> 13) & 0x00007C00u) + (b & 0x00000FFFu);
    OPS(12);
    return (uint16_t)((sgn >> 16) | (w2 > 0xFF000000u ? 0x7E00u : nonsign));
}

/* exact half -> float (gpuq/gpuq.hip:2108-2120) */
static float f16_to_f32(uint16_t h) {
    const uint32_t sgn = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1f, m = h & 0x3ffu;
    if (e == 0) {
        if (m == 0) return float_of(sgn);
        int sh = 0;
        while (!(m & 0x400u)) { m <<= 1; ++sh; }
        return float_of(sgn | ((uint32_t)(113 - sh) << 23) | ((m & 0x3ffu) << 13));
    }
    if (e == 31) return float_of(sgn | 0x7f800000u | (m << 13));
    return float_of(sgn | ((e + 112) << 23) | (m << 13));
}

/* round half to even for |v| < 2^22 via the fp32 adder (gpuq/gpuq.hip:108-112) */
static inline int near_int(float v) {
    const float t = v + 12582912.f;
    OPS(2);
    return (int)(bits_of(t) & 0x007fffffu) - 0x00400000;
}

/* ggml's GGML_E8M0_TO_FP32_HALF: 2^(e - 128) (gpuq/gpuq.hip:2121) */
static inline float e8m0_half(uint8_t e) { return float_of(e < 2 ? 0x00200000u << e : (uint32_t)(e - 1) << 23); }

static inline void put16(uint8_t *p, uint16_t v) { p[0] = (uint8_t)v; p[1] = (uint8_t)(v >> 8); }
static inline uint16_t get16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

uint16_t gqo_fp32_to_fp16(float f) { return f32_to_f16(f); }
float gqo_fp16_to_fp32(uint16_t h) { return f16_to_f32(h); }
int gqo_nearest_int(float f) { return near_int(f); }
void gqo_fp32_to_fp16_range(uint32_t first, uint32_t count, uint16_t *out) {
    for (uint32_t i = 0; i < count; ++i) out[i] = f32_to_f16(float_of(first + i));
}
void gqo_fp16_to_fp32_all(float *out) { for (uint32_t h = 0; h < 65536; ++h) out[h] = f16_to_f32((uint16_t)h); }

/* ------------------------------------------------------------------ tables (gpuq/gpuq_tables.c:5-8) */
typedef struct {
    int type, grid_size, map_size, neigh_len;
    uint64_t *grid;
    int32_t *map;
    uint16_t *neigh;
} otab;
static otab g_tabs[32];
static int g_ntabs;

int gqo_load_tables(const char *path) {
    FILE *f = fopen(path, "rb");
    if (!f) return 2;
    for (int i = 0; i < g_ntabs; ++i) { free(g_tabs[i].grid); free(g_tabs[i].map); free(g_tabs[i].neigh); }
    g_ntabs = 0;
    int32_t hdr[4];
    while (fread(hdr, sizeof hdr, 1, f) == 1) {
        if (g_ntabs == 32 || hdr[1] < 0 || hdr[2] < 0 || hdr[3] < 0) { fclose(f); return 3; }
        otab t = {hdr[0], hdr[1], hdr[2], hdr[3], NULL, NULL, NULL};
        t.grid = malloc((size_t)hdr[1] * 8 + 8);
        t.map = malloc((size_t)hdr[2] * 4 + 4);
        t.neigh = malloc((size_t)hdr[3] * 2 + 2);
        if (fread(t.grid, 8, hdr[1], f) != (size_t)hdr[1] || fread(t.map, 4, hdr[2], f) != (size_t)hdr[2] ||
            fread(t.neigh, 2, hdr[3], f) != (size_t)hdr[3]) {
            free(t.grid); free(t.map); free(t.neigh); fclose(f); return 3;
        }
        g_tabs[g_ntabs++] = t;
    }
    fclose(f);
    return 0;
}

static const otab *tab_find(int type) {
    for (int i = 0; i < g_ntabs; ++i) if (g_tabs[i].type == type) return &g_tabs[i];
    return NULL;
}
/* search tables of a type: IQ1_M reads IQ1_S's (gpuq/gpuq.hip:2051-2056) */
static const otab *tab_search(int type) { return tab_find(type == GQO_IQ1_M ? GQO_IQ1_S : type); }
/* dequant grid: type 1000 + t, IQ1_M reads IQ1_S's (gpuq/gpuq.hip:2045-2049) */
static const otab *tab_dq(int type) { return tab_find(1000 + (type == GQO_IQ1_M ? GQO_IQ1_S : type)); }

int gqo_have_tables(int type) { return tab_search(type) != NULL && tab_dq(type) != NULL; }

/* map lookup with the bounds the reference leaves unchecked */
static inline int map_at(const otab *t, int u) {
    if (u < 0 || u >= t->map_size) { t_err = 1; return 0; }
    return t->map[u];
}
static inline const uint16_t *neigh_at(const otab *t, int m) {
    const int off = -m - 1;
    if (off < 0 || off >= t->neigh_len || off + t->neigh[off] >= t->neigh_len) { t_err = 1; static uint16_t z; return &z; }
    return t->neigh + off;
}
static inline const int8_t *grid_pt(const otab *t, int g) {
    if (g < 0 || g >= t->grid_size) { t_err = 1; return (const int8_t *)t->grid; }
    return (const int8_t *)(t->grid + g);
}

/* ------------------------------------------------------------------ shared searches */
/* make_qp_quants: non-negative levels 0..nmax for non-negative x (gpuq/gpuq.hip:114-176) */
static float qp_levels(int n, int nmax, const float *x, uint8_t *L, const float *qw) {
    float mx = 0;
    for (int i = 0; i < n; ++i) mx = GMAX(mx, x[i]);
    OPS(n);
    if (mx < EPS_GROUP) {
        for (int i = 0; i < n; ++i) L[i] = 0;
        return 0.f;
    }
    float iscale = nmax / mx;
    for (int i = 0; i < n; ++i) L[i] = (uint8_t)near_int(iscale * x[i]);
    float scale = 1 / iscale;
    float best_mse = 0;
    for (int i = 0; i < n; ++i) {
        const float diff = x[i] - scale * L[i];
        best_mse += qw[i] * diff * diff;
    }
    OPS(2 * C_DIV + n + 6 * n);
    for (int is = -4; is <= 4; ++is) {
        if (is == 0) continue;
        const float iscale_is = (0.1f * is + nmax) / mx;
        const float scale_is = 1 / iscale_is;
        float mse = 0;
        for (int i = 0; i < n; ++i) {
            int l = near_int(iscale_is * x[i]);
            l = GMIN(nmax, l);
            const float diff = x[i] - scale_is * l;
            mse += qw[i] * diff * diff;
        }
        OPS(3 + 2 * C_DIV + n * 8 + 1);
        if (mse < best_mse) { best_mse = mse; iscale = iscale_is; }
    }
    float sumlx = 0, suml2 = 0;
    for (int i = 0; i < n; ++i) {
        int l = near_int(iscale * x[i]);
        l = GMIN(nmax, l);
        L[i] = (uint8_t)l;
        sumlx += qw[i] * x[i] * l;
        suml2 += qw[i] * l * l;
    }
    OPS(n * 9);
    for (int pass = 0; pass < 5; ++pass) {
        int changed = 0;
        for (int i = 0; i < n; ++i) {
            const float w = qw[i];
            float slx = sumlx - w * x[i] * L[i];
            float sl2 = suml2 - w * L[i] * L[i];
            OPS(8);
            if (slx > 0 && sl2 > 0) {
                int nl = near_int(x[i] * sl2 / slx);
                nl = GMIN(nmax, nl);
                OPS(3 + C_DIV);
                if (nl != L[i]) {
                    slx += w * x[i] * nl;
                    sl2 += w * nl * nl;
                    OPS(11);
                    if (slx * slx * suml2 > sumlx * sumlx * sl2) {
                        L[i] = (uint8_t)nl; sumlx = slx; suml2 = sl2;
                        ++changed;
                    }
                }
            }
        }
        if (!changed) break;
    }
    OPS(1 + C_DIV);
    return suml2 > 0.0f ? sumlx / suml2 : 0.0f;
}

/* iq2_find_best_neighbour: weighted-nearest point of a neighbour list, first wins on ties (gpuq/gpuq.hip:178-197) */
static int nb_iq2(const otab *t, const uint16_t *nb, const float *xv, const float *wa, float scale, int8_t *L) {
    const int cnt = nb[0];
    float best = FLT_MAX;
    int gi = -1, nbest = 0;
    for (int j = 1; j <= cnt; ++j) {
        const int8_t *pg = grid_pt(t, nb[j]);
        float d2 = 0;
        for (int i = 0; i < 8; ++i) {
            const float q = pg[i];
            const float diff = scale * q - xv[i];
            d2 += wa[i] * diff * diff;
        }
        OPS(8 * 6 + 3);
        if (d2 < best) { best = d2; gi = nb[j]; nbest = 1; }
        else if (d2 == best) ++nbest;
    }
    STAT(GQO_STAT_NB8_SEARCHES);
    if (nbest > 1) STAT(GQO_STAT_NB8_TIES);
    if (gi < 0) { t_err = 1; gi = 0; }
    const int8_t *pg = grid_pt(t, gi);
    for (int i = 0; i < 8; ++i) L[i] = (int8_t)((pg[i] - 1) / 2);
    return gi;
}

/* iq1_find_best_neighbour2 (gpuq/gpuq.hip:199-232). The full-grid fallback of the reference (reached only when no
 * neighbour has a finite distance, i.e. for non-finite input) reads past the block; it is flagged as an error. */
static int nb_iq1(const otab *t, const uint16_t *nb, const float *xv, const float *w, float scale, const float *xg,
                  int8_t *L) {
    const int cnt = nb[0];
    float best = FLT_MAX;
    int gi = -1;
    for (int j = 1; j <= cnt; ++j) {
        const int8_t *pg = grid_pt(t, nb[j]);
        float d2 = 0;
        for (int i = 0; i < 8; ++i) {
            const float q = xg[(pg[i] - 1) / 2];
            const float diff = scale * q - xv[i];
            d2 += w[i] * diff * diff;
        }
        OPS(8 * 7 + 2);
        if (d2 < best) { best = d2; gi = nb[j]; }
    }
    if (gi >= 0 && best < 0) STAT(GQO_STAT_NB1_NEGATIVE);
    if (gi < 0) { t_err = 1; gi = 0; }
    const int8_t *pg = grid_pt(t, gi);
    for (int i = 0; i < 8; ++i) L[i] = (int8_t)((pg[i] - 1) / 2);
    return gi;
}

/* iq3_find_best_neighbour: 4-value groups (gpuq/gpuq.hip:971-992) */
static int nb_iq3(const otab *t, const uint16_t *nb, const float *xv, const float *wa, float scale, int8_t *L) {
    const int cnt = nb[0];
    if (cnt <= 0) t_err = 1;
    float best = FLT_MAX;
    int gi = -1;
    for (int j = 1; j <= cnt; ++j) {
        const int8_t *pg = grid_pt(t, nb[j]);
        float d2 = 0;
        for (int i = 0; i < 4; ++i) {
            const float q = pg[i];
            const float diff = scale * q - xv[i];
            d2 += wa[i] * diff * diff;
        }
        OPS(4 * 6 + 2);
        if (d2 < best) { best = d2; gi = nb[j]; }
    }
    if (gi < 0) { t_err = 1; gi = 0; }
    const int8_t *pg = grid_pt(t, gi);
    for (int i = 0; i < 4; ++i) L[i] = (int8_t)((pg[i] - 1) / 2);
    return gi;
}

/* stable ascending sort of (key, index) pairs: glibc's merge-sort qsort order (gpuq/gpuq.hip:234-243) */
static void sort_stable(float *key, int *idx, int n) {
    for (int i = 1; i < n; ++i) {
        const float k = key[i];
        const int v = idx[i];
        int j = i - 1;
        while (j >= 0 && key[j] > k) { key[j + 1] = key[j]; idx[j + 1] = idx[j]; --j; OPS(2); }
        key[j + 1] = k; idx[j + 1] = v;
        OPS(2);
    }
}

/* signs of 8 values with the even-parity rule: an odd count flips the least important weight
 * (gpuq/gpuq.hip:272-289) */
static uint8_t signs_even(const float *xb, const float *weight, float *xval) {
    int nflip = 0;
    uint8_t s = 0;
    for (int i = 0; i < 8; ++i) {
        if (xb[i] >= 0) xval[i] = xb[i];
        else { xval[i] = -xb[i]; ++nflip; s |= (uint8_t)(1 << i); }
    }
    OPS(8 * 3);
    if (nflip % 2) {
        int imin = 0;
        float mn = weight[0] * xb[0] * xb[0];
        for (int i = 1; i < 8; ++i) {
            const float ax = weight[i] * xb[i] * xb[i];
            if (ax < mn) { mn = ax; imin = i; }
        }
        OPS(8 * 4);
        xval[imin] = -xval[imin];
        s ^= (uint8_t)(1 << imin);
    }
    return s & 127;
}

static float sum_sq(const float *x, int n) {
    float s = 0;
    for (int i = 0; i < n; ++i) s += x[i] * x[i];
    OPS(2 * n);
    return s;
}

static void iq_weights(const float *qw, const float *xb, float sigma2, float *weight, int n) {
    for (int i = 0; i < n; ++i) weight[i] = qw[i] * sqrtf(sigma2 + xb[i] * xb[i]);
    OPS(n * (2 + C_SQRT));
}

/* ------------------------------------------------------------------ IQ2_XXS (gpuq/gpuq.hip:245-387) */
static void o_iq2_xxs(const float *xbl, const float *qwbl, uint8_t *y, const otab *t) {
    const int kMaxQ = 3;
    float scales[8], weight[32], xval[32], waux[32];
    int8_t L[32], Laux[32];
    uint8_t bsg[4];
    uint32_t q2[16];
    memset(q2, 0, sizeof q2);
    put16(y, f32_to_f16(0.f));
    float max_scale = 0;
    const float sigma2 = sum_sq(xbl, QK) / QK;
    for (int ib = 0; ib < 8; ++ib) {
        const float *xb = xbl + 32 * ib;
        iq_weights(qwbl + 32 * ib, xb, sigma2, weight, 32);
        for (int i = 0; i < 32; ++i) waux[i] = sqrtf(weight[i]);
        OPS(32 * C_SQRT);
        for (int k = 0; k < 4; ++k) bsg[k] = signs_even(xb + 8 * k, weight + 8 * k, xval + 8 * k);
        float mx = xval[0];
        for (int i = 1; i < 32; ++i) mx = GMAX(mx, xval[i]);
        OPS(32 + 32);
        if (mx < EPS_GROUP) {
            scales[ib] = 0;
            memset(L, 0, sizeof L);
            continue;
        }
        float scale = qp_levels(32, kMaxQ + 1, xval, (uint8_t *)L, weight);
        const float eff_max = scale * kMaxQ;
        if (eff_max <= 0) {
            scales[ib] = 0;
            memset(L, 0, sizeof L);
            continue;
        }
        float best = 0;
        for (int is = -6; is <= 6; ++is) {
            const float id = (2 * kMaxQ - 1 + is * 0.1f) / eff_max;
            const float this_scale = 1 / id;
            OPS(3 + 2 * C_DIV);
            for (int k = 0; k < 4; ++k) {
                int u = 0;
                for (int i = 0; i < 8; ++i) {
                    const int l = near_int(0.5f * (id * xval[8 * k + i] - 1));
                    Laux[8 * k + i] = (int8_t)GMAX(0, GMIN(kMaxQ - 1, l));
                    u |= Laux[8 * k + i] << 2 * i;
                }
                OPS(8 * 5 + 1);
                const int m = map_at(t, u);
                if (m < 0) nb_iq2(t, neigh_at(t, m), xval + 8 * k, waux + 8 * k, this_scale, Laux + 8 * k);
            }
            float sumqx = 0, sumq2 = 0;
            for (int i = 0; i < 32; ++i) {
                const float w = weight[i];
                const float q = 2 * Laux[i] + 1;
                sumqx += w * xval[i] * q;
                sumq2 += w * q * q;
            }
            OPS(32 * 6 + 5);
            if (sumq2 > 0 && sumqx * sumqx > best * sumq2) {
                scale = sumqx / sumq2;
                best = scale * sumqx;
                memcpy(L, Laux, sizeof L);
                OPS(2 + C_DIV);
            }
        }
        if (!(scale > 0)) STAT(GQO_STAT_IQ2XXS_NEGCHAIN);
        if (scale > 0) {
            const float id = 1 / scale;
            for (int k = 0; k < 4; ++k) {
                int u = 0;
                for (int i = 0; i < 8; ++i) {
                    int l = near_int(0.5f * (id * xval[8 * k + i] - 1));
                    l = GMAX(0, GMIN(kMaxQ - 1, l));
                    u |= l << 2 * i;
                }
                OPS(8 * 5);
                int gi = map_at(t, u);
                if (gi < 0) gi = nb_iq2(t, neigh_at(t, gi), xval + 8 * k, waux + 8 * k, scale, L + 8 * k);
                const int8_t *pg = grid_pt(t, gi);
                for (int i = 0; i < 8; ++i) L[8 * k + i] = (int8_t)((pg[i] - 1) / 2);
            }
            float sumqx = 0, sumq2 = 0;
            for (int i = 0; i < 32; ++i) {
                const float w = weight[i];
                const float q = 2 * L[i] + 1;
                sumqx += w * xval[i] * q;
                sumq2 += w * q * q;
            }
            OPS(32 * 6 + C_DIV * 2);
            if (sumq2 > 0) scale = sumqx / sumq2;
        }
        if (scale < 0) {
            scale = -scale;
            for (int k = 0; k < 4; ++k) bsg[k] = (uint8_t)(~bsg[k]) & 127;
        }
        for (int k = 0; k < 4; ++k) {
            int u = 0;
            for (int i = 0; i < 8; ++i) u |= L[8 * k + i] << 2 * i;
            const int gi = map_at(t, u);
            if (gi < 0) t_err = 1;
            q2[2 * ib + 0] |= (uint32_t)gi << 8 * k;
            q2[2 * ib + 1] |= (uint32_t)bsg[k] << 7 * k;
        }
        scales[ib] = scale;
        max_scale = GMAX(max_scale, scale);
    }
    if (!max_scale) {
        memset(y + 2, 0, 64);
        return;
    }
    const float d = max_scale / 31;
    put16(y, f32_to_f16(d));
    const float id = 1 / d;
    for (int ib = 0; ib < 8; ++ib) {
        int l = near_int(0.5f * (id * scales[ib] - 1));
        l = GMAX(0, GMIN(15, l));
        q2[2 * ib + 1] |= (uint32_t)l << 28;
    }
    OPS(2 * C_DIV + 8 * 6);
    for (int i = 0; i < 16; ++i) {
        put16(y + 2 + 4 * i, (uint16_t)(q2[i] & 0xffff));
        put16(y + 4 + 4 * i, (uint16_t)(q2[i] >> 16));
    }
}

/* ------------------------------------------------------------------ IQ2_XS / IQ2_S share the 16-block search
 * (gpuq/gpuq.hip:690-822 and 824-969): 19 trial scales, an on-grid re-search, plain (IQ2_S) or parity (IQ2_XS)
 * signs. Returns the sub-block's scale, writes its 16 levels, 2 grid indices and 2 sign bytes. */
static float iq2_16_search(const float *xb, const float *qw, float sigma2, int parity, float eps, const otab *t,
                           int *gidx, uint8_t *bsg) {
    const int kMaxQ = 3;
    float weight[16], xval[16], waux[16];
    int8_t L[16], Laux[16];
    int on_grid[2], on_grid_aux[2];
    iq_weights(qw, xb, sigma2, weight, 16);
    for (int i = 0; i < 16; ++i) waux[i] = sqrtf(weight[i]);
    OPS(16 * C_SQRT);
    for (int k = 0; k < 2; ++k) {
        if (parity) {
            bsg[k] = signs_even(xb + 8 * k, weight + 8 * k, xval + 8 * k);
        } else {
            uint8_t s = 0;
            for (int i = 0; i < 8; ++i) {
                if (xb[8 * k + i] >= 0) xval[8 * k + i] = xb[8 * k + i];
                else { xval[8 * k + i] = -xb[8 * k + i]; s |= (uint8_t)(1 << i); }
            }
            OPS(8 * 3);
            bsg[k] = s;
        }
    }
    float mx = xval[0];
    for (int i = 1; i < 16; ++i) mx = GMAX(mx, xval[i]);
    OPS(16 + 16);
    memset(L, 0, sizeof L);
    gidx[0] = gidx[1] = -1;
    if (mx < eps) return 0.f;   /* the caller writes nothing for this sub-block */
    float best = 0;
    float scale = mx / (2 * kMaxQ - 1);
    on_grid[0] = on_grid[1] = 1;
    OPS(C_DIV);
    for (int is = -9; is <= 9; ++is) {
        const float id = (2 * kMaxQ - 1 + is * 0.1f) / mx;
        const float this_scale = 1 / id;
        OPS(3 + 2 * C_DIV);
        for (int k = 0; k < 2; ++k) {
            int u = 0;
            for (int i = 0; i < 8; ++i) {
                const int l = near_int(0.5f * (id * xval[8 * k + i] - 1));
                Laux[8 * k + i] = (int8_t)GMAX(0, GMIN(kMaxQ - 1, l));
                u |= Laux[8 * k + i] << 2 * i;
            }
            OPS(8 * 5 + 1);
            const int m = map_at(t, u);
            on_grid_aux[k] = 1;
            if (m < 0) {
                on_grid_aux[k] = 0;
                nb_iq2(t, neigh_at(t, m), xval + 8 * k, waux + 8 * k, this_scale, Laux + 8 * k);
            }
        }
        float sumqx = 0, sumq2 = 0;
        for (int i = 0; i < 16; ++i) {
            const float w = weight[i];
            const float q = 2 * Laux[i] + 1;
            sumqx += w * xval[i] * q;
            sumq2 += w * q * q;
        }
        OPS(16 * 6 + 5);
        if (sumq2 > 0 && sumqx * sumqx > best * sumq2) {
            scale = sumqx / sumq2;
            best = scale * sumqx;
            memcpy(L, Laux, sizeof L);
            on_grid[0] = on_grid_aux[0];
            on_grid[1] = on_grid_aux[1];
            OPS(2 + C_DIV);
        }
    }
    const int n_off = (!on_grid[0]) + (!on_grid[1]);
    if (!(scale > 0)) STAT(GQO_STAT_IQ2X16_NEGCHAIN);
    if (n_off > 0 && scale > 0) {
        const float id = 1 / scale;
        OPS(C_DIV);
        for (int k = 0; k < 2; ++k) {
            if (on_grid[k]) continue;
            int u = 0;
            for (int i = 0; i < 8; ++i) {
                int l = near_int(0.5f * (id * xval[8 * k + i] - 1));
                l = GMAX(0, GMIN(kMaxQ - 1, l));
                u |= l << 2 * i;
                L[8 * k + i] = (int8_t)l;
            }
            OPS(8 * 5);
            const int m = map_at(t, u);
            if (m < 0) nb_iq2(t, neigh_at(t, m), xval + 8 * k, waux + 8 * k, scale, L + 8 * k);
        }
        float sumqx = 0, sumq2 = 0;
        for (int i = 0; i < 16; ++i) {
            const float w = weight[i];
            const float q = 2 * L[i] + 1;
            sumqx += w * xval[i] * q;
            sumq2 += w * q * q;
        }
        OPS(16 * 6 + C_DIV);
        if (sumq2 > 0) scale = sumqx / sumq2;
    }
    if (scale < 0) {
        scale = -scale;
        for (int k = 0; k < 2; ++k) bsg[k] = parity ? ((uint8_t)(~bsg[k]) & 127) : (uint8_t)~bsg[k];
    }
    for (int k = 0; k < 2; ++k) {
        int u = 0;
        for (int i = 0; i < 8; ++i) u |= L[8 * k + i] << 2 * i;
        gidx[k] = map_at(t, u);
        if (gidx[k] < 0) { t_err = 1; gidx[k] = 0; }
    }
    return scale;
}

static void o_iq2_s(const float *xbl, const float *qwbl, uint8_t *y, const otab *t) {
    /* block_iq2_s: d(2) qs[64] qh[8] scales[8] (gpuq/gpuq.hip:59) */
    memset(y, 0, 82);
    put16(y, f32_to_f16(0.f));
    uint8_t *qs = y + 2, *qh = y + 66, *sc = y + 74;
    float scales[16], max_scale = 0;
    const float sigma2 = 2 * sum_sq(xbl, QK) / QK;
    for (int ib = 0; ib < 16; ++ib) {
        int gidx[2];
        uint8_t bsg[2];
        const float s = iq2_16_search(xbl + 16 * ib, qwbl + 16 * ib, sigma2, 0, EPS_IQ2S, t, gidx, bsg);
        if (gidx[0] < 0) { scales[ib] = 0; continue; }
        for (int k = 0; k < 2; ++k) {
            const int i8 = 2 * ib + k;
            qs[i8] = (uint8_t)(gidx[k] & 255);
            qh[i8 / 4] |= (uint8_t)((gidx[k] >> 8) << 2 * (i8 % 4));
            qs[32 + i8] = bsg[k];
        }
        scales[ib] = s;
        max_scale = GMAX(max_scale, s);
    }
    if (!max_scale) return;
    const float d = max_scale / 31;
    put16(y, f32_to_f16(d * 0.9875f));
    const float id = 1 / d;
    for (int ib = 0; ib < 16; ++ib) {
        int l = near_int(0.5f * (id * scales[ib] - 1));
        l = GMAX(0, GMIN(15, l));
        if (ib % 2 == 0) sc[ib / 2] = (uint8_t)l;
        else sc[ib / 2] |= (uint8_t)(l << 4);
    }
    OPS(2 * C_DIV + 16 * 6);
}

static void o_iq2_xs(const float *xbl, const float *qwbl, uint8_t *y, const otab *t) {
    /* block_iq2_xs: d(2) qs[32] u16 scales[8] (gpuq/gpuq.hip:62) */
    uint16_t q2[32];
    memset(q2, 0, sizeof q2);
    put16(y, f32_to_f16(0.f));
    uint8_t *sc = y + 66;
    memset(sc, 0, 8);
    float scales[16], max_scale = 0;
    const float sigma2 = sum_sq(xbl, QK) / QK;
    for (int ib = 0; ib < 16; ++ib) {
        int gidx[2];
        uint8_t bsg[2];
        const float s = iq2_16_search(xbl + 16 * ib, qwbl + 16 * ib, sigma2, 1, EPS_GROUP, t, gidx, bsg);
        if (gidx[0] < 0) { scales[ib] = 0; continue; }
        for (int k = 0; k < 2; ++k) q2[2 * ib + k] = (uint16_t)(gidx[k] | (bsg[k] << 9));
        scales[ib] = s;
        max_scale = GMAX(max_scale, s);
    }
    if (!max_scale) {
        memset(y + 2, 0, 64);
        return;
    }
    const float d = max_scale / 31;
    put16(y, f32_to_f16(d));
    const float id = 1 / d;
    for (int ib = 0; ib < 16; ++ib) {
        int l = near_int(0.5f * (id * scales[ib] - 1));
        l = GMAX(0, GMIN(15, l));
        if (ib % 2 == 0) sc[ib / 2] = (uint8_t)l;
        else sc[ib / 2] |= (uint8_t)(l << 4);
    }
    OPS(2 * C_DIV + 16 * 6);
    for (int i = 0; i < 32; ++i) put16(y + 2 + 2 * i, q2[i]);
}

/* ------------------------------------------------------------------ IQ1_S (gpuq/gpuq.hip:389-514) */
static void o_iq1_s(const float *xbl, const float *qwbl, uint8_t *y, const otab *t) {
    /* block_iq1_s: d(2) qs[32] qh[8] u16 (gpuq/gpuq.hip:60) */
    const int bs = 32;
    float scales[8], weight[32], sumx[33], sumw[33], key[32];
    int8_t L[32], shifts[8];
    int idx[32];
    uint16_t index[4], qh[8];
    const float x_p[3] = {-1 + DELTA_IQ1, DELTA_IQ1, 1 + DELTA_IQ1};
    const float x_m[3] = {-1 - DELTA_IQ1, -DELTA_IQ1, 1 - DELTA_IQ1};
    uint8_t *qs = y + 2;
    put16(y, f32_to_f16(0.f));
    memset(qs, 0, 32);
    memset(qh, 0, sizeof qh);
    float max_scale = 0;
    const float sigma2 = 2 * sum_sq(xbl, QK) / QK;
    for (int ib = 0; ib < 8; ++ib) {
        const float *xb = xbl + bs * ib;
        iq_weights(qwbl + bs * ib, xb, sigma2, weight, bs);
        float mx = fabsf(xb[0]);
        for (int i = 1; i < bs; ++i) mx = GMAX(mx, fabsf(xb[i]));
        OPS(bs);
        if (mx < EPS_IQ1S) {
            scales[ib] = 0;
            shifts[ib] = 1;
            continue;
        }
        for (int j = 0; j < bs; ++j) { key[j] = xb[j]; idx[j] = j; }
        sort_stable(key, idx, bs);
        sumx[0] = sumw[0] = 0;
        for (int j = 0; j < bs; ++j) {
            const int i = idx[j];
            sumx[j + 1] = sumx[j] + weight[i] * xb[i];
            sumw[j + 1] = sumw[j] + weight[i];
        }
        OPS(3 * bs);
        float best_score = -FLT_MAX, scale = mx;
        int besti1 = -1, besti2 = -1, best_shift = 0;
        for (int i1 = 0; i1 <= bs; ++i1) {
            for (int i2 = i1; i2 <= bs; ++i2) {
                float sumqx = (sumx[i1] - sumx[0]) * x_p[0] + (sumx[i2] - sumx[i1]) * x_p[1] + (sumx[bs] - sumx[i2]) * x_p[2];
                float sumq2 = (sumw[i1] - sumw[0]) * x_p[0] * x_p[0] + (sumw[i2] - sumw[i1]) * x_p[1] * x_p[1] +
                              (sumw[bs] - sumw[i2]) * x_p[2] * x_p[2];
                OPS(17);
                if (sumq2 > 0 && sumqx * sumqx > best_score * sumq2) {
                    scale = sumqx / sumq2;
                    best_score = scale * sumqx;
                    besti1 = i1; besti2 = i2; best_shift = 1;
                    OPS(5 + C_DIV);
                }
                sumqx = (sumx[i1] - sumx[0]) * x_m[0] + (sumx[i2] - sumx[i1]) * x_m[1] + (sumx[bs] - sumx[i2]) * x_m[2];
                sumq2 = (sumw[i1] - sumw[0]) * x_m[0] * x_m[0] + (sumw[i2] - sumw[i1]) * x_m[1] * x_m[1] +
                        (sumw[bs] - sumw[i2]) * x_m[2] * x_m[2];
                OPS(17);
                if (sumq2 > 0 && sumqx * sumqx > best_score * sumq2) {
                    scale = sumqx / sumq2;
                    best_score = scale * sumqx;
                    besti1 = i1; besti2 = i2; best_shift = -1;
                    OPS(5 + C_DIV);
                }
            }
        }
        if (besti1 < 0 || besti2 < 0 || best_shift == 0) {
            scales[ib] = 0;
            shifts[ib] = 1;
            continue;
        }
        for (int j = 0; j < besti1; ++j) L[idx[j]] = 0;
        for (int j = besti1; j < besti2; ++j) L[idx[j]] = 1;
        for (int j = besti2; j < bs; ++j) L[idx[j]] = 2;
        if (scale < 0) {
            for (int j = 0; j < bs; ++j) L[j] = (int8_t)(2 - L[j]);
            scale = -scale;
            best_shift = -best_shift;
        }
        int all_on_grid = 1;
        const float *xx = best_shift == 1 ? x_p : x_m;
        for (int k = 0; k < bs / 8; ++k) {
            int u = 0;
            for (int j = 0; j < 8; ++j) u |= L[8 * k + j] << 2 * j;
            int gi = map_at(t, u);
            if (gi < 0) {
                all_on_grid = 0;
                gi = nb_iq1(t, neigh_at(t, gi), xb + 8 * k, weight + 8 * k, scale, xx, L + 8 * k);
            }
            index[k] = (uint16_t)gi;
        }
        if (!all_on_grid) {
            float sumqx = 0, sumq2 = 0;
            for (int k = 0; k < bs / 8; ++k) {
                const int8_t *pg = grid_pt(t, index[k]);
                for (int j = 0; j < 8; ++j) {
                    const float w = weight[8 * k + j];
                    const float q = xx[(pg[j] - 1) / 2];
                    sumqx += w * q * xb[8 * k + j];
                    sumq2 += w * q * q;
                }
            }
            OPS(bs * 7 + 2 + C_DIV);
            if (sumqx > 0 && sumq2 > 0) scale = sumqx / sumq2;
        }
        uint16_t h = 0;
        for (int k = 0; k < bs / 8; ++k) {
            qs[(bs / 8) * ib + k] = (uint8_t)(index[k] & 255);
            h |= (uint16_t)((index[k] >> 8) << 3 * k);
        }
        qh[ib] = h;
        scales[ib] = scale;
        shifts[ib] = (int8_t)best_shift;
        max_scale = GMAX(max_scale, scale);
    }
    if (max_scale) {
        const float d = max_scale / 15;
        put16(y, f32_to_f16(d * 1.125f));
        const float id = 1 / d;
        for (int ib = 0; ib < 8; ++ib) {
            int l = near_int(0.5f * (id * scales[ib] - 1));
            l = GMAX(0, GMIN(7, l));
            if (shifts[ib] == -1) l |= 8;
            qh[ib] |= (uint16_t)(l << 12);
        }
        OPS(2 * C_DIV + 8 * 6);
    }
    for (int ib = 0; ib < 8; ++ib) put16(y + 34 + 2 * ib, qh[ib]);
}

/* ------------------------------------------------------------------ IQ1_M (gpuq/gpuq.hip:516-688) */
static void o_iq1_m(const float *xbl, const float *qwbl, uint8_t *y, const otab *t) {
    /* block_iq1_m: qs[32] qh[16] scales[8] (gpuq/gpuq.hip:61) */
    const int bs = 16;
    float scales[16], weight[16], key[16];
    int8_t L[16], shifts[16];
    int idx[16];
    uint16_t index[2];
    const float x_p[3] = {-1 + DELTA_IQ1, DELTA_IQ1, 1 + DELTA_IQ1};
    const float x_m[3] = {-1 - DELTA_IQ1, -DELTA_IQ1, 1 - DELTA_IQ1};
    const uint8_t masks[4] = {0x00, 0x80, 0x08, 0x88};
    uint8_t *qs = y, *qh = y + 32, *ysc = y + 48;
    memset(y, 0, 56);
    float max_scale = 0;
    const float sigma2 = 2 * sum_sq(xbl, QK) / QK;
    for (int ib = 0; ib < 16; ++ib) {
        const float *xb = xbl + bs * ib;
        iq_weights(qwbl + bs * ib, xb, sigma2, weight, bs);
        float mx = fabsf(xb[0]);
        for (int i = 1; i < bs; ++i) mx = GMAX(mx, fabsf(xb[i]));
        OPS(bs);
        if (mx < EPS_IQ1M) {
            scales[ib] = 0;
            shifts[ib] = 0;
            continue;
        }
        for (int j = 0; j < bs; ++j) { key[j] = xb[j]; idx[j] = j; }
        sort_stable(key, idx, bs);
        float best_score = -FLT_MAX, scale = mx;
        int besti1 = -1, besti2 = -1, best_k = -1;
        float px[2][17], pw[2][17];
        px[0][0] = px[1][0] = 0;
        pw[0][0] = pw[1][0] = 0;
        for (int j = 0; j < bs; ++j) {
            const int i = idx[j];
            const int h = i < bs / 2 ? 0 : 1;
            px[h][j + 1] = px[h][j] + weight[i] * xb[i];
            px[1 - h][j + 1] = px[1 - h][j];
            pw[h][j + 1] = pw[h][j] + weight[i];
            pw[1 - h][j + 1] = pw[1 - h][j];
        }
        OPS(4 * bs);
        const float txs[2] = {px[0][bs], px[1][bs]};
        const float tws[2] = {pw[0][bs], pw[1][bs]};
        const float p2 = x_p[2], m2 = x_m[2];
        const float cp1 = x_p[0] * x_p[0] - x_p[1] * x_p[1];
        const float cp2 = x_p[1] * x_p[1] - x_p[2] * x_p[2];
        const float cm1 = x_m[0] * x_m[0] - x_m[1] * x_m[1];
        const float cm2 = x_m[1] * x_m[1] - x_m[2] * x_m[2];
        for (int i1 = 0; i1 <= bs; ++i1) {
            for (int i2 = i1; i2 <= bs; ++i2) {
                float qx_p[2], qx_m[2], q2_p[2], q2_m[2], sumqx[4], sumq2[4];
                for (int h = 0; h < 2; ++h) {
                    const float sx = px[h][i1] + px[h][i2];
                    qx_p[h] = txs[h] * p2 - sx;
                    qx_m[h] = txs[h] * m2 - sx;
                    q2_p[h] = tws[h] * p2 * p2 + pw[h][i1] * cp1 + pw[h][i2] * cp2;
                    q2_m[h] = tws[h] * m2 * m2 + pw[h][i1] * cm1 + pw[h][i2] * cm2;
                }
                sumqx[0] = qx_p[0] + qx_p[1];
                sumqx[1] = qx_p[0] + qx_m[1];
                sumqx[2] = qx_m[0] + qx_p[1];
                sumqx[3] = qx_m[0] + qx_m[1];
                sumq2[0] = q2_p[0] + q2_p[1];
                sumq2[1] = q2_p[0] + q2_m[1];
                sumq2[2] = q2_m[0] + q2_p[1];
                sumq2[3] = q2_m[0] + q2_m[1];
                OPS(26);
                for (int k = 0; k < 4; ++k) {
                    OPS(5);
                    if (sumq2[k] > 0 && sumqx[k] * sumqx[k] > best_score * sumq2[k]) {
                        scale = sumqx[k] / sumq2[k];
                        best_score = scale * sumqx[k];
                        besti1 = i1; besti2 = i2; best_k = k;
                        OPS(5 + C_DIV);
                    }
                }
            }
        }
        if (besti1 < 0 || besti2 < 0 || best_k < 0) {
            scales[ib] = 0;
            shifts[ib] = 0;
            continue;
        }
        for (int j = 0; j < besti1; ++j) L[idx[j]] = 0;
        for (int j = besti1; j < besti2; ++j) L[idx[j]] = 1;
        for (int j = besti2; j < bs; ++j) L[idx[j]] = 2;
        if (scale < 0) {
            for (int j = 0; j < bs; ++j) L[j] = (int8_t)(2 - L[j]);
            scale = -scale;
            best_k = best_k == 0 ? 3 : best_k == 1 ? 2 : best_k == 2 ? 1 : 0;
        }
        int all_on_grid = 1;
        for (int k = 0; k < 2; ++k) {
            const float *xx = k == 0 ? (best_k < 2 ? x_p : x_m) : (best_k % 2 == 0 ? x_p : x_m);
            int u = 0;
            for (int j = 0; j < 8; ++j) u |= L[8 * k + j] << 2 * j;
            int gi = map_at(t, u);
            if (gi < 0) {
                all_on_grid = 0;
                gi = nb_iq1(t, neigh_at(t, gi), xb + 8 * k, weight + 8 * k, scale, xx, L + 8 * k);
            }
            index[k] = (uint16_t)gi;
        }
        if (!all_on_grid) {
            float sqx = 0, sq2 = 0;
            for (int k = 0; k < 2; ++k) {
                const float *xx = k == 0 ? (best_k < 2 ? x_p : x_m) : (best_k % 2 == 0 ? x_p : x_m);
                const int8_t *pg = grid_pt(t, index[k]);
                for (int j = 0; j < 8; ++j) {
                    const float w = weight[8 * k + j];
                    const float q = xx[(pg[j] - 1) / 2];
                    sqx += w * q * xb[8 * k + j];
                    sq2 += w * q * q;
                }
            }
            OPS(bs * 7 + 2 + C_DIV);
            if (sqx > 0 && sq2 > 0) scale = sqx / sq2;
        }
        qs[2 * ib + 0] = (uint8_t)(index[0] & 255);
        qs[2 * ib + 1] = (uint8_t)(index[1] & 255);
        qh[ib] = (uint8_t)((index[0] >> 8) | ((index[1] >> 8) << 4));
        scales[ib] = scale;
        shifts[ib] = (int8_t)best_k;
        max_scale = GMAX(max_scale, scale);
    }
    if (!max_scale) return;
    uint16_t sc[4] = {0, 0, 0, 0};
    float d = max_scale / 15;
    const float id = 1 / d;
    float sqx = 0, sq2 = 0;
    OPS(2 * C_DIV);
    for (int ib = 0; ib < 16; ++ib) {
        int l = near_int(0.5f * (id * scales[ib] - 1));
        l = GMAX(0, GMIN(7, l));
        sc[ib / 4] |= (uint16_t)(l << 3 * (ib % 4));
        qh[ib] |= masks[shifts[ib]];
        const float *xb = xbl + bs * ib;
        for (int i = 0; i < bs; ++i) weight[i] = qwbl[bs * ib + i] * sqrtf(sigma2 + xb[i] * xb[i]);   /* (same values as the first pass: not counted again) */
        for (int k = 0; k < 2; ++k) {
            const float *xx = k == 0 ? (shifts[ib] < 2 ? x_p : x_m) : (shifts[ib] % 2 == 0 ? x_p : x_m);
            const int8_t *pg = grid_pt(t, qs[2 * ib + k] + ((qh[ib] << (8 - 4 * k)) & 0x700));
            for (int j = 0; j < 8; ++j) {
                const float w = weight[8 * k + j];
                const float q = xx[(pg[j] - 1) / 2] * (2 * l + 1);
                sqx += w * q * xb[8 * k + j];
                sq2 += w * q * q;
            }
        }
        OPS(6 + 16 * 8);
    }
    if (sq2 > 0) d = sqx / sq2;
    const uint16_t s = f32_to_f16(d * 1.1125f);
    sc[0] |= (uint16_t)((s & 0x000f) << 12);
    sc[1] |= (uint16_t)((s & 0x00f0) << 8);
    sc[2] |= (uint16_t)((s & 0x0f00) << 4);
    sc[3] |= (uint16_t)((s & 0xf000) << 0);
    for (int i = 0; i < 4; ++i) { ysc[2 * i] = (uint8_t)(sc[i] & 0xff); ysc[2 * i + 1] = (uint8_t)(sc[i] >> 8); }
}

/* ------------------------------------------------------------------ IQ3_XXS (gpuq/gpuq.hip:994-1143) */
static void o_iq3_xxs(const float *xbl, const float *qwbl, uint8_t *y, const otab *t) {
    /* block_iq3_xxs: d(2) qs[96] = 64 grid bytes then 8 u32 scales-and-signs (gpuq/gpuq.hip:63) */
    const int kMaxQ = 8;
    float scales[8], weight[32], xval[32], waux[32];
    int8_t L[32], Laux[32];
    int on_grid[8], on_grid_aux[8];
    uint8_t bsg[4], q3[64];
    uint32_t sas[8];
    put16(y, f32_to_f16(0.f));
    memset(q3, 0, sizeof q3);
    memset(sas, 0, sizeof sas);
    float max_scale = 0;
    const float sigma2 = 2 * sum_sq(xbl, QK) / QK;
    for (int ib = 0; ib < 8; ++ib) {
        const float *xb = xbl + 32 * ib;
        iq_weights(qwbl + 32 * ib, xb, sigma2, weight, 32);
        for (int i = 0; i < 32; ++i) waux[i] = sqrtf(weight[i]);
        OPS(32 * C_SQRT);
        for (int k = 0; k < 4; ++k) bsg[k] = signs_even(xb + 8 * k, weight + 8 * k, xval + 8 * k);
        float mx = xval[0];
        for (int i = 1; i < 32; ++i) mx = GMAX(mx, xval[i]);
        OPS(32 + 32);
        memset(L, 0, sizeof L);
        if (mx < EPS_IQ3XXS) {
            scales[ib] = 0;
            continue;
        }
        float best = 0;
        float scale = mx / (2 * kMaxQ - 1);
        for (int k = 0; k < 8; ++k) on_grid[k] = 1;
        OPS(C_DIV);
        for (int is = -15; is <= 15; ++is) {
            const float id = (2 * kMaxQ - 1 + is * 0.2f) / mx;
            const float this_scale = 1 / id;
            OPS(3 + 2 * C_DIV);
            for (int k = 0; k < 8; ++k) {
                int u = 0;
                for (int i = 0; i < 4; ++i) {
                    const int l = near_int(0.5f * (id * xval[4 * k + i] - 1));
                    Laux[4 * k + i] = (int8_t)GMAX(0, GMIN(kMaxQ - 1, l));
                    u |= Laux[4 * k + i] << 3 * i;
                }
                OPS(4 * 5 + 1);
                const int m = map_at(t, u);
                on_grid_aux[k] = 1;
                if (m < 0) {
                    on_grid_aux[k] = 0;
                    nb_iq3(t, neigh_at(t, m), xval + 4 * k, waux + 4 * k, this_scale, Laux + 4 * k);
                }
            }
            float sumqx = 0, sumq2 = 0;
            for (int i = 0; i < 32; ++i) {
                const float w = weight[i];
                const float q = 2 * Laux[i] + 1;
                sumqx += w * xval[i] * q;
                sumq2 += w * q * q;
            }
            OPS(32 * 6 + 5);
            if (sumq2 > 0 && sumqx * sumqx > best * sumq2) {
                scale = sumqx / sumq2;
                best = scale * sumqx;
                memcpy(L, Laux, sizeof L);
                for (int k = 0; k < 8; ++k) on_grid[k] = on_grid_aux[k];
                OPS(2 + C_DIV);
            }
        }
        int n_off = 0;
        for (int k = 0; k < 8; ++k) if (!on_grid[k]) ++n_off;
        if (n_off > 0 && scale > 0) {
            const float id = 1 / scale;
            OPS(C_DIV);
            for (int k = 0; k < 8; ++k) {
                if (on_grid[k]) continue;
                int u = 0;
                for (int i = 0; i < 4; ++i) {
                    int l = near_int(0.5f * (id * xval[4 * k + i] - 1));
                    l = GMAX(0, GMIN(kMaxQ - 1, l));
                    u |= l << 3 * i;
                }
                OPS(4 * 5);
                int gi = map_at(t, u);
                if (gi < 0) gi = nb_iq3(t, neigh_at(t, gi), xval + 4 * k, waux + 4 * k, scale, L + 4 * k);
                const int8_t *pg = grid_pt(t, gi);
                for (int i = 0; i < 4; ++i) L[4 * k + i] = (int8_t)((pg[i] - 1) / 2);
            }
            float sumqx = 0, sumq2 = 0;
            for (int i = 0; i < 32; ++i) {
                const float w = weight[i];
                const float q = 2 * L[i] + 1;
                sumqx += w * xval[i] * q;
                sumq2 += w * q * q;
            }
            OPS(32 * 6 + C_DIV);
            if (sumq2 > 0) scale = sumqx / sumq2;
        }
        if (scale < 0) {
            scale = -scale;
            for (int k = 0; k < 4; ++k) bsg[k] = (uint8_t)(~bsg[k]) & 127;
        }
        for (int k = 0; k < 8; ++k) {
            int u = 0;
            for (int i = 0; i < 4; ++i) u |= L[4 * k + i] << 3 * i;
            const int gi = map_at(t, u);
            if (gi < 0) t_err = 1;
            q3[8 * ib + k] = (uint8_t)gi;
        }
        sas[ib] = bsg[0] | (bsg[1] << 7) | (bsg[2] << 14) | ((uint32_t)bsg[3] << 21);
        scales[ib] = scale;
        max_scale = GMAX(max_scale, scale);
    }
    if (!max_scale) {
        memset(y + 2, 0, 96);
        return;
    }
    const float d = max_scale / 31;
    put16(y, f32_to_f16(d * 1.0125f));
    const float id = 1 / d;
    for (int ib = 0; ib < 8; ++ib) {
        int l = near_int(0.5f * (id * scales[ib] - 1));
        l = GMAX(0, GMIN(15, l));
        sas[ib] |= (uint32_t)l << 28;
    }
    OPS(2 * C_DIV + 8 * 6);
    memcpy(y + 2, q3, 64);
    for (int ib = 0; ib < 8; ++ib)
        for (int j = 0; j < 4; ++j) y[2 + 64 + 4 * ib + j] = (uint8_t)((sas[ib] >> 8 * j) & 0xff);
}

/* ------------------------------------------------------------------ IQ3_S (gpuq/gpuq.hip:1145-1283) */
static void o_iq3_s(const float *xbl, const float *qwbl, uint8_t *y, const otab *t) {
    /* block_iq3_s: d(2) qs[64] qh[8] signs[32] scales[4] (gpuq/gpuq.hip:64) */
    const int kMaxQ = 8, bs = 32, bs4 = 8, bs8 = 4;
    float scales[8], weight[32], xval[32], waux[32];
    int8_t L[32], Laux[32];
    int on_grid[8], on_grid_aux[8];
    uint8_t bsg[4];
    memset(y, 0, 110);
    put16(y, f32_to_f16(0.f));
    uint8_t *qs = y + 2, *qh = y + 66, *signs = y + 74, *ysc = y + 106;
    float max_scale = 0;
    const float sigma2 = 2 * sum_sq(xbl, QK) / QK;
    for (int ib = 0; ib < QK / bs; ++ib) {
        const float *xb = xbl + bs * ib;
        iq_weights(qwbl + bs * ib, xb, sigma2, weight, bs);
        for (int i = 0; i < bs; ++i) waux[i] = sqrtf(weight[i]);
        OPS(32 * C_SQRT);
        for (int k = 0; k < bs8; ++k) {
            uint8_t s = 0;
            for (int i = 0; i < 8; ++i) {
                if (xb[8 * k + i] >= 0) xval[8 * k + i] = xb[8 * k + i];
                else { xval[8 * k + i] = -xb[8 * k + i]; s |= (uint8_t)(1 << i); }
            }
            OPS(8 * 3);
            bsg[k] = s;
        }
        float mx = xval[0];
        for (int i = 1; i < bs; ++i) mx = GMAX(mx, xval[i]);
        OPS(32);
        memset(L, 0, sizeof L);
        if (!mx) {   /* (the qs / signs cursors stay put, as in the reference: the next sub-block takes the slot) */
            scales[ib] = 0;
            continue;
        }
        float best = 0;
        float scale = mx / (2 * kMaxQ - 1);
        for (int k = 0; k < bs4; ++k) on_grid[k] = 0;
        OPS(C_DIV);
        for (int is = -9; is <= 9; ++is) {
            const float id = (2 * kMaxQ - 1 + is * 0.2f) / mx;
            const float this_scale = 1 / id;
            OPS(3 + 2 * C_DIV);
            for (int k = 0; k < bs4; ++k) {
                int u = 0;
                for (int i = 0; i < 4; ++i) {
                    const int l = near_int(0.5f * (id * xval[4 * k + i] - 1));
                    Laux[4 * k + i] = (int8_t)GMAX(0, GMIN(kMaxQ - 1, l));
                    u |= Laux[4 * k + i] << 3 * i;
                }
                OPS(4 * 5 + 1);
                const int m = map_at(t, u);
                on_grid_aux[k] = 1;
                if (m < 0) {
                    on_grid_aux[k] = 0;
                    nb_iq3(t, neigh_at(t, m), xval + 4 * k, waux + 4 * k, this_scale, Laux + 4 * k);
                }
            }
            float sumqx = 0, sumq2 = 0;
            for (int i = 0; i < bs; ++i) {
                const float w = weight[i];
                const float q = 2 * Laux[i] + 1;
                sumqx += w * xval[i] * q;
                sumq2 += w * q * q;
            }
            OPS(32 * 6 + 5);
            if (sumq2 > 0 && sumqx * sumqx > best * sumq2) {
                scale = sumqx / sumq2;
                best = scale * sumqx;
                memcpy(L, Laux, sizeof L);
                for (int k = 0; k < bs4; ++k) on_grid[k] = on_grid_aux[k];
                OPS(2 + C_DIV);
            }
        }
        int n_off = 0;
        for (int k = 0; k < bs4; ++k) if (!on_grid[k]) ++n_off;
        if (n_off > 0 && scale > 0) {
            const float id = 1 / scale;
            OPS(C_DIV);
            for (int k = 0; k < bs4; ++k) {
                int u = 0;
                for (int i = 0; i < 4; ++i) {
                    int l = near_int(0.5f * (id * xval[4 * k + i] - 1));
                    l = GMAX(0, GMIN(kMaxQ - 1, l));
                    u |= l << 3 * i;
                }
                OPS(4 * 5);
                int gi = map_at(t, u);
                if (gi < 0) gi = nb_iq3(t, neigh_at(t, gi), xval + 4 * k, waux + 4 * k, scale, L + 4 * k);
                const int8_t *pg = grid_pt(t, gi);
                for (int i = 0; i < 4; ++i) L[4 * k + i] = (int8_t)((pg[i] - 1) / 2);
            }
            float sumqx = 0, sumq2 = 0;
            for (int i = 0; i < bs; ++i) {
                const float w = weight[i];
                const float q = 2 * L[i] + 1;
                sumqx += w * xval[i] * q;
                sumq2 += w * q * q;
            }
            OPS(32 * 6 + C_DIV);
            if (sumq2 > 0) scale = sumqx / sumq2;
        }
        if (scale < 0) {
            scale = -scale;
            for (int k = 0; k < bs8; ++k) bsg[k] = (uint8_t)~bsg[k];
        }
        for (int k = 0; k < bs4; ++k) {
            int u = 0;
            for (int i = 0; i < 4; ++i) u |= L[4 * k + i] << 3 * i;
            const int gi = map_at(t, u);
            if (gi < 0) t_err = 1;
            qs[k] = (uint8_t)(gi & 255);
            qh[(ib * bs4 + k) / 8] |= (uint8_t)((gi >> 8) << ((ib * bs4 + k) % 8));
        }
        qs += bs4;
        for (int k = 0; k < bs8; ++k) signs[k] = bsg[k];
        signs += bs8;
        scales[ib] = scale;
        max_scale = GMAX(max_scale, scale);
    }
    if (!max_scale) return;
    const float d = max_scale / 31;
    put16(y, f32_to_f16(d * 1.033f));
    const float id = 1 / d;
    for (int ib = 0; ib < QK / bs; ib += 2) {
        int l1 = near_int(0.5f * (id * scales[ib + 0] - 1));
        l1 = GMAX(0, GMIN(15, l1));
        int l2 = near_int(0.5f * (id * scales[ib + 1] - 1));
        l2 = GMAX(0, GMIN(15, l2));
        ysc[ib / 2] = (uint8_t)(l1 | (l2 << 4));
    }
    OPS(2 * C_DIV + 8 * 6);
}

/* ------------------------------------------------------------------ IQ4_NL / IQ4_XS (gpuq/gpuq.hip:1285-1398) */
static const int8_t k_iq4nl[16] = {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113};

/* index of the nearest codebook value, the lower one on ties away from it (gpuq/gpuq.hip:1286-1295) */
static int nearest_iq4(float x, int value_only) {
    /* charged as the table form (the interval kv[ml] <= x < kv[ml+1] read from a table indexed by floor(x), the
     * codebook values being integers): floor-and-convert (one instruction), an integer clamp, NaN select, then the
     * two differences, their compare and two selects; where only the value is used (the trial scales, whose |x|
     * stays within the table for finite values) floor-and-convert, the two differences, their compare and one
     * select. The bisection below gives the same index (tests/test_iq4_table.py) */
    const int8_t *val = k_iq4nl;
    OPS(value_only ? 5 : 8);
    if (x <= val[0]) return 0;
    if (x >= val[15]) return 15;
    int lo = 0, hi = 15;
    while (hi - lo > 1) {
        const int mid = (lo + hi) / 2;
        if (x < val[mid]) hi = mid; else lo = mid;
    }
    return x - val[hi - 1] < val[hi] - x ? hi - 1 : hi;
}

static void iq4_impl(int SB, const float *x, uint8_t *dh, uint8_t *q4, uint16_t *scales_h, uint8_t *scales_l,
                     const float *qweights) {
    const int bsz = 32, ntry = 7;
    float scales[8], weight[32];
    uint8_t L[256];
    float sigma2 = 0;
    for (int j = 0; j < SB; ++j) sigma2 += x[j] * x[j];
    sigma2 *= 2.f / SB;
    OPS(2 * SB + 2);
    memset(q4, 0, SB / 2);
    put16(dh, f32_to_f16(0.f));
    float max_scale = 0, amax_scale = 0;
    for (int ib = 0; ib < SB / bsz; ++ib) {
        const float *xb = x + ib * bsz;
        uint8_t *Lb = L + ib * bsz;
        if (qweights) {
            iq_weights(qweights + ib * bsz, xb, sigma2, weight, bsz);
        } else {
            for (int j = 0; j < bsz; ++j) weight[j] = xb[j] * xb[j];
        }
        float amax = 0, mx = 0;
        for (int j = 0; j < bsz; ++j) {
            const float ax = fabsf(xb[j]);
            if (ax > amax) { amax = ax; mx = xb[j]; }
        }
        OPS(3 * bsz);
        if (amax < EPS_GROUP) {
            scales[ib] = 0;
            continue;
        }
        float d = ntry > 0 ? -mx / k_iq4nl[0] : mx / k_iq4nl[0];
        float id = 1 / d;
        float sumqx = 0, sumq2 = 0;
        for (int j = 0; j < bsz; ++j) {
            const float al = id * xb[j];
            const int l = nearest_iq4(al, 0);
            Lb[j] = (uint8_t)l;
            const float q = k_iq4nl[l];
            const float w = weight[j];
            sumqx += w * q * xb[j];
            sumq2 += w * q * q;
        }
        OPS(2 * C_DIV + bsz * 7 + C_DIV + 2);
        d = sumq2 > 0 ? sumqx / sumq2 : 0.f;
        float best = d * sumqx;
        for (int itry = -ntry; itry <= ntry; ++itry) {
            id = (itry + k_iq4nl[0]) / mx;
            sumqx = sumq2 = 0;
            for (int j = 0; j < bsz; ++j) {
                const float al = id * xb[j];
                const int l = nearest_iq4(al, 1);
                const float q = k_iq4nl[l];
                const float w = weight[j];
                sumqx += w * q * xb[j];
                sumq2 += w * q * q;
            }
            OPS(2 + C_DIV + bsz * 7 + 4);
            if (sumq2 > 0 && sumqx * sumqx > best * sumq2) {
                d = sumqx / sumq2;
                best = d * sumqx;
                OPS(1 + C_DIV);
            }
        }
        scales[ib] = d;
        const float abs_d = fabsf(d);
        if (abs_d > amax_scale) { amax_scale = abs_d; max_scale = d; }
    }
    if (SB / bsz > 1) {
        const int nb = SB / bsz;
        for (int i = 0; i < (nb + 7) / 8; ++i) scales_h[i] = 0;
        const float d = -max_scale / 32;
        put16(dh, f32_to_f16(d));
        const float id = d ? 1 / d : 0.f;
        OPS(2 * C_DIV);
        for (int ib = 0; ib < nb; ++ib) {
            int l = near_int(id * scales[ib]);
            l = GMAX(-32, GMIN(31, l));
            const float dl = d * l;
            const float idl = dl ? 1 / dl : 0.f;
            uint8_t *Lb = L + ib * bsz;
            const float *xb = x + ib * bsz;
            for (int j = 0; j < bsz; ++j) Lb[j] = (uint8_t)nearest_iq4(idl * xb[j], 0);
            OPS(6 + C_DIV + bsz);
            l += 32;
            const uint8_t l_l = (uint8_t)(l & 0xf);
            const uint8_t l_h = (uint8_t)(l >> 4);
            if (ib % 2 == 0) scales_l[ib / 2] = l_l;
            else scales_l[ib / 2] |= (uint8_t)(l_l << 4);
            scales_h[ib / 8] |= (uint16_t)(l_h << 2 * (ib % 8));
        }
    } else {
        put16(dh, f32_to_f16(scales[0]));
        const float id = scales[0] ? 1 / scales[0] : 0;
        for (int j = 0; j < SB; ++j) L[j] = (uint8_t)nearest_iq4(id * x[j], 0);
        OPS(C_DIV + SB);
    }
    for (int i = 0; i < SB / 32; ++i)
        for (int j = 0; j < 16; ++j) q4[16 * i + j] = (uint8_t)(L[32 * i + j] | (L[32 * i + 16 + j] << 4));
}

static void o_iq4_xs(const float *xbl, const float *qwbl, uint8_t *y) {
    /* block_iq4_xs: d(2) scales_h(2) scales_l[4] qs[128] (gpuq/gpuq.hip:66) */
    uint16_t sh = 0;
    iq4_impl(QK, xbl, y, y + 8, &sh, y + 4, qwbl);
    put16(y + 2, sh);
}
static void o_iq4_nl(const float *xbl, const float *qwbl, uint8_t *y) {
    /* block_iq4_nl: d(2) qs[16] (gpuq/gpuq.hip:65) */
    uint16_t unused_h;
    iq4_impl(32, xbl, y, y + 2, &unused_h, NULL, qwbl);
}

/* ------------------------------------------------------------------ k-quants (gpuq/gpuq.hip:1403-1829) */
static inline float kw(const float *qw, const float *x, int i) { return qw ? qw[i] : x[i] * x[i]; }

/* symmetric levels in [0, 2*nmax) around a signed scale, best of 19 trial scales (gpuq/gpuq.hip:1427-1466) */
static float sym_levels(int n, int nmax, const float *x, int8_t *L, const float *qw) {
    float amax = 0, mx = 0;
    for (int i = 0; i < n; ++i) {
        const float ax = fabsf(x[i]);
        if (ax > amax) { amax = ax; mx = x[i]; }
    }
    OPS(3 * n);
    if (amax < EPS_GROUP) {
        for (int i = 0; i < n; ++i) L[i] = 0;
        return 0.f;
    }
    float iscale = -nmax / mx;
    float sumlx = 0, suml2 = 0;
    for (int i = 0; i < n; ++i) {
        const int l = GMAX(-nmax, GMIN(nmax - 1, near_int(iscale * x[i])));
        L[i] = (int8_t)(l + nmax);
        const float w = kw(qw, x, i);
        sumlx += w * x[i] * l;
        suml2 += w * l * l;
    }
    OPS(C_DIV + n * 10 + C_DIV + 2);
    float scale = suml2 ? sumlx / suml2 : 0.0f;
    float best = scale * sumlx;
    for (int is = -9; is <= 9; ++is) {
        if (is == 0) continue;
        iscale = -(nmax + 0.1f * is) / mx;
        sumlx = suml2 = 0;
        for (int i = 0; i < n; ++i) {
            const int l = GMAX(-nmax, GMIN(nmax - 1, near_int(iscale * x[i])));
            const float w = kw(qw, x, i);
            sumlx += w * x[i] * l;
            suml2 += w * l * l;
        }
        OPS(3 + C_DIV + n * 9 + 5);
        if (suml2 > 0 && sumlx * sumlx > best * suml2) {
            for (int i = 0; i < n; ++i) L[i] = (int8_t)(nmax + GMAX(-nmax, GMIN(nmax - 1, near_int(iscale * x[i]))));
            scale = sumlx / suml2;
            best = scale * sumlx;
            OPS(C_DIV + 1);
        }
    }
    return scale;
}

/* Q3_K's no-imatrix levels: 3-bit symmetric rounding then up to 5 coordinate-descent passes on x^2-weighted error
 * (gpuq/gpuq.hip:1468-1508) */
static float sym3_levels(int n, int nmax, const float *x, int8_t *L) {
    float amax = 0, mx = 0;
    for (int i = 0; i < n; ++i) {
        const float ax = fabsf(x[i]);
        if (ax > amax) { amax = ax; mx = x[i]; }
    }
    OPS(3 * n);
    if (amax < EPS_GROUP) {
        for (int i = 0; i < n; ++i) L[i] = 0;
        return 0.f;
    }
    const float iscale = -nmax / mx;
    float sumlx = 0, suml2 = 0;
    for (int i = 0; i < n; ++i) {
        const int l = GMAX(-nmax, GMIN(nmax - 1, near_int(iscale * x[i])));
        L[i] = (int8_t)l;
        const float w = x[i] * x[i];
        sumlx += w * x[i] * l;
        suml2 += w * l * l;
    }
    OPS(C_DIV + n * 13);
    for (int pass = 0; pass < 5; ++pass) {
        int changed = 0;
        for (int i = 0; i < n; ++i) {
            const float w = x[i] * x[i];
            float slx = sumlx - w * x[i] * L[i];
            OPS(6);
            if (!(slx > 0)) continue;
            float sl2 = suml2 - w * L[i] * L[i];
            const int nl = GMAX(-nmax, GMIN(nmax - 1, near_int(x[i] * sl2 / slx)));
            OPS(8 + C_DIV);
            if (nl == L[i]) continue;
            slx += w * x[i] * nl;
            sl2 += w * nl * nl;
            OPS(17);
            if (sl2 > 0 && slx * slx * suml2 > sumlx * sumlx * sl2) {
                L[i] = (int8_t)nl; sumlx = slx; suml2 = sl2;
                ++changed;
            }
        }
        if (!changed) break;
    }
    for (int i = 0; i < n; ++i) L[i] = (int8_t)(L[i] + nmax);
    OPS(1 + C_DIV);
    return suml2 > 0.0f ? sumlx / suml2 : 0.0f;
}

/* affine levels in [0, nmax], x ~ scale*L - the_min, over nstep+1 trial scales; with_im selects ggml's imatrix
 * search (make_qkx3) or the plain one (make_qkx2) (gpuq/gpuq.hip:1510-1587) */
static float affine_levels(int with_im, int n, int nmax, const float *x, const float *weights, uint8_t *L,
                           float *the_min, uint8_t *Laux, float rmin, float rdelta, int nstep, int use_mad) {
    float mn = x[0], mx = x[0];
    float sum_w = with_im ? kw(weights, x, 0) : weights[0];
    float sum_x = sum_w * x[0];
    for (int i = 1; i < n; ++i) {
        if (x[i] < mn) mn = x[i];
        if (x[i] > mx) mx = x[i];
        const float w = with_im ? kw(weights, x, i) : weights[i];
        sum_w += w;
        sum_x += w * x[i];
    }
    OPS(1 + n * 5 + 1);
    if (mn > 0) mn = 0;
    if (with_im ? mx <= mn : mx == mn) {
        for (int i = 0; i < n; ++i) L[i] = 0;
        *the_min = -mn;
        return 0.f;
    }
    float iscale = nmax / (mx - mn);
    float scale = 1 / iscale;
    float best = 0;
    for (int i = 0; i < n; ++i) {
        L[i] = (uint8_t)GMAX(0, GMIN(nmax, near_int(iscale * (x[i] - mn))));
        float diff = scale * L[i] + mn - x[i];
        diff = use_mad ? fabsf(diff) : diff * diff;
        const float w = with_im ? kw(weights, x, i) : weights[i];
        best += w * diff;
    }
    OPS(2 + 2 * C_DIV + n * 11);
    if (nstep < 1) {
        *the_min = -mn;
        return scale;
    }
    for (int is = 0; is <= nstep; ++is) {
        iscale = (rmin + rdelta * is + nmax) / (mx - mn);
        float sum_l = 0, sum_l2 = 0, sum_xl = 0;
        for (int i = 0; i < n; ++i) {
            int l;
            if (with_im) {
                const float v = iscale * (x[i] - mn);
                l = v > 0 ? near_int(v < nmax ? v : (float)nmax) : 0;
            } else {
                l = GMAX(0, GMIN(nmax, near_int(iscale * (x[i] - mn))));
            }
            Laux[i] = (uint8_t)l;
            const float w = with_im ? kw(weights, x, i) : weights[i];
            sum_l += w * l;
            sum_l2 += w * l * l;
            sum_xl += w * l * x[i];
        }
        const float D = sum_w * sum_l2 - sum_l * sum_l;
        /* a level with the imatrix rule: x - mn, the product, one clamp to [0, nmax] (NaN to 0) and the rounding
         * of a value in [0, nmax] as two float adds (exact there); the plain rule's ggml rounding of an unbounded
         * value is the integer nearest_int plus the clamp and a conversion; then the three sums (6) */
        OPS(5 + C_DIV + n * (with_im ? 11 : 13) + 4);
        if (!(D > 0)) continue;
        float this_scale = (sum_w * sum_xl - sum_x * sum_l) / D;
        float this_min = (sum_l2 * sum_x - sum_l * sum_xl) / D;
        OPS(6 + 2 * C_DIV + 1);
        if (this_min > 0) {
            this_min = 0;
            this_scale = sum_xl / sum_l2;
            OPS(C_DIV);
        }
        float err = 0;
        for (int i = 0; i < n; ++i) {
            float diff = this_scale * Laux[i] + this_min - x[i];
            diff = use_mad ? fabsf(diff) : diff * diff;
            const float w = with_im ? kw(weights, x, i) : weights[i];
            err += w * diff;
        }
        OPS(n * (with_im ? 6 : 7) + 1);     /* (the imatrix rule's levels are floats already: no conversion) */
        if (err < best) {
            for (int i = 0; i < n; ++i) L[i] = Laux[i];
            best = err;
            scale = this_scale;
            mn = this_min;
        }
    }
    *the_min = -mn;
    return scale;
}

/* four 2-bit fields, 32 apart, a byte (gpuq/gpuq.hip:1589-1594) */
static void pack2(const uint8_t *L, uint8_t *qs) {
    for (int base = 0; base < QK; base += 128)
        for (int l = 0; l < 32; ++l)
            qs[base / 4 + l] = (uint8_t)(L[base + l] | (L[base + l + 32] << 2) | (L[base + l + 64] << 4) |
                                         (L[base + l + 96] << 6));
}

/* Q4_K / Q5_K 12-byte scale block: eight 6-bit scales and mins (gpuq/gpuq.hip:1596-1608) */
static void k4_pack(const uint8_t *ls, const uint8_t *lm, uint8_t *s) {
    for (int j = 0; j < 4; ++j) { s[j] = ls[j]; s[j + 4] = lm[j]; }
    for (int j = 4; j < 8; ++j) {
        s[j + 4] = (uint8_t)((ls[j] & 0xF) | ((lm[j] & 0xF) << 4));
        s[j - 4] |= (uint8_t)((ls[j] >> 4) << 6);
        s[j] |= (uint8_t)((lm[j] >> 4) << 6);
    }
}
static void k4_unpack(int j, const uint8_t *s, uint8_t *sc, uint8_t *m) {
    if (j < 4) { *sc = s[j] & 63; *m = s[j + 4] & 63; }
    else { *sc = (uint8_t)((s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4)); *m = (uint8_t)((s[j + 4] >> 4) | ((s[j] >> 6) << 4)); }
}

/* final affine rounding against the stored scales (gpuq/gpuq.hip:1610-1619) */
static void affine_final(const float *x, uint8_t *L, int g, int ng, int nmax, float d, float dmin, const uint8_t *sc,
                         const uint8_t *mn) {
    for (int j = 0; j < ng; ++j) {
        const float dj = d * sc[j];
        OPS(2);
        if (!dj) continue;
        const float mj = dmin * mn[j];
        for (int i = 0; i < g; ++i) L[g * j + i] = (uint8_t)GMAX(0, GMIN(nmax, near_int((x[g * j + i] + mj) / dj)));
        OPS(2 + g * (2 + C_DIV));
    }
}

/* Q2_K (gpuq/gpuq.hip:1621-1668); block: scales[16] qs[64] d dmin */
static void o_q2_k(const float *x, const float *qw, uint8_t *y) {
    uint8_t L[QK], Laux[16], Ls[16], Lm[16];
    float scales[16], mins[16], w[16];
    uint8_t *ysc = y, *qs = y + 16;
    if (!qw) {
        float max_scale = 0, max_min = 0;
        for (int j = 0; j < 16; ++j) {
            for (int l = 0; l < 16; ++l) w[l] = fabsf(x[16 * j + l]);
            scales[j] = affine_levels(0, 16, 3, x + 16 * j, w, L + 16 * j, &mins[j], Laux, -0.5f, 0.1f, 15, 1);
            if (scales[j] > max_scale) max_scale = scales[j];
            if (mins[j] > max_min) max_min = mins[j];
        }
        for (int j = 0; j < 16; ++j) ysc[j] = 0;
        if (max_scale > 0) {
            const float is = 15.f / max_scale;
            for (int j = 0; j < 16; ++j) ysc[j] = (uint8_t)near_int(is * scales[j]);
            put16(y + 80, f32_to_f16(max_scale / 15.f));
        } else {
            put16(y + 80, f32_to_f16(0.f));
        }
        if (max_min > 0) {
            const float im = 15.f / max_min;
            for (int j = 0; j < 16; ++j) ysc[j] |= (uint8_t)(near_int(im * mins[j]) << 4);
            put16(y + 82, f32_to_f16(max_min / 15.f));
        } else {
            put16(y + 82, f32_to_f16(0.f));
        }
    } else {
        const float sigma2 = sum_sq(x, QK) / QK;
        float sw[16];
        for (int j = 0; j < 16; ++j) {
            iq_weights(qw + 16 * j, x + 16 * j, sigma2, w, 16);
            sw[j] = 0;
            for (int l = 0; l < 16; ++l) sw[j] += w[l];
            scales[j] = affine_levels(1, 16, 3, x + 16 * j, w, L + 16 * j, &mins[j], Laux, -0.9f, 0.05f, 36, 0);
        }
        const float dm = qp_levels(16, 15, scales, Ls, sw);
        const float mm = qp_levels(16, 15, mins, Lm, sw);
        put16(y + 80, f32_to_f16(dm));
        put16(y + 82, f32_to_f16(mm));
        for (int j = 0; j < 16; ++j) ysc[j] = (uint8_t)(Ls[j] | (Lm[j] << 4));
    }
    uint8_t sc[16], mn[16];
    for (int j = 0; j < 16; ++j) { sc[j] = ysc[j] & 0xF; mn[j] = ysc[j] >> 4; }
    affine_final(x, L, 16, 16, 3, f16_to_f32(get16(y + 80)), f16_to_f32(get16(y + 82)), sc, mn);
    pack2(L, qs);
}

/* Q3_K (gpuq/gpuq.hip:1670-1724); block: hmask[32] qs[64] scales[12] d */
static void o_q3_k(const float *x, const float *qw, uint8_t *y) {
    int8_t L[QK], Ls[16];
    float scales[16];
    uint8_t *hmask = y, *qs = y + 32, *ysc = y + 96;
    for (int j = 0; j < 12; ++j) ysc[j] = 0;
    if (!qw) {
        float amax = 0, max_scale = 0;
        for (int j = 0; j < 16; ++j) {
            scales[j] = sym3_levels(16, 4, x + 16 * j, L + 16 * j);
            const float a = fabsf(scales[j]);
            if (a > amax) { amax = a; max_scale = scales[j]; }
        }
        if (max_scale) {
            const float iscale = -32.f / max_scale;
            for (int j = 0; j < 16; ++j) {
                const int8_t l = (int8_t)near_int(iscale * scales[j]);
                Ls[j] = (int8_t)(GMAX(-32, GMIN(31, l)) + 32);
            }
            put16(y + 108, f32_to_f16(1 / iscale));
        } else {
            for (int j = 0; j < 16; ++j) Ls[j] = -1;
            put16(y + 108, f32_to_f16(0.f));
        }
    } else {
        const float sigma2 = 2 * sum_sq(x, QK) / QK;
        float w[16], sw[16];
        for (int j = 0; j < 16; ++j) {
            iq_weights(qw + 16 * j, x + 16 * j, sigma2, w, 16);
            float s = 0;
            for (int l = 0; l < 16; ++l) s += w[l];
            sw[j] = s;
            scales[j] = sym_levels(16, 4, x + 16 * j, L + 16 * j, w);
        }
        put16(y + 108, f32_to_f16(sym_levels(16, 32, scales, Ls, sw)));
    }
    for (int j = 0; j < 16; ++j) {
        if (Ls[j] < 0) break;
        const int l = Ls[j];
        if (j < 8) ysc[j] = (uint8_t)(l & 0xF); else ysc[j - 8] |= (uint8_t)((l & 0xF) << 4);
        ysc[j % 4 + 8] |= (uint8_t)((l >> 4) << (2 * (j / 4)));
    }
    const float d = f16_to_f32(get16(y + 108));
    for (int j = 0; j < 16; ++j) {
        int8_t sc = (int8_t)(j < 8 ? ysc[j] & 0xF : ysc[j - 8] >> 4);
        sc = (int8_t)((sc | (((ysc[8 + j % 4] >> (2 * (j / 4))) & 3) << 4)) - 32);
        const float dj = d * sc;
        OPS(2);
        if (!dj) continue;
        for (int i = 0; i < 16; ++i) L[16 * j + i] = (int8_t)(GMAX(-4, GMIN(3, near_int(x[16 * j + i] / dj))) + 4);
        OPS(16 * (C_DIV + 2));
    }
    for (int j = 0; j < 32; ++j) hmask[j] = 0;
    for (int j = 0; j < QK; ++j)
        if (L[j] > 3) { hmask[j % 32] |= (uint8_t)(1 << (j / 32)); L[j] = (int8_t)(L[j] - 4); }
    pack2((const uint8_t *)L, qs);
}

/* Q4_K / Q5_K (gpuq/gpuq.hip:1726-1774) */
static void affine32(int nmax, const float *x, const float *qw, uint8_t *y, uint8_t *L, float rmin_plain,
                     int nstep_plain) {
    uint8_t Laux[32], ls[8], lm[8];
    float scales[8], mins[8], w[32];
    if (!qw) {
        float max_scale = 0, max_min = 0;
        for (int j = 0; j < 8; ++j) {
            const float s2 = sum_sq(x + 32 * j, 32);
            const float av = sqrtf(s2 / 32);
            for (int l = 0; l < 32; ++l) w[l] = av + fabsf(x[32 * j + l]);
            OPS(C_DIV + C_SQRT + 64);
            scales[j] = affine_levels(0, 32, nmax, x + 32 * j, w, L + 32 * j, &mins[j], Laux, rmin_plain, 0.1f,
                                      nstep_plain, 0);
            if (scales[j] > max_scale) max_scale = scales[j];
            if (mins[j] > max_min) max_min = mins[j];
        }
        const float is = max_scale > 0 ? 63.f / max_scale : 0.f;
        const float im = max_min > 0 ? 63.f / max_min : 0.f;
        for (int j = 0; j < 8; ++j) {
            const uint8_t a = (uint8_t)near_int(is * scales[j]), b = (uint8_t)near_int(im * mins[j]);
            ls[j] = GMIN(63, a);
            lm[j] = GMIN(63, b);
        }
        put16(y, f32_to_f16(max_scale / 63.f));
        put16(y + 2, f32_to_f16(max_min / 63.f));
    } else {
        const float sigma2 = 2 * sum_sq(x, QK) / QK;
        float sw[8];
        for (int j = 0; j < 8; ++j) {
            iq_weights(qw + 32 * j, x + 32 * j, sigma2, w, 32);
            float s = 0;
            for (int l = 0; l < 32; ++l) s += w[l];
            sw[j] = s;
            scales[j] = affine_levels(1, 32, nmax, x + 32 * j, w, L + 32 * j, &mins[j], Laux, -0.9f, 0.05f, 36, 0);
        }
        const float db = qp_levels(8, 63, scales, ls, sw);
        const float mb = qp_levels(8, 63, mins, lm, sw);
        if (nmax == 31) for (int j = 0; j < 8; ++j) { ls[j] = GMIN(63, ls[j]); lm[j] = GMIN(63, lm[j]); }
        put16(y, f32_to_f16(db));
        put16(y + 2, f32_to_f16(mb));
    }
    k4_pack(ls, lm, y + 4);
    uint8_t sc[8], mn[8];
    for (int j = 0; j < 8; ++j) k4_unpack(j, y + 4, &sc[j], &mn[j]);
    affine_final(x, L, 32, 8, nmax, f16_to_f32(get16(y)), f16_to_f32(get16(y + 2)), sc, mn);
}

/* block_q4_K: d dmin scales[12] qs[128] (gpuq/gpuq.hip:1776-1781) */
static void o_q4_k(const float *x, const float *qw, uint8_t *y) {
    uint8_t L[QK];
    affine32(15, x, qw, y, L, -1.f, 20);
    uint8_t *qs = y + 16;
    for (int base = 0, o = 0; base < QK; base += 64, o += 32)
        for (int l = 0; l < 32; ++l) qs[o + l] = (uint8_t)(L[base + l] | (L[base + l + 32] << 4));
}

/* block_q5_K: d dmin scales[12] qh[32] qs[128] (gpuq/gpuq.hip:1783-1794) */
static void o_q5_k(const float *x, const float *qw, uint8_t *y) {
    uint8_t L[QK];
    affine32(31, x, qw, y, L, -0.5f, 15);
    uint8_t *qh = y + 16, *qs = y + 48;
    for (int j = 0; j < 32; ++j) qh[j] = 0;
    for (int base = 0, o = 0, bit = 0; base < QK; base += 64, o += 32, bit += 2)
        for (int j = 0; j < 32; ++j) {
            int a = L[base + j], b = L[base + j + 32];
            if (a > 15) { a -= 16; qh[j] |= (uint8_t)(1 << bit); }
            if (b > 15) { b -= 16; qh[j] |= (uint8_t)(2 << bit); }
            qs[o + j] = (uint8_t)(a | (b << 4));
        }
}

/* block_q6_K: ql[128] qh[64] scales[16] d (gpuq/gpuq.hip:1796-1829) */
static void o_q6_k(const float *x, const float *qw, uint8_t *y) {
    int8_t L[QK];
    float scales[16];
    float amax = 0, max_scale = 0;
    uint8_t *ql = y, *qh = y + 128;
    int8_t *ysc = (int8_t *)(y + 192);
    for (int b = 0; b < 16; ++b) {
        scales[b] = sym_levels(16, 32, x + 16 * b, L + 16 * b, qw ? qw + 16 * b : NULL);
        const float a = fabsf(scales[b]);
        if (a > amax) { amax = a; max_scale = scales[b]; }
    }
    if (amax < EPS_GROUP) {
        memset(y, 0, 210);
        return;
    }
    const float iscale = -128.f / max_scale;
    put16(y + 208, f32_to_f16(1 / iscale));
    for (int b = 0; b < 16; ++b) ysc[b] = (int8_t)GMIN(127, near_int(iscale * scales[b]));
    OPS(2 * C_DIV + 16 * 4);
    const float d = f16_to_f32(get16(y + 208));
    for (int j = 0; j < 16; ++j) {
        const float dj = d * ysc[j];
        OPS(2);
        if (!dj) continue;
        for (int i = 0; i < 16; ++i) L[16 * j + i] = (int8_t)(GMAX(-32, GMIN(31, near_int(x[16 * j + i] / dj))) + 32);
        OPS(16 * (C_DIV + 2));
    }
    for (int half = 0; half < 2; ++half) {
        const int8_t *Lh = L + 128 * half;
        uint8_t *qlh = ql + 64 * half, *qhh = qh + 32 * half;
        for (int l = 0; l < 32; ++l) {
            qlh[l] = (uint8_t)((Lh[l] & 0xF) | ((Lh[l + 64] & 0xF) << 4));
            qlh[l + 32] = (uint8_t)((Lh[l + 32] & 0xF) | ((Lh[l + 96] & 0xF) << 4));
            qhh[l] = (uint8_t)((Lh[l] >> 4) | ((Lh[l + 32] >> 4) << 2) | ((Lh[l + 64] >> 4) << 4) | ((Lh[l + 96] >> 4) << 6));
        }
    }
}

/* block_q8_0: d qs[32] (gpuq/gpuq.hip:1831-1838) */
static void o_q8_0(const float *x, uint8_t *y) {
    float amax = 0.0f;
    for (int j = 0; j < 32; ++j) amax = GMAX(amax, fabsf(x[j]));
    const float d = amax / 127;
    const float id = d ? 1.0f / d : 0.0f;
    put16(y, f32_to_f16(d));
    for (int j = 0; j < 32; ++j) y[2 + j] = (uint8_t)(int8_t)roundf(x[j] * id);
    OPS(32 + 2 * C_DIV + 2 + 32 * 4);
}

/* ------------------------------------------------------------------ llama-quantize's fallback types
 * Q4_0 / Q5_0 / Q5_1 and F16, for rows that are not whole 256-weight super-blocks (tools/requant_experts.py:180-192);
 * the reference writes them through ggml on the CPU (tools/requant_experts.py:732-747, ggml_quantize_chunk). ggml is a
 * third-party library absent from the reference (llama.cpp's ggml-quants.c, the revision its build.sh compiles):
 * without an imatrix quantize_row_q4_0_ref / q5_0_ref / q5_1_ref, with one quantize_row_q4_0_impl / q5_0_impl /
 * q5_1_impl (weights qw * sqrt(sigma2 + x^2), sigma2 the mean of x^2 over the whole row; make_qx_quants(32, nmax, x,
 * L, 1, weight) = sym_levels above, make_qkx3_quants(32, 31, ..., -0.9, 0.05, 36, false) = affine_levels above); F16
 * is ggml_fp32_to_fp16_row (GGML_FP32_TO_FP16 a value). */

/* C's float -> int8_t / uint8_t conversion as x86 builds of ggml perform it: cvttss2si (INT_MIN for NaN or out of
 * range), then the low byte */
static inline int cvt_i32_x86(float v) { return (v >= -2147483648.f && v < 2147483648.f) ? (int)v : INT32_MIN; }
static inline int cvt_i8_x86(float v) { return (int)(int8_t)(uint8_t)((uint32_t)cvt_i32_x86(v) & 0xffu); }
static inline uint8_t cvt_u8_x86(float v) { return (uint8_t)((uint32_t)cvt_i32_x86(v) & 0xffu); }

/* 5-bit levels into ggml's Q5 layout: qh bit j (j < 16: value j, else value j), qs[j] = low nibbles of j, j + 16 */
static void q5_pack(const uint8_t *lv, uint8_t *qh4, uint8_t *qs) {
    uint32_t qh = 0;
    for (int j = 0; j < 16; ++j) {
        qs[j] = (uint8_t)((lv[j] & 0x0F) | ((lv[j + 16] & 0x0F) << 4));
        qh |= ((lv[j] & 0x10u) >> 4) << j;
        qh |= ((lv[j + 16] & 0x10u) >> 4) << (j + 16);
    }
    memcpy(qh4, &qh, 4);
}

/* Q4_0 (nmax 8, 18-byte blocks d qs[16]) and Q5_0 (nmax 16, 22 bytes d qh[4] qs[16]); qw NULL: the _ref rule */
static void o_q0(int nmax, const float *x, const float *qw, float sigma2, uint8_t *y) {
    uint8_t lv[32];
    float d;
    if (!qw) {
        float amax = 0.0f, mx = 0.0f;
        for (int j = 0; j < 32; ++j) {
            const float v = x[j];
            if (amax < fabsf(v)) { amax = fabsf(v); mx = v; }
        }
        d = mx / -(float)nmax;
        const float id = d ? 1.0f / d : 0.0f;
        for (int j = 0; j < 32; ++j) {
            const int l = cvt_i8_x86(x[j] * id + ((float)nmax + 0.5f));
            lv[j] = (uint8_t)GMIN(2 * nmax - 1, l);
        }
        OPS(32 * 3 + 2 * C_DIV + 32 * 5);
    } else {
        float w[32];
        int8_t L[32];
        iq_weights(qw, x, sigma2, w, 32);
        d = sym_levels(32, nmax, x, L, w);
        for (int j = 0; j < 32; ++j) lv[j] = (uint8_t)L[j];
    }
    put16(y, f32_to_f16(d));
    if (nmax == 8) {
        for (int j = 0; j < 16; ++j) y[2 + j] = (uint8_t)(lv[j] | (lv[j + 16] << 4));
    } else {
        q5_pack(lv, y + 2, y + 6);
    }
}

/* Q5_1: d m qh[4] qs[16], x ~ d * l + m; qw NULL: the _ref rule */
static void o_q5_1(const float *x, const float *qw, float sigma2, uint8_t *y) {
    uint8_t lv[32];
    float d, m;
    if (!qw) {
        float mn = FLT_MAX, mx = -FLT_MAX;
        for (int j = 0; j < 32; ++j) {
            if (x[j] < mn) mn = x[j];
            if (x[j] > mx) mx = x[j];
        }
        d = (mx - mn) / ((1 << 5) - 1);
        m = mn;
        const float id = d ? 1.0f / d : 0.0f;
        for (int j = 0; j < 32; ++j) lv[j] = cvt_u8_x86((x[j] - mn) * id + 0.5f);
        OPS(32 * 2 + 2 * C_DIV + 32 * 4);
    } else {
        float w[32], the_min;
        uint8_t Laux[32];
        iq_weights(qw, x, sigma2, w, 32);
        d = affine_levels(1, 32, 31, x, w, lv, &the_min, Laux, -0.9f, 0.05f, 36, 0);
        m = -the_min;
    }
    put16(y, f32_to_f16(d));
    put16(y + 2, f32_to_f16(m));
    q5_pack(lv, y + 4, y + 8);
}

static int legacy_type(int type) { return type == GQO_Q4_0 || type == GQO_Q5_0 || type == GQO_Q5_1; }

/* one row of a fallback type: the imatrix rules' sigma2 is sum(x^2) over the row, in index order, over its length */
static void quant_row_legacy(int type, const float *x, int64_t n, const float *qw, uint8_t *y) {
    float sigma2 = 0.f;
    if (qw) {
        float s = 0;
        for (int64_t j = 0; j < n; ++j) s += x[j] * x[j];
        sigma2 = s / (float)n;
        OPS(2 * n + C_DIV);
    }
    const size_t bb = type == GQO_Q4_0 ? 18 : type == GQO_Q5_0 ? 22 : 24;
    for (int64_t ib = 0; ib < n / 32; ++ib) {
        const float *xb = x + 32 * ib, *wb = qw ? qw + 32 * ib : NULL;
        if (type == GQO_Q5_1) o_q5_1(xb, wb, sigma2, y + ib * bb);
        else o_q0(type == GQO_Q4_0 ? 8 : 16, xb, wb, sigma2, y + ib * bb);
    }
}

/* ------------------------------------------------------------------ type traits and dispatch */
size_t gqo_block_bytes(int type) {
    switch (type) {
        case GQO_IQ2_XXS: return 66;
        case GQO_IQ2_S: return 82;
        case GQO_IQ1_S: return 50;
        case GQO_IQ1_M: return 56;
        case GQO_IQ2_XS: return 74;
        case GQO_IQ3_XXS: return 98;
        case GQO_IQ3_S: return 110;
        case GQO_IQ4_NL: return 18;
        case GQO_IQ4_XS: return 136;
        case GQO_Q2_K: return 84;
        case GQO_Q3_K: return 110;
        case GQO_Q4_K: return 144;
        case GQO_Q5_K: return 176;
        case GQO_Q6_K: return 210;
        case GQO_Q8_0: return 34;
        case GQO_Q4_0: return 18;
        case GQO_Q5_0: return 22;
        case GQO_Q5_1: return 24;
        case GQO_F16: return 2;
        default: return 0;
    }
}
int gqo_block_len(int type) {
    if (type == GQO_F16) return 1;
    if (type == GQO_IQ4_NL || type == GQO_Q8_0 || legacy_type(type)) return 32;
    return gqo_block_bytes(type) ? QK : 0;
}

static int needs_tables(int type) {
    return type == GQO_IQ2_XXS || type == GQO_IQ2_XS || type == GQO_IQ2_S || type == GQO_IQ1_S || type == GQO_IQ1_M ||
           type == GQO_IQ3_XXS || type == GQO_IQ3_S;
}
static int takes_no_imatrix(int type) {
    return type == GQO_Q2_K || type == GQO_Q3_K || type == GQO_Q4_K || type == GQO_Q5_K || type == GQO_Q6_K ||
           type == GQO_Q8_0 || type == GQO_IQ4_NL || type == GQO_IQ4_XS || legacy_type(type) || type == GQO_F16;
}

static void quant_block(int type, const float *x, const float *qw, uint8_t *y, const otab *t) {
    switch (type) {
        case GQO_IQ2_XXS: o_iq2_xxs(x, qw, y, t); break;
        case GQO_IQ2_XS: o_iq2_xs(x, qw, y, t); break;
        case GQO_IQ2_S: o_iq2_s(x, qw, y, t); break;
        case GQO_IQ1_S: o_iq1_s(x, qw, y, t); break;
        case GQO_IQ1_M: o_iq1_m(x, qw, y, t); break;
        case GQO_IQ3_XXS: o_iq3_xxs(x, qw, y, t); break;
        case GQO_IQ3_S: o_iq3_s(x, qw, y, t); break;
        case GQO_IQ4_XS: o_iq4_xs(x, qw, y); break;
        case GQO_IQ4_NL: o_iq4_nl(x, qw, y); break;
        case GQO_Q2_K: o_q2_k(x, qw, y); break;
        case GQO_Q3_K: o_q3_k(x, qw, y); break;
        case GQO_Q4_K: o_q4_k(x, qw, y); break;
        case GQO_Q5_K: o_q5_k(x, qw, y); break;
        case GQO_Q6_K: o_q6_k(x, qw, y); break;
        case GQO_Q8_0: o_q8_0(x, y); break;
        default: t_err = 1;
    }
}

size_t gqo_quantize_chunk(int type, const float *src, void *dst, int64_t start, int64_t nrows, int64_t n_per_row,
                         const float *imatrix) {
    const size_t bb = gqo_block_bytes(type);
    const int bs = gqo_block_len(type);
    if (!bb || nrows < 0 || n_per_row <= 0 || n_per_row % bs || start % n_per_row) return 0;
    if (!imatrix && !takes_no_imatrix(type)) return 0;
    const otab *t = NULL;
    if (needs_tables(type)) {
        t = tab_search(type);
        if (!t) return 0;
    }
    if (type == GQO_Q8_0 || type == GQO_F16) imatrix = NULL;   /* (ggml_quantize_chunk ignores it for these) */
    const int64_t nb_row = n_per_row / bs;
    const size_t row_size = (size_t)nb_row * bb;
    uint8_t *out = (uint8_t *)dst + (size_t)(start / n_per_row) * row_size;
    t_err = 0;
    if (type == GQO_F16) {
        for (int64_t i = 0; i < nrows * n_per_row; ++i) put16(out + 2 * i, f32_to_f16(src[start + i]));
        ops_flush();
        return (size_t)nrows * row_size;
    }
    if (legacy_type(type)) {
        for (int64_t r = 0; r < nrows; ++r)
            quant_row_legacy(type, src + start + r * n_per_row, n_per_row, imatrix, out + r * row_size);
        ops_flush();
        stat_flush();
        return (size_t)nrows * row_size;
    }
    for (int64_t r = 0; r < nrows; ++r) {
        const float *x = src + start + r * n_per_row;
        for (int64_t ib = 0; ib < nb_row; ++ib)
            quant_block(type, x + ib * bs, imatrix ? imatrix + ib * bs : NULL, out + r * row_size + ib * bb, t);
    }
    ops_flush();
    stat_flush();
    return t_err ? 0 : (size_t)nrows * row_size;
}

/* ------------------------------------------------------------------ ggml's to_float (gpuq/gpuq.hip:1850-2021) */
static inline uint8_t ksigns(uint32_t k) { return (uint8_t)(k | ((__builtin_popcount(k) & 1) << 7)); }
static inline float sgn8(uint8_t s, int j) { return (s >> j) & 1 ? -1.f : 1.f; }

static void d_iq2_xxs(const uint8_t *x, float *y, const uint64_t *g) {
    const float d = f16_to_f32(get16(x));
    for (int ib = 0; ib < 8; ++ib) {
        uint32_t a0, a1;
        memcpy(&a0, x + 2 + 8 * ib, 4);
        memcpy(&a1, x + 6 + 8 * ib, 4);
        const uint8_t *a8 = (const uint8_t *)&a0;
        const float db = d * (0.5f + (a1 >> 28)) * 0.25f;
        for (int l = 0; l < 4; ++l) {
            const uint8_t *gp = (const uint8_t *)(g + a8[l]);
            const uint8_t s = ksigns((a1 >> 7 * l) & 127);
            for (int j = 0; j < 8; ++j) y[j] = db * gp[j] * sgn8(s, j);
            y += 8;
        }
    }
}
static void d_iq2_xs(const uint8_t *x, float *y, const uint64_t *g) {
    const float d = f16_to_f32(get16(x));
    const uint8_t *sc = x + 66;
    for (int ib = 0; ib < 8; ++ib) {
        float db[2];
        db[0] = d * (0.5f + (sc[ib] & 0xf)) * 0.25f;
        db[1] = d * (0.5f + (sc[ib] >> 4)) * 0.25f;
        for (int l = 0; l < 4; ++l) {
            const uint16_t q = get16(x + 2 + 2 * (4 * ib + l));
            const uint8_t *gp = (const uint8_t *)(g + (q & 511));
            const uint8_t s = ksigns(q >> 9);
            for (int j = 0; j < 8; ++j) y[j] = db[l / 2] * gp[j] * sgn8(s, j);
            y += 8;
        }
    }
}
static void d_iq2_s(const uint8_t *x, float *y, const uint64_t *g) {
    const float d = f16_to_f32(get16(x));
    const uint8_t *qs = x + 2, *qh = x + 66, *sc = x + 74;
    const uint8_t *signs = qs + 32;
    for (int ib = 0; ib < 8; ++ib) {
        float db[2];
        db[0] = d * (0.5f + (sc[ib] & 0xf)) * 0.25f;
        db[1] = d * (0.5f + (sc[ib] >> 4)) * 0.25f;
        for (int l = 0; l < 4; ++l) {
            const float dl = db[l / 2];
            const uint8_t *gp = (const uint8_t *)(g + (qs[l] | ((qh[ib] << (8 - 2 * l)) & 0x300)));
            for (int j = 0; j < 8; ++j) y[j] = dl * gp[j] * sgn8(signs[l], j);
            y += 8;
        }
        qs += 4;
        signs += 4;
    }
}
static void d_iq3_xxs(const uint8_t *x, float *y, const uint64_t *g) {
    const float d = f16_to_f32(get16(x));
    const uint8_t *qs = x + 2, *sas = x + 2 + 64;
    for (int ib = 0; ib < 8; ++ib) {
        uint32_t a;
        memcpy(&a, sas + 4 * ib, 4);
        const float db = d * (0.5f + (a >> 28)) * 0.5f;
        for (int l = 0; l < 4; ++l) {
            const uint8_t s = ksigns((a >> 7 * l) & 127);
            const uint8_t *g1 = (const uint8_t *)(g + qs[2 * l + 0]);
            const uint8_t *g2 = (const uint8_t *)(g + qs[2 * l + 1]);
            for (int j = 0; j < 4; ++j) {
                y[j + 0] = db * g1[j] * sgn8(s, j + 0);
                y[j + 4] = db * g2[j] * sgn8(s, j + 4);
            }
            y += 8;
        }
        qs += 8;
    }
}
static void d_iq3_s(const uint8_t *x, float *y, const uint64_t *g) {
    const float d = f16_to_f32(get16(x));
    const uint8_t *qs = x + 2, *qh = x + 66, *signs = x + 74, *sc = x + 106;
    for (int ib = 0; ib < 8; ib += 2) {
        const float db1 = d * (1 + 2 * (sc[ib / 2] & 0xf));
        const float db2 = d * (1 + 2 * (sc[ib / 2] >> 4));
        for (int l = 0; l < 4; ++l) {
            const uint8_t *g1 = (const uint8_t *)(g + (qs[2 * l + 0] | ((qh[0] << (8 - 2 * l)) & 256)));
            const uint8_t *g2 = (const uint8_t *)(g + (qs[2 * l + 1] | ((qh[0] << (7 - 2 * l)) & 256)));
            for (int j = 0; j < 4; ++j) {
                y[j + 0] = db1 * g1[j] * sgn8(signs[l], j + 0);
                y[j + 4] = db1 * g2[j] * sgn8(signs[l], j + 4);
            }
            y += 8;
        }
        qs += 8;
        signs += 4;
        for (int l = 0; l < 4; ++l) {
            const uint8_t *g1 = (const uint8_t *)(g + (qs[2 * l + 0] | ((qh[1] << (8 - 2 * l)) & 256)));
            const uint8_t *g2 = (const uint8_t *)(g + (qs[2 * l + 1] | ((qh[1] << (7 - 2 * l)) & 256)));
            for (int j = 0; j < 4; ++j) {
                y[j + 0] = db2 * g1[j] * sgn8(signs[l], j + 0);
                y[j + 4] = db2 * g2[j] * sgn8(signs[l], j + 4);
            }
            y += 8;
        }
        qh += 2;
        qs += 8;
        signs += 4;
    }
}
static void d_iq1_s(const uint8_t *x, float *y, const uint64_t *g) {
    const float d = f16_to_f32(get16(x));
    const uint8_t *qs = x + 2;
    for (int ib = 0; ib < 8; ++ib) {
        const uint16_t qh = get16(x + 34 + 2 * ib);
        const float dl = d * (2 * ((qh >> 12) & 7) + 1);
        const float delta = qh & 0x8000 ? -DELTA_IQ1 : DELTA_IQ1;
        for (int l = 0; l < 4; ++l) {
            const int8_t *gp = (const int8_t *)(g + (qs[l] | (((qh >> 3 * l) & 7) << 8)));
            for (int j = 0; j < 8; ++j) y[j] = dl * (gp[j] + delta);
            y += 8;
        }
        qs += 4;
    }
}
static void d_iq1_m(const uint8_t *x, float *y, const uint64_t *g) {
    const uint8_t *qs = x, *qh = x + 32, *scb = x + 48;
    uint16_t sc[4];
    for (int i = 0; i < 4; ++i) sc[i] = get16(scb + 2 * i);
    const uint16_t scale = (uint16_t)((sc[0] >> 12) | ((sc[1] >> 8) & 0x00f0) | ((sc[2] >> 4) & 0x0f00) | (sc[3] & 0xf000));
    const float d = f16_to_f32(scale);
    for (int ib = 0; ib < 8; ++ib) {
        const float dl1 = d * (2 * ((sc[ib / 2] >> (6 * (ib % 2) + 0)) & 0x7) + 1);
        const float dl2 = d * (2 * ((sc[ib / 2] >> (6 * (ib % 2) + 3)) & 0x7) + 1);
        uint16_t idx[4];
        float delta[4];
        idx[0] = (uint16_t)(qs[0] | ((qh[0] << 8) & 0x700));
        idx[1] = (uint16_t)(qs[1] | ((qh[0] << 4) & 0x700));
        idx[2] = (uint16_t)(qs[2] | ((qh[1] << 8) & 0x700));
        idx[3] = (uint16_t)(qs[3] | ((qh[1] << 4) & 0x700));
        delta[0] = qh[0] & 0x08 ? -DELTA_IQ1 : DELTA_IQ1;
        delta[1] = qh[0] & 0x80 ? -DELTA_IQ1 : DELTA_IQ1;
        delta[2] = qh[1] & 0x08 ? -DELTA_IQ1 : DELTA_IQ1;
        delta[3] = qh[1] & 0x80 ? -DELTA_IQ1 : DELTA_IQ1;
        for (int l = 0; l < 2; ++l) {
            const int8_t *gp = (const int8_t *)(g + idx[l]);
            for (int j = 0; j < 8; ++j) y[j] = dl1 * (gp[j] + delta[l]);
            y += 8;
        }
        for (int l = 2; l < 4; ++l) {
            const int8_t *gp = (const int8_t *)(g + idx[l]);
            for (int j = 0; j < 8; ++j) y[j] = dl2 * (gp[j] + delta[l]);
            y += 8;
        }
        qs += 4;
        qh += 2;
    }
}
static void d_iq4_xs(const uint8_t *x, float *y) {
    const float d = f16_to_f32(get16(x));
    const uint16_t sh = get16(x + 2);
    const uint8_t *sl = x + 4, *qs = x + 8;
    for (int ib = 0; ib < 8; ++ib) {
        const int ls = ((sl[ib / 2] >> 4 * (ib % 2)) & 0xf) | (((sh >> 2 * ib) & 3) << 4);
        const float dl = d * (ls - 32);
        for (int j = 0; j < 16; ++j) {
            y[j + 0] = dl * k_iq4nl[qs[j] & 0xf];
            y[j + 16] = dl * k_iq4nl[qs[j] >> 4];
        }
        y += 32;
        qs += 16;
    }
}

/* ggml's to_float of the k-quants (ggml-quants.c dequantize_row_q2_K .. q6_K, which the reference calls through
 * libggml-base for its LDLQ loop, tools/requant_experts.py:588-591), in ggml's loop order over the block layouts the
 * quantizers above write: y = d * sc * q - dmin * m, every product and difference rounded as written. */
static void d_q2_k(const uint8_t *x, float *y) {
    const float d = f16_to_f32(get16(x + 80)), dmin = f16_to_f32(get16(x + 82));
    const uint8_t *q = x + 16;
    int is = 0;
    for (int n = 0; n < QK; n += 128) {
        for (int shift = 0; shift < 8; shift += 2) {
            for (int h = 0; h < 2; ++h) {
                const uint8_t sc = x[is++];
                const float dl = d * (sc & 0xF), ml = dmin * (sc >> 4);
                for (int l = 0; l < 16; ++l) *y++ = dl * (int8_t)((q[l + 16 * h] >> shift) & 3) - ml;
            }
        }
        q += 32;
    }
}
static void d_q3_k(const uint8_t *x, float *y) {
    const uint8_t *hm = x, *q = x + 32, *s = x + 96;
    const float d = f16_to_f32(get16(x + 108));
    int8_t sc[16];   /* the 16 6-bit scales: low 4 bits from nibbles of s[0..7], high 2 bits from s[8..11] */
    for (int i = 0; i < 16; ++i) {
        const int lo = i < 8 ? (s[i] & 0xF) : (s[i - 8] >> 4);
        sc[i] = (int8_t)(lo | (((s[8 + i % 4] >> (2 * (i / 4))) & 3) << 4));
    }
    int is = 0;
    uint8_t m = 1;
    for (int n = 0; n < QK; n += 128) {
        for (int shift = 0; shift < 8; shift += 2) {
            for (int h = 0; h < 2; ++h) {
                const float dl = d * (sc[is++] - 32);
                for (int l = 0; l < 16; ++l)
                    *y++ = dl * ((int8_t)((q[l + 16 * h] >> shift) & 3) - ((hm[l + 16 * h] & m) ? 0 : 4));
            }
            m <<= 1;
        }
        q += 32;
    }
}
static void d_q45_k(const uint8_t *x, float *y, int five) {
    const float d = f16_to_f32(get16(x)), dmin = f16_to_f32(get16(x + 2));
    const uint8_t *s = x + 4, *qh = x + 16, *ql = x + (five ? 48 : 16);
    uint8_t u1 = 1, u2 = 2;
    for (int j = 0, is = 0; j < QK; j += 64, is += 2) {
        uint8_t sc, m;
        k4_unpack(is, s, &sc, &m);
        const float d1 = d * sc, m1 = dmin * m;
        k4_unpack(is + 1, s, &sc, &m);
        const float d2 = d * sc, m2 = dmin * m;
        for (int l = 0; l < 32; ++l) *y++ = d1 * ((ql[l] & 0xF) + (five && (qh[l] & u1) ? 16 : 0)) - m1;
        for (int l = 0; l < 32; ++l) *y++ = d2 * ((ql[l] >> 4) + (five && (qh[l] & u2) ? 16 : 0)) - m2;
        ql += 32;
        u1 <<= 2;
        u2 <<= 2;
    }
}
static void d_q6_k(const uint8_t *x, float *y) {
    const float d = f16_to_f32(get16(x + 208));
    const uint8_t *ql = x, *qh = x + 128;
    const int8_t *sc = (const int8_t *)(x + 192);
    for (int n = 0; n < QK; n += 128) {
        for (int l = 0; l < 32; ++l) {
            const int is = l / 16;
            const int8_t q1 = (int8_t)((ql[l] & 0xF) | (((qh[l] >> 0) & 3) << 4)) - 32;
            const int8_t q2 = (int8_t)((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
            const int8_t q3 = (int8_t)((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
            const int8_t q4 = (int8_t)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
            y[l] = d * sc[is + 0] * q1;
            y[l + 32] = d * sc[is + 2] * q2;
            y[l + 64] = d * sc[is + 4] * q3;
            y[l + 96] = d * sc[is + 6] * q4;
        }
        y += 128;
        ql += 64;
        qh += 32;
        sc += 8;
    }
}

size_t gqo_dequantize(int type, const void *src, float *dst, int64_t n) {
    const uint8_t *x = (const uint8_t *)src;
    const size_t bb = gqo_block_bytes(type);
    const int bs = gqo_block_len(type);
    if (!bb || n < 0 || n % bs) return 0;
    const int64_t nb = n / bs;
    if (type == GQO_IQ4_XS || (type >= GQO_Q2_K && type <= GQO_Q6_K)) {
        for (int64_t b = 0; b < nb; ++b) {
            const uint8_t *xb = x + b * bb;
            float *y = dst + b * QK;
            switch (type) {
                case GQO_IQ4_XS: d_iq4_xs(xb, y); break;
                case GQO_Q2_K: d_q2_k(xb, y); break;
                case GQO_Q3_K: d_q3_k(xb, y); break;
                case GQO_Q4_K: d_q45_k(xb, y, 0); break;
                case GQO_Q5_K: d_q45_k(xb, y, 1); break;
                default: d_q6_k(xb, y); break;
            }
        }
        return (size_t)n * 4;
    }
    if (type == GQO_Q8_0) return gqo_decode_src(GQO_Q8_0, src, dst, n);
    const otab *t = tab_dq(type);
    if (!t) return 0;
    for (int64_t b = 0; b < nb; ++b) {
        const uint8_t *xb = x + b * bb;
        float *y = dst + b * QK;
        switch (type) {
            case GQO_IQ2_XXS: d_iq2_xxs(xb, y, t->grid); break;
            case GQO_IQ2_XS: d_iq2_xs(xb, y, t->grid); break;
            case GQO_IQ2_S: d_iq2_s(xb, y, t->grid); break;
            case GQO_IQ3_XXS: d_iq3_xxs(xb, y, t->grid); break;
            case GQO_IQ3_S: d_iq3_s(xb, y, t->grid); break;
            case GQO_IQ1_S: d_iq1_s(xb, y, t->grid); break;
            case GQO_IQ1_M: d_iq1_m(xb, y, t->grid); break;
            default: return 0;
        }
    }
    return (size_t)n * 4;
}

/* ------------------------------------------------------------------ source decode (gpuq/gpuq.hip:2123-2154) */
size_t gqo_src_bytes(int src, int64_t n) {
    switch (src) {
        case GQO_F32: return (size_t)n * 4;
        case GQO_F16: case GQO_BF16: return (size_t)n * 2;
        case GQO_Q8_0: return (size_t)(n / 32) * 34;
        case GQO_MXFP4: return (size_t)(n / 32) * 17;
        default: return 0;
    }
}

size_t gqo_decode_src(int src, const void *raw, float *y, int64_t n) {
    static const int8_t kv[16] = {0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12};
    if (!gqo_src_bytes(src, 32) || n < 0 || n % 32) return 0;
    const uint8_t *in = (const uint8_t *)raw;
    for (int64_t b = 0; b < n / 32; ++b) {
        float *o = y + b * 32;
        switch (src) {
            case GQO_F32: memcpy(o, in + b * 128, 128); break;
            case GQO_F16: for (int j = 0; j < 32; ++j) o[j] = f16_to_f32(get16(in + b * 64 + 2 * j)); break;
            case GQO_BF16: for (int j = 0; j < 32; ++j) o[j] = float_of((uint32_t)get16(in + b * 64 + 2 * j) << 16); break;
            case GQO_Q8_0: {
                const uint8_t *x = in + b * 34;
                const float d = f16_to_f32(get16(x));
                for (int j = 0; j < 32; ++j) o[j] = (int8_t)x[2 + j] * d;
                break;
            }
            case GQO_MXFP4: {
                const uint8_t *x = in + b * 17;
                const float d = e8m0_half(x[0]);
                for (int j = 0; j < 16; ++j) { o[j] = kv[x[1 + j] & 0x0f] * d; o[j + 16] = kv[x[1 + j] >> 4] * d; }
                break;
            }
        }
    }
    return (size_t)n * 4;
}

/* ------------------------------------------------------------------ the all-core CPU baseline */
typedef struct {
    int src_type, type;
    const uint8_t *raw;
    uint8_t *dst;
    int64_t nmat, nrow, n_per_row, unit_rows, nunits;
    const float *imatrix;
    int64_t next;
    int failed;
    pthread_mutex_t mu;
} mt_job;

static void *mt_worker(void *arg) {
    mt_job *j = (mt_job *)arg;
    const size_t row_out = (size_t)(j->n_per_row / gqo_block_len(j->type)) * gqo_block_bytes(j->type);
    const size_t row_in = gqo_src_bytes(j->src_type, j->n_per_row);
    const int64_t units_per_mat = (j->nrow + j->unit_rows - 1) / j->unit_rows;
    float *buf = malloc((size_t)j->unit_rows * j->n_per_row * 4);
    for (;;) {
        pthread_mutex_lock(&j->mu);
        const int64_t u = j->next++;
        pthread_mutex_unlock(&j->mu);
        if (u >= j->nunits) break;
        const int64_t m = u / units_per_mat, r0 = (u % units_per_mat) * j->unit_rows;
        const int64_t nr = r0 + j->unit_rows <= j->nrow ? j->unit_rows : j->nrow - r0;
        const int64_t row = m * j->nrow + r0;
        gqo_decode_src(j->src_type, j->raw + row * row_in, buf, nr * j->n_per_row);
        const size_t got = gqo_quantize_chunk(j->type, buf, j->dst + row * row_out, 0, nr, j->n_per_row,
                                              j->imatrix ? j->imatrix + m * j->n_per_row : NULL);
        if (got != (size_t)nr * row_out) j->failed = 1;
    }
    free(buf);
    ops_flush();
    stat_flush();
    return NULL;
}

size_t gqo_requantize_batch_mt(int src_type, const void *raw, int type, void *dst, int64_t nmat, int64_t nrow,
                               int64_t n_per_row, const float *imatrix, int64_t unit_rows, int nthreads) {
    if (!gqo_block_bytes(type) || !gqo_src_bytes(src_type, 32) || nmat <= 0 || nrow <= 0 || unit_rows <= 0 ||
        n_per_row % 32 || nthreads <= 0)
        return 0;
    mt_job j = {src_type, type, (const uint8_t *)raw, (uint8_t *)dst, nmat, nrow, n_per_row, unit_rows,
                nmat * ((nrow + unit_rows - 1) / unit_rows), imatrix, 0, 0, PTHREAD_MUTEX_INITIALIZER};
    pthread_t th[256];
    if (nthreads > 256) nthreads = 256;
    for (int i = 0; i < nthreads; ++i) pthread_create(&th[i], NULL, mt_worker, &j);
    for (int i = 0; i < nthreads; ++i) pthread_join(th[i], NULL);
    if (j.failed) return 0;
    return (size_t)nmat * nrow * (n_per_row / gqo_block_len(type)) * gqo_block_bytes(type);
}

/* ------------------------------------------------------------------ LDLQ with a fixed summation order
 * The loop of tools/ldlq.py:71-107 (quantize_matrix) / 391-431 (quantize_matrix_torch): quantize permuted block k,
 * dequantize it, E = blk - q (f32), then Es = E U_BB^-1 by forward substitution over the block's columns and
 * Wp[:, rest] -= (float)(Es U_B,rest). The summation order is fixed (the reference leaves it to LAPACK / BLAS):
 *   Es[r][j] = fma(-Es[r][i], U[c0+i][c0+j], ...) for i = 0..j-1 in order, starting from (double)E[r][j], then
 *              divided by U[c0+j][c0+j];
 *   acc[r][c] = fma(Es[r][i], U[c0+i][c], acc) for i = 0..255 in order, starting from 0.0;
 *   Wp[r][c] = Wp[r][c] - (float)acc[r][c].
 */
size_t gqo_ldlq(int type, float *Wp, const double *U, const float *qw, int64_t nmat, int64_t ne1, int64_t ne0,
                const int64_t *blk_order, int feedback, void *out) {
    const size_t bb = gqo_block_bytes(type);
    if (!bb || gqo_block_len(type) != QK || ne0 % QK || nmat <= 0 || ne1 <= 0) return 0;
    const int64_t nblk = ne0 / QK;
    uint8_t *raw = malloc((size_t)ne1 * bb);
    float *q = malloc((size_t)ne1 * QK * 4);
    float *blk = malloc((size_t)ne1 * QK * 4);
    double *Es = malloc((size_t)QK * 8);
    size_t ok = 1;
    for (int64_t m = 0; m < nmat && ok; ++m) {
        float *W = Wp + m * ne1 * ne0;
        uint8_t *o = (uint8_t *)out + m * ne1 * nblk * bb;
        for (int64_t k = 0; k < nblk && ok; ++k) {
            const int64_t c0 = k * QK;
            for (int64_t r = 0; r < ne1; ++r) memcpy(blk + r * QK, W + r * ne0 + c0, QK * 4);
            if (gqo_quantize_chunk(type, blk, raw, 0, ne1, QK, qw + m * ne0 + c0) != (size_t)ne1 * bb) { ok = 0; break; }
            for (int64_t r = 0; r < ne1; ++r) memcpy(o + (r * nblk + blk_order[k]) * bb, raw + r * bb, bb);
            if (!feedback || k + 1 >= nblk) continue;
            if (gqo_dequantize(type, raw, q, ne1 * QK) != (size_t)ne1 * QK * 4) { ok = 0; break; }
            for (int64_t r = 0; r < ne1; ++r) {
                for (int j = 0; j < QK; ++j) {
                    double acc = (double)(blk[r * QK + j] - q[r * QK + j]);
                    for (int i = 0; i < j; ++i) acc = fma(-Es[i], U[(c0 + i) * ne0 + c0 + j], acc);
                    Es[j] = acc / U[(c0 + j) * ne0 + c0 + j];
                }
                float *wr = W + r * ne0;
                for (int64_t c = c0 + QK; c < ne0; ++c) {
                    double acc = 0.0;
                    for (int i = 0; i < QK; ++i) acc = fma(Es[i], U[(c0 + i) * ne0 + c], acc);
                    wr[c] = wr[c] - (float)acc;
                }
            }
        }
    }
    free(raw); free(q); free(blk); free(Es);
    return ok ? (size_t)nmat * ne1 * nblk * bb : 0;
}

/* ------------------------------------------------------------------ the 'schur' importance, fixed order
 * tools/ldlq.py:90-93: qw = diag((U_BB^T U_BB)^-1) for each 256-column diagonal block U_BB of the factor (there
 * np.linalg.inv). (U_BB^T U_BB)^-1 = X X^T with X = U_BB^-1, so qw[i] is the squared norm of X's row i, which comes
 * from X U_BB = I by substitution along the row: x_t = ((t == i) - sum_{s=i}^{t-1} x_s U[s][t]) / U[t][t], each sum an
 * fma chain over s ascending from 0.0, and qw[i] = (float)(sum_t x_t^2), an fma chain over t ascending from 0.0. */
void gqo_schur_weights(const double *U, int64_t ne0, float *w) {
    double acc[QK];
    for (int64_t c0 = 0; c0 + QK <= ne0; c0 += QK) {
        for (int i = 0; i < QK; ++i) {
            for (int j = 0; j < QK; ++j) acc[j] = 0.0;
            double ws = 0.0;
            for (int t = i; t < QK; ++t) {
                const double x = ((t == i ? 1.0 : 0.0) - acc[t]) / U[(c0 + t) * ne0 + c0 + t];
                ws = fma(x, x, ws);
                for (int j = t + 1; j < QK; ++j) acc[j] = fma(x, U[(c0 + t) * ne0 + c0 + j], acc[j]);
            }
            w[c0 + i] = (float)ws;
        }
    }
}
