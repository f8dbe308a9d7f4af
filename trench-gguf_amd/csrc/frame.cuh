// trench-gguf_amd/csrc/frame.cuh - the launch frame shared by the super-block quantizers.
//
// Work decomposition (gfx950, wave64): a super-block of 256 weights is owned by G consecutive lanes (G = 8 for the
// 32-weight sub-block types, 16 for the 16-weight ones), lane g holding sub-block g's weights, importances and
// search state in registers. The per-sub-block searches of ggml run on their lane in ggml's own serial order, so no
// cross-lane arithmetic reorders a sum; the few super-block-wide quantities are lane-to-lane chains (sums) or
// order-free reductions (max). A wave therefore quantizes 64/G super-blocks at once, with 100% lane occupancy in the
// fixed-trip-count search loops. Each wave assembles its super-blocks' output bytes in an LDS image and writes them
// to HBM as one contiguous, dword-coalesced range. For the types with neighbour searches (tiles of varying cost) the
// launch holds as many workgroups as the CUs keep resident, and each wave takes its tiles (64/G super-blocks) one at
// a time from a counter: the waves sweep the tensor once, in order (an expert's importance row is read while the
// whole chip works on that expert), every wave busy until the counter runs past the end. The other types loop over
// the tiles grid-stride. The per-workgroup LDS table staging of the i-quants is paid once per workgroup.
#pragma once
#include "common.cuh"

#define WG_THREADS 256
#define WG_WAVES 4

struct QParams {
    const uint8_t *src;     // source tensor bytes (type SRC), super-block b at element b*QK
    const float *qw;        // importance rows or nullptr
    int64_t qw_mat, qw_mod, qw_div;   // block b reads row (b / qw_mat) * qw_mod + (b % qw_mod) / qw_div
    uint8_t *dst;           // output blocks
    int64_t nsb;            // units: super-blocks, or 32-blocks for Q8_0 / IQ4_NL
    // i-quant tables (device): search grid, full 2-bit / 3-bit key map, ggml-layout neighbour lists, and for the
    // 8-value types the map re-indexed by base-3 keys (levels 0..2, off-grid entries packed as below), staged into
    // LDS by the kernels
    const uint64_t *grid;
    const int32_t *map;
    const uint16_t *neigh;
    const uint32_t *npt;    // the 4-value types: neigh's entries as grid points (same offsets; counts read 0)
    const int32_t *map3;
    int grid_size, map_size, neigh_len;
    int *err;               // set when a search finds no candidate (the reference traps there)
    // the launch's tile counter (zeroed on the stream before the launch): after its first chunk of tiles (its wave
    // number) each wave takes the next from it (grid waves + the counter's old value), so the resident waves sweep
    // the tensor once, in order, and finish together; nullptr: a fixed grid-stride order
    unsigned long long *tiles;
    // strided views (the LDLQ loop quantizes one block column of every row): unit b reads its weights at element
    // b*sb_stride + sb_off, its importance at row*qw_stride + qw_off, and writes its block at byte
    // b*out_stride + out_off. The contiguous defaults are sb_stride = BS, qw_stride = BS, out_stride = BB, 0 offsets.
    int64_t sb_stride, sb_off, qw_stride, qw_off, out_stride, out_off;
    // the row-wide sigma2 of the Q4_0 / Q5_0 / Q5_1 imatrix rules (one a row: unit b is in row b / row_units)
    const float *rsig;
    int64_t row_units;
};

// map3 entries: >= 0 a grid index; < 0 an off-grid key, -1 - (list offset | list length << M3_OFF_BITS)
#define M3_OFF_BITS 21
DEV int m3_off(int m) { return (-m - 1) & ((1 << M3_OFF_BITS) - 1); }
DEV int m3_cnt(int m) { return (-m - 1) >> M3_OFF_BITS; }

DEV int64_t qw_row(const QParams &p, int64_t b) { return (b / p.qw_mat) * p.qw_mod + (b % p.qw_mod) / p.qw_div; }

template <int N> DEV void load_qw(const float *row, float (&w)[N]) {
    const float4 *p = (const float4 *)row;
#pragma unroll
    for (int i = 0; i < N / 4; ++i) {
        const float4 q = p[i];
        w[4 * i + 0] = q.x; w[4 * i + 1] = q.y; w[4 * i + 2] = q.z; w[4 * i + 3] = q.w;
    }
}

// ------------------------------------------------------------------ the LDS block image
// Bytes are combined with LDS atomic ORs on the containing dword, so fields that several lanes fill (shared high
// bits, packed nibbles) need no ordering between lanes. The image is zeroed before every tile. `img` is the wave's
// 16-byte aligned image and `off` a byte offset in it (a block's fields sit at blk_off + field offset).
DEV void img_or8(uint8_t *img, int off, uint32_t v) {
    atomicOr((unsigned int *)(img + (off & ~3)), (v & 0xffu) << (8 * (off & 3)));
}
DEV void img_or16(uint8_t *img, int off, uint32_t v) {   // off even
    atomicOr((unsigned int *)(img + (off & ~3)), (v & 0xffffu) << (8 * (off & 3)));
}
DEV void img_or32(uint8_t *img, int off, uint32_t v) {   // off even
    if ((off & 3) == 0) atomicOr((unsigned int *)(img + off), v);
    else { img_or16(img, off, v & 0xffffu); img_or16(img, off + 2, v >> 16); }
}

DEV void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
}

DEV void img_zero(uint8_t *img, int nbytes) {
    for (int i = lane_id() * 4; i < nbytes; i += 64 * 4) *(uint32_t *)(img + i) = 0u;
}

typedef unsigned int v4u32 __attribute__((ext_vector_type(4)));

// copy nbytes (even) of the image to global dst (2-byte aligned) with coalesced stores: 16 bytes a lane when dst and
// nbytes allow it, else dwords. NT: nontemporal stores (the Q8_0 stream, whose tiles are whole 16-byte runs; for
// tiles that end inside a cache line they raise the written bytes, the L2 no longer merging neighbouring tiles).
template <bool NT = false> DEV void img_store(uint8_t *dst, const uint8_t *img, int nbytes) {
    const int lane = lane_id();
    if ((((uintptr_t)dst) & 15) == 0 && (nbytes & 15) == 0) {
        for (int i = lane; i < nbytes / 16; i += 64) {
            const v4u32 v = *(const v4u32 *)(img + 16 * i);
            if (NT) __builtin_nontemporal_store(v, (v4u32 *)(dst + 16 * i));
            else *(v4u32 *)(dst + 16 * i) = v;
        }
        return;
    }
    int head = ((uintptr_t)dst & 3) ? 2 : 0;            // dst is at least 2-byte aligned
    if (head > nbytes) head = nbytes;
    if (head && lane == 0) *(uint16_t *)dst = *(const uint16_t *)img;
    const int nw = (nbytes - head) / 4;
    for (int i = lane; i < nw; i += 64) {
        const uint8_t *s = img + head + 4 * i;
        uint32_t v;
        if (head) v = (uint32_t)*(const uint16_t *)s | ((uint32_t)*(const uint16_t *)(s + 2) << 16);
        else v = *(const uint32_t *)s;
        if (NT) __builtin_nontemporal_store(v, (uint32_t *)(dst + head + 4 * i));
        else *(uint32_t *)(dst + head + 4 * i) = v;
    }
    const int tail = nbytes - head - 4 * nw;             // 0 or 2
    if (tail && lane == 0) *(uint16_t *)(dst + nbytes - 2) = *(const uint16_t *)(img + nbytes - 2);
}

// ------------------------------------------------------------------ the tile queue
// lane 0's 64-bit value on every lane (wave-uniform)
DEV int64_t wave_u64(unsigned long long v) {
    const unsigned lo = __builtin_amdgcn_readfirstlane((unsigned)v);
    const unsigned hi = __builtin_amdgcn_readfirstlane((unsigned)(v >> 32));
    return (int64_t)(((unsigned long long)hi << 32) | lo);
}

// ------------------------------------------------------------------ the kernel
// T provides: BS (weights a unit: 256, or 32 for Q8_0 / IQ4_NL), G (lanes a unit), N (= BS / G), BB (unit bytes),
// TAB (LDS table bytes, 0 for none),
// stage(p, lds) (cooperative table staging, before the barrier), and
// quant(x, qw, g, img, boff, lds, p): lane g's part of one super-block, OR-ing its bytes into img at boff.
// WS (optional, bytes, multiple of 16): a per-wave LDS workspace placed right after the wave's image
template <class T> constexpr int img_bytes() { return ((64 / T::G) * T::BB + 15) & ~15; }
template <class T, class = void> struct ws_of { static constexpr int v = 0; };
template <class T> struct ws_of<T, decltype((void)T::WS)> { static constexpr int v = T::WS; };
template <class T> constexpr int wave_bytes() { return img_bytes<T>() + ws_of<T>::v; }
template <class T> DEV uint8_t *wave_ws(uint8_t *img) { return img + img_bytes<T>(); }
// WGW (optional): waves a workgroup (default WG_WAVES), for types whose per-wave LDS would not let two workgroups
// share a CU's LDS: one workgroup of twice the waves shares one copy of the tables
template <class T, class = void> struct wgw_of { static constexpr int v = WG_WAVES; };
template <class T> struct wgw_of<T, decltype((void)T::WGW)> { static constexpr int v = T::WGW; };
// QUEUE (optional): tiles from the launch's counter (types whose tiles vary in cost: the neighbour searches), one
// resident grid; without it a grid-stride order over up to 32 waves a CU (tiles of equal cost)
template <class T, class = void> struct queue_of { static constexpr bool v = false; };
template <class T> struct queue_of<T, decltype((void)T::QUEUE)> { static constexpr bool v = T::QUEUE; };
// ROWSIG (optional): quant_rs takes the unit's row-wide sigma2 (p.rsig) after its importance row
template <class T, class = void> struct rowsig_of { static constexpr bool v = false; };
template <class T> struct rowsig_of<T, decltype((void)T::ROWSIG)> { static constexpr bool v = T::ROWSIG; };
// WPE (optional): the waves per SIMD the register allocation must allow (default 2)
template <class T, class = void> struct wpe_of { static constexpr int v = 2; };
template <class T> struct wpe_of<T, decltype((void)T::WPE)> { static constexpr int v = T::WPE; };

template <class T, int SRC>
__global__ __launch_bounds__(64 * wgw_of<T>::v) __attribute__((amdgpu_waves_per_eu(wpe_of<T>::v))) void k_quant(
    QParams p) {
    extern __shared__ __align__(16) uint8_t lds[];
    constexpr int SPW = 64 / T::G, WGW = wgw_of<T>::v;
    if (T::TAB) {
        T::stage(p, lds);
        __syncthreads();
    }
    const int wave = (int)(threadIdx.x >> 6), lane = lane_id();
    const int g = lane % T::G, slot = lane / T::G;
    uint8_t *img = lds + T::TAB + wave * wave_bytes<T>();
    const int64_t nwaves = (int64_t)gridDim.x * WGW;
    const bool queue = queue_of<T>::v && p.tiles != nullptr;       // (compile-time false for the other types)
    // queued tiles come in chunks of KT whose source bytes start and end on 128-byte lines (the 17-byte MXFP4 and
    // 34-byte Q8_0 blocks), so that no line is fetched by two waves of different XCDs
    constexpr int KT = !queue_of<T>::v ? 1 : SRC == T_MXFP4 ? (SPW >= 16 ? 1 : 16 / SPW)
                                           : SRC == T_Q8_0 ? (SPW >= 8 ? 1 : 8 / SPW) : 1;
    int64_t c = (int64_t)blockIdx.x * WGW + wave;        // (the first chunks in wave order: no burst on the counter)
    int k = 0;                                           // the tile in the chunk
    int64_t t = c * KT;
    unsigned long long tn = 0;
    while (t * SPW < p.nsb) {
        const int64_t b0 = t * SPW;
        const int nact = (int)(p.nsb - b0 < SPW ? p.nsb - b0 : SPW);
        const int64_t b = b0 + (slot < nact ? slot : nact - 1);
        img_zero(img, img_bytes<T>());
        wave_sync();
        float x[T::N];
        SrcLoad<SRC, T::N>::load(p.src, b * p.sb_stride + p.sb_off + g * T::N, x);
        // the next chunk, asked for at a chunk's first tile (lane 0's atomic returns while the chunk is quantized)
        if (queue && k == 0 && lane == 0) tn = atomicAdd(p.tiles, 1ull);
        const float *qw = p.qw ? p.qw + qw_row(p, b) * p.qw_stride + p.qw_off + g * T::N : nullptr;
        if constexpr (rowsig_of<T>::v)
            T::quant_rs(x, qw, qw ? p.rsig[b / p.row_units] : 0.f, g, img, slot * T::BB, lds, p);
        else
            T::quant(x, qw, g, img, slot * T::BB, lds, p);
        wave_sync();
        if (p.out_stride == T::BB && p.out_off == 0) {
            img_store(p.dst + b0 * T::BB, img, nact * T::BB);
        } else if (slot < nact) {         // strided: each group copies its own block, 16 bits a lane
            uint16_t *o = (uint16_t *)(p.dst + b * p.out_stride + p.out_off);
            const uint16_t *s = (const uint16_t *)(img + slot * T::BB);
            for (int h = g; h < T::BB / 2; h += T::G) o[h] = s[h];
        }
        wave_sync();
        if (++k == KT) {
            c = queue ? nwaves + wave_u64(tn) : c + nwaves;
            k = 0;
        }
        t = c * KT + k;
    }
}
