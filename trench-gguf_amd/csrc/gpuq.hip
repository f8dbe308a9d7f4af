// trench-gguf_amd/csrc/gpuq.hip - libgpuq.so: the GGUF quantizer for MI355X (gfx950), C ABI.
//
// Build: hipcc -O3 -ffp-contract=off -fno-fast-math --offload-arch=gfx950 -fPIC -shared (see the package Makefile).
// The exported functions keep the reference library's signatures, return conventions and table file format
// (gpuq/gpuq.hip:2059-2328 of the reference), so its Python drivers load this library unchanged; they are declared
// with their reference counterparts in include/gpuq.h.
#include <dlfcn.h>
#include <hip/hip_runtime.h>
#include <rocblas/rocblas.h>
#include <rocsolver/rocsolver.h>

#include <cstdio>
#include <cstring>
#include <algorithm>
#include <cstdlib>
#include <atomic>
#include <mutex>
#include <thread>
#include <unordered_map>
#include <vector>

#include "common.cuh"
#include "frame.cuh"
#include "kquants.cuh"
#include "legacy.cuh"
#include "iq2.cuh"
#include "iq1.cuh"
#include "iq3.cuh"
#include "dequant.cuh"
#include "ldlq.cuh"
#include "hessian.cuh"

extern "C" size_t gpuq_block_bytes(int type);

// The Es scratch of gpuq_ldlq_dev_noalloc, the entry point that allocates nothing: two blocks of Es (2 x 256 doubles
// a row) for up to LDLQ_SCRATCH_ROWS rows (nmat * ne1), 32 MiB, held by every device the library runs on for the
// life of the process. Host code never passes this name to a kernel or a copy (on the host it is only a stand-in):
// gpuq_init takes each device's address of it with hipGetSymbolAddress, once per device, into g_scratch.
static constexpr int64_t LDLQ_SCRATCH_ROWS = 8192;
static __device__ __align__(256) double scratch[2 * LDLQ_SCRATCH_ROWS * 256];

// The quantize launches' tile counters (the tile queue of k_quant), zeroed by a kernel on the launch's stream before
// the quantize kernel. Eager launches cycle through the first TILE_EAGER slots, so launches in flight at once on any
// streams use distinct counters while there are at most TILE_EAGER of them. A launch recorded under stream capture
// keeps its slot in the graph for good, so each takes one of the other TILE_SLOTS - TILE_EAGER slots, never handed
// out again (eager launches cannot alias a graph's counter; once they are used up a captured launch fails). Addresses
// taken per device at gpuq_init, as for `scratch`.
static constexpr unsigned TILE_SLOTS = 16384, TILE_EAGER = 4096;
static __device__ __align__(256) unsigned long long tile_ctr[TILE_SLOTS];

__global__ void k_tile_reset(unsigned long long *ctr) {
    if (threadIdx.x == 0) *ctr = 0ull;
}

namespace {

double *g_scratch[64] = {};    // per device: the device address of `scratch`
unsigned long long *g_tile_ctr[64] = {};   // per device: the device address of `tile_ctr`
std::atomic<unsigned> g_tile_slot{0};      // eager launches: the next slot (mod TILE_EAGER)
std::atomic<unsigned> g_tile_graph{0};     // captured launches: slots TILE_EAGER + n taken so far

struct Tabs {
    bool ok = false;
    uint64_t *grid = nullptr;   // search grid
    int32_t *map = nullptr;     // full key map (2-bit keys, 43692; 3-bit keys, 4096)
    int32_t *map3 = nullptr;    // the staged map, off-grid entries packed: base-3 keys (6561) or 3-bit keys (4096)
    uint16_t *neigh = nullptr;
    uint32_t *npt = nullptr;    // the 4-value types: each list entry's grid point, beside neigh (same offsets)
    int grid_size = 0, map_size = 0, neigh_len = 0;
    uint64_t *dq = nullptr;     // dequantizer grid (record 1000 + type)
    int dq_size = 0;
};

Tabs g_tabs[64];
std::vector<void *> g_retired;  // device tables replaced by a later gpuq_init (never freed: see gpuq_init)
// the record type that marks a table file holding stand-in codebooks instead of ggml's (the build's own generator
// writes it; a file written from ggml by the reference's gpuq_tables.c has none)
constexpr int SYNTHETIC_MARK = 0x53594e54;
int g_device = -1;
int g_ncu = 256;
int *g_err = nullptr;          // device flag: a search found no candidate (the reference traps there)
std::mutex g_mu;               // the host API's staging buffers are process-global

struct Buf {
    void *p = nullptr;
    size_t cap = 0;
    bool grow(size_t need) {
        if (need <= cap) return true;
        if (p) (void)hipFree(p);
        p = nullptr;
        cap = 0;
        if (hipMalloc(&p, need) != hipSuccess) return false;
        cap = need;
        return true;
    }
};
Buf g_qw, g_es;

bool is_search_type(int t) {
    return t == T_IQ2_XXS || t == T_IQ2_XS || t == T_IQ2_S || t == T_IQ1_S || t == T_IQ3_XXS || t == T_IQ3_S;
}
int expected_grid(int t) {
    switch (t) {
        case T_IQ2_XXS: return 256;
        case T_IQ2_XS: return 512;
        case T_IQ2_S: return 1024;
        case T_IQ1_S: return 2048;
        case T_IQ3_XXS: return 256;
        case T_IQ3_S: return 512;
        default: return 0;
    }
}
bool eight_values(int t) { return t != T_IQ3_XXS && t != T_IQ3_S; }

// search tables of a type: IQ1_M searches IQ1_S's (gpuq/gpuq.hip:2051-2056)
const Tabs &tab_of(int type) { return g_tabs[type == T_IQ1_M ? T_IQ1_S : type]; }

// The checks that make the LDS layout exact: every point's key is in the map and maps back to the point, and every
// key the trial rounding can produce is on the grid or has a non-empty, in-range neighbour list.
bool valid_search(int t, const std::vector<uint64_t> &grid, const std::vector<int32_t> &map,
                  const std::vector<uint16_t> &neigh) {
    const bool e8 = eight_values(t);
    const int nv = e8 ? 8 : 4, bits = e8 ? 2 : 3, maxlev = e8 ? 3 : 7;
    if ((int)grid.size() != expected_grid(t) || (int)map.size() != (e8 ? 43692 : 4096)) return false;
    const int G = (int)grid.size(), M = (int)map.size(), NL = (int)neigh.size();
    for (int g = 0; g < G; ++g) {
        int u = 0;
        for (int i = 0; i < nv; ++i) {
            const int b = (int)((grid[g] >> (8 * i)) & 0xff);
            if (b < 1 || b > 2 * maxlev + 1 || !(b & 1)) return false;
            u |= ((b - 1) / 2) << (bits * i);
        }
        if (e8 && ((grid[g] >> 0) >> 63)) return false;
        if (!e8 && (grid[g] >> 32)) return false;
        if (u >= M || map[u] != g) return false;
    }
    const int nkeys = e8 ? 6561 : 4096;
    for (int k = 0; k < nkeys; ++k) {
        int u = k;
        if (e8) {
            u = 0;
            int r = k;
            for (int i = 0; i < 8; ++i) { u |= (r % 3) << (2 * i); r /= 3; }
        }
        const int m = map[u];
        if (m >= 0) {
            if (m >= G) return false;
            continue;
        }
        const int64_t off = -(int64_t)m - 1;
        if (off >= NL) return false;
        const int cnt = neigh[off];
        if (cnt < 1 || off + cnt >= NL) return false;
        for (int j = 1; j <= cnt; ++j)
            if (neigh[off + j] >= G) return false;
    }
    return true;
}

// The map the kernels stage and the neighbour lists they read, from a validated record: for the 8-value types the
// map re-indexed by base-3 keys (6561; the trial rounding's levels are 0..2, so no other key is ever looked up), for
// the 4-value types the 4096 3-bit keys as they are. Only the lists these keys reach are kept, in the file's layout
// (a count, then the points), each once, in key order; an off-grid entry packs the list's offset in that buffer and
// its length (m3_off / m3_cnt). False when a list's offset or length does not fit the packing (M3_OFF_BITS).
bool pack_search(int t, const std::vector<int32_t> &map, const std::vector<uint16_t> &neigh,
                 std::vector<int32_t> &m3, std::vector<uint16_t> &nb) {
    const bool e8 = eight_values(t);
    m3.assign(e8 ? 6561 : 4096, 0);
    nb.clear();
    std::unordered_map<int64_t, int> moved;             // file offset -> offset in nb
    for (int k = 0; k < (int)m3.size(); ++k) {
        int u = k, rr = k;
        if (e8) {
            u = 0;
            for (int i = 0; i < 8; ++i) { u |= (rr % 3) << (2 * i); rr /= 3; }
        }
        const int m = map[u];
        if (m >= 0) {
            m3[k] = m;
            continue;
        }
        const int64_t off = -(int64_t)m - 1;
        const int cnt = neigh[off];
        auto it = moved.find(off);
        int noff;
        if (it != moved.end()) {
            noff = it->second;
        } else {
            noff = (int)nb.size();
            if ((int64_t)noff + 1 + cnt > (int64_t)1 << 30) return false;
            nb.insert(nb.end(), neigh.begin() + off, neigh.begin() + off + 1 + cnt);
            moved.emplace(off, noff);
        }
        if (noff + 1 >= (1 << M3_OFF_BITS) || cnt >= (1 << (31 - M3_OFF_BITS))) return false;
        m3[k] = -1 - (noff | (cnt << M3_OFF_BITS));
    }
    return true;
}

template <class V> bool upload(V **dst, const std::vector<V> &src) {
    if (src.empty()) return true;
    if (hipMalloc((void **)dst, src.size() * sizeof(V)) != hipSuccess) return false;
    return hipMemcpy(*dst, src.data(), src.size() * sizeof(V), hipMemcpyHostToDevice) == hipSuccess;
}

// ------------------------------------------------------------------ launch plumbing
// the launch. Queue types: as many workgroups as the CUs hold at once (the kernel's occupancy, queried once), each
// wave taking tiles from a zeroed counter until they run out. Others: up to 32 waves a CU in flight or queued,
// grid-stride.
template <class T, int SRC> bool launch_q(const QParams &p0, hipStream_t st) {
    constexpr int spw = 64 / T::G, wgw = wgw_of<T>::v;
    static_assert((size_t)T::TAB + wgw * wave_bytes<T>() <= 160 * 1024, "a workgroup's LDS within a CU's 160 KiB");
    const size_t lds = (size_t)T::TAB + wgw * wave_bytes<T>();
    const int64_t tiles = (p0.nsb + spw - 1) / spw;
    int64_t wgs = (tiles + wgw - 1) / wgw;
    int64_t cap = (int64_t)g_ncu * 32 / wgw;
    QParams p = p0;
    p.tiles = nullptr;
    if (queue_of<T>::v && g_device >= 0 && g_device < 64 && g_tile_ctr[g_device]) {
        static std::atomic<int> occ{0};
        int n = occ.load();
        if (n == 0) {
            if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, k_quant<T, SRC>, 64 * wgw, lds) != hipSuccess ||
                n < 1)
                return false;
            occ.store(n);
        }
        cap = (int64_t)g_ncu * n;
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        if (hipStreamIsCapturing(st, &cs) != hipSuccess) return false;
        unsigned slot;
        if (cs == hipStreamCaptureStatusNone) {
            slot = g_tile_slot.fetch_add(1) % TILE_EAGER;
        } else {
            const unsigned c = g_tile_graph.fetch_add(1);
            if (cs != hipStreamCaptureStatusActive || c >= TILE_SLOTS - TILE_EAGER) {
                if (cs == hipStreamCaptureStatusActive)
                    fprintf(stderr, "gpuq: the %u tile counters reserved for captured launches are used up\n",
                            TILE_SLOTS - TILE_EAGER);
                return false;
            }
            slot = TILE_EAGER + c;
        }
        p.tiles = g_tile_ctr[g_device] + slot;
    }
    if (wgs > cap) wgs = cap;
    if (wgs < 1) wgs = 1;
    if (p.tiles) hipLaunchKernelGGL(k_tile_reset, dim3(1), dim3(64), 0, st, p.tiles);
    hipLaunchKernelGGL((k_quant<T, SRC>), dim3((unsigned)wgs), dim3(64 * wgw), lds, st, p);
    return hipGetLastError() == hipSuccess;
}

template <int SRC> bool launch_q8_stream(const QParams &p, hipStream_t st) {
    constexpr int E = SRC == T_F32 ? 4 : 8, TB = (64 / (32 / E)) * 4;
    const int64_t tiles = (p.nsb + TB - 1) / TB;
    int64_t wgs = (tiles + WG_WAVES - 1) / WG_WAVES;
    const int64_t cap = (int64_t)g_ncu * 16;
    if (wgs > cap) wgs = cap;
    if (wgs < 1) wgs = 1;
    hipLaunchKernelGGL((k_q8_0_stream<SRC>), dim3((unsigned)wgs), dim3(WG_THREADS), 0, st, p.src, p.dst, p.nsb);
    return hipGetLastError() == hipSuccess;
}

template <int SRC> bool dispatch_src(int type, const QParams &p, hipStream_t st) {
    switch (type) {
        case T_Q2_K: return launch_q<KQ2K, SRC>(p, st);
        case T_Q3_K: return launch_q<KQ3K, SRC>(p, st);
        case T_Q4_K: return launch_q<KQ45K<15>, SRC>(p, st);
        case T_Q5_K: return launch_q<KQ45K<31>, SRC>(p, st);
        case T_Q6_K: return launch_q<KQ6K, SRC>(p, st);
        case T_Q8_0:
            if (SRC == T_F32 || SRC == T_BF16) return launch_q8_stream<SRC == T_F32 ? T_F32 : T_BF16>(p, st);
            return launch_q<KQ80, SRC>(p, st);
        case T_IQ4_NL: return launch_q<KIQ4NL, SRC>(p, st);
        case T_IQ4_XS: return launch_q<KIQ4XS, SRC>(p, st);
        case T_Q4_0: return launch_q<KQ40, SRC>(p, st);
        case T_Q5_0: return launch_q<KQ50, SRC>(p, st);
        case T_Q5_1: return launch_q<KQ51, SRC>(p, st);
        case T_IQ2_XXS: return launch_q<KIQ2XXS, SRC>(p, st);
        case T_IQ2_XS: return launch_q<KIQ2XS, SRC>(p, st);
        case T_IQ2_S: return launch_q<KIQ2S, SRC>(p, st);
        case T_IQ1_S: return launch_q<KIQ1S, SRC>(p, st);
        case T_IQ1_M: return launch_q<KIQ1M, SRC>(p, st);
        case T_IQ3_XXS: return launch_q<KIQ3XXS, SRC>(p, st);
        case T_IQ3_S: return launch_q<KIQ3S, SRC>(p, st);
        default: return false;
    }
}

// every stored source encoding is decoded in registers inside the quantize kernel (SrcLoad in common.cuh)
bool fused_src(int src) {
    return src == T_F32 || src == T_F16 || src == T_BF16 || src == T_Q8_0 || src == T_MXFP4;
}

bool dispatch(int type, int src, const QParams &p, hipStream_t st) {
    switch (src) {
        case T_F32: return dispatch_src<T_F32>(type, p, st);
        case T_F16: return dispatch_src<T_F16>(type, p, st);
        case T_BF16: return dispatch_src<T_BF16>(type, p, st);
        case T_Q8_0: return dispatch_src<T_Q8_0>(type, p, st);
        case T_MXFP4: return dispatch_src<T_MXFP4>(type, p, st);
        default: return false;
    }
}

// the source pointer alignment and row length the fused loads need: F32 / F16 / BF16 read 16 bytes a load (base and
// row starts 16-byte aligned), Q8_0 16-bit words (2-byte blocks), MXFP4 bytes
bool src_aligned(int src, const void *raw, int64_t n_per_row) {
    const uintptr_t a = (uintptr_t)raw;
    switch (src) {
        case T_F32: return (a & 15) == 0 && (n_per_row * 4) % 16 == 0;
        case T_F16: case T_BF16: return (a & 15) == 0 && (n_per_row * 2) % 16 == 0;
        case T_Q8_0: return (a & 1) == 0;
        case T_MXFP4: return true;
        default: return false;
    }
}

bool launch_decode(int src, const void *in, float *out, int64_t n, hipStream_t st) {
    const int64_t nblk = n / 32;
    const unsigned grid = (unsigned)((nblk + 255) / 256);
    switch (src) {
        case T_F32: hipLaunchKernelGGL((k_decode<T_F32>), dim3(grid), dim3(256), 0, st, (const uint8_t *)in, out, nblk); break;
        case T_F16: hipLaunchKernelGGL((k_decode<T_F16>), dim3(grid), dim3(256), 0, st, (const uint8_t *)in, out, nblk); break;
        case T_BF16: hipLaunchKernelGGL((k_decode<T_BF16>), dim3(grid), dim3(256), 0, st, (const uint8_t *)in, out, nblk); break;
        case T_Q8_0: hipLaunchKernelGGL((k_decode<T_Q8_0>), dim3(grid), dim3(256), 0, st, (const uint8_t *)in, out, nblk); break;
        case T_MXFP4: hipLaunchKernelGGL((k_decode<T_MXFP4>), dim3(grid), dim3(256), 0, st, (const uint8_t *)in, out, nblk); break;
        default: return false;
    }
    return hipGetLastError() == hipSuccess;
}

bool takes_no_imatrix(int t) {
    return t == T_Q2_K || t == T_Q3_K || t == T_Q4_K || t == T_Q5_K || t == T_Q6_K || t == T_Q8_0 || t == T_IQ4_NL ||
           t == T_IQ4_XS || t == T_Q4_0 || t == T_Q5_0 || t == T_Q5_1 || t == T_F16;
}
// ggml's block length of an output type (F16: one value)
int block_len(int t) {
    return t == T_F16 ? 1 : t == T_IQ4_NL || t == T_Q8_0 || t == T_Q4_0 || t == T_Q5_0 || t == T_Q5_1 ? 32 : QK;
}
// the 32-weight types whose imatrix rule weighs by the row-wide sigma2
bool rowsig_type(int t) { return t == T_Q4_0 || t == T_Q5_0 || t == T_Q5_1; }
// sources F16 output reads value by value, for rows of any length
bool elementwise_src(int src) { return src == T_F32 || src == T_F16 || src == T_BF16; }
bool needs_tables(int t) { return is_search_type(t) || t == T_IQ1_M; }

int64_t src_bytes(int src, int64_t n) {
    switch (src) {
        case T_F32: return n * 4;
        case T_F16: case T_BF16: return n * 2;
        case T_Q8_0: return n / 32 * 34;
        case T_MXFP4: return n / 32 * 17;
        default: return 0;
    }
}

QParams params_for(int type, const void *src, void *dst, int64_t nunits, const float *qw, int64_t qw_mat,
                   int64_t qw_mod, int64_t qw_div) {
    QParams p{};
    p.src = (const uint8_t *)src;
    p.dst = (uint8_t *)dst;
    p.nsb = nunits;
    p.qw = type == T_Q8_0 || type == T_F16 ? nullptr : qw;   // (ggml_quantize_chunk ignores the imatrix for these)
    p.qw_mat = qw_mat;
    p.qw_mod = qw_mod;
    p.qw_div = qw_div;
    const Tabs &t = tab_of(type);
    p.grid = t.grid;
    p.map = t.map;
    p.neigh = t.neigh;
    p.npt = t.npt;
    p.map3 = t.map3;
    p.grid_size = t.grid_size;
    p.map_size = t.map_size;
    p.neigh_len = t.neigh_len;
    p.err = g_err;
    p.sb_stride = block_len(type);
    p.sb_off = 0;
    p.qw_stride = block_len(type);
    p.qw_off = 0;
    p.out_stride = (int64_t)gpuq_block_bytes(type);
    p.out_off = 0;
    return p;
}

bool type_ok(int type, int64_t n_per_row, bool with_imatrix) {
    if (g_device < 0 || !gpuq_block_bytes(type)) return false;
    if (needs_tables(type) && !tab_of(type).ok) return false;
    if (!with_imatrix && !takes_no_imatrix(type)) return false;
    return n_per_row > 0 && n_per_row % block_len(type) == 0;
}

// One launch of `rows` rows of n_per_row values (p: the quantize parameters of those rows' units): F16 one value a
// thread; the Q4_0 / Q5_0 / Q5_1 imatrix rules first write every row's sigma2 into sig (rows floats); the rest the
// quantize kernel.
bool launch_rows(int type, int src, QParams p, int64_t rows, int64_t n_per_row, float *sig, hipStream_t st) {
    if (type == T_F16) {
        const int64_t n = rows * n_per_row;
        const unsigned grid = (unsigned)((n + 255) / 256);
        uint16_t *o = (uint16_t *)p.dst;
        switch (src) {
            case T_F32: hipLaunchKernelGGL((k_to_f16<T_F32>), dim3(grid), dim3(256), 0, st, p.src, o, n); break;
            case T_F16: hipLaunchKernelGGL((k_to_f16<T_F16>), dim3(grid), dim3(256), 0, st, p.src, o, n); break;
            case T_BF16: hipLaunchKernelGGL((k_to_f16<T_BF16>), dim3(grid), dim3(256), 0, st, p.src, o, n); break;
            case T_Q8_0: hipLaunchKernelGGL((k_to_f16<T_Q8_0>), dim3(grid), dim3(256), 0, st, p.src, o, n); break;
            case T_MXFP4: hipLaunchKernelGGL((k_to_f16<T_MXFP4>), dim3(grid), dim3(256), 0, st, p.src, o, n); break;
            default: return false;
        }
        return hipGetLastError() == hipSuccess;
    }
    if (rowsig_type(type) && p.qw) {
        const unsigned grid = (unsigned)((rows + 255) / 256);
#define KSIG(S) hipLaunchKernelGGL((k_rowsig<S>), dim3(grid), dim3(256), 0, st, p.src, sig, rows, n_per_row)
        switch (src) {
            case T_F32: KSIG(T_F32); break;
            case T_F16: KSIG(T_F16); break;
            case T_BF16: KSIG(T_BF16); break;
            case T_Q8_0: KSIG(T_Q8_0); break;
            case T_MXFP4: KSIG(T_MXFP4); break;
            default: return false;
        }
#undef KSIG
        if (hipGetLastError() != hipSuccess) return false;
        p.rsig = sig;
        p.row_units = n_per_row / 32;
    }
    return dispatch(type, src, p, st);
}

// ------------------------------------------------------------------ the host API's streamed pipeline
// The reference's host entry points copy the whole input to the device, quantize, and copy the whole output back,
// one synchronous step after another (gpuq/gpuq.hip:2160-2250). Here one call is cut into chunks of whole rows
// (whole matrices when a matrix fits the chunk, else rows of one matrix, so every chunk keeps its imatrix row), and
// the chunks run through three slots: while chunk i is quantized, chunk i+1's source bytes go into pinned memory
// and on to the device, and chunk i-1's blocks come back; the host takes a chunk's blocks out of pinned memory two
// chunks later, so that waiting for them never holds up the next chunk's copy in (PCIe, ~57 GB/s each way, is the
// bound for the fast types). The bytes written equal those of one launch over the whole input: a block's result
// depends only on its own values and its matrix's imatrix row.

// pinned host memory (hipHostMalloc), kept for the process like the device buffers
struct PinBuf {
    void *p = nullptr;
    size_t cap = 0;
    bool grow(size_t need) {
        if (need <= cap) return true;
        if (p) (void)hipHostFree(p);
        p = nullptr;
        cap = 0;
        if (hipHostMalloc(&p, need, hipHostMallocDefault) != hipSuccess) {
            p = nullptr;
            return false;
        }
        cap = need;
        return true;
    }
};

constexpr int NSLOT = 3;
struct Slot {
    Buf in, out;                      // device: source bytes, blocks
    Buf sig;                          // device: the rows' sigma2 (Q4_0 / Q5_0 / Q5_1 with an imatrix)
    PinBuf pin_in, pin_out;
    hipEvent_t copied = nullptr;      // the slot's H2D copy is done: pin_in may be refilled
    hipEvent_t quantized = nullptr;   // the slot's kernels are done: in and f32 may be refilled, out is complete
    hipEvent_t returned = nullptr;    // the slot's D2H copy is done: out may be rewritten, pin_out is complete
    int64_t r0 = 0, rows = 0;         // the chunk the slot holds
    bool used = false;
};
Slot g_slot[NSLOT];
hipStream_t g_st_in = nullptr, g_st_q = nullptr, g_st_out = nullptr;   // default priority, non-blocking

bool pipe_ready() {
    if (g_st_out) return true;
    for (hipStream_t *s : {&g_st_in, &g_st_q, &g_st_out})
        if (hipStreamCreateWithFlags(s, hipStreamNonBlocking) != hipSuccess) return false;
    for (Slot &s : g_slot)
        for (hipEvent_t *e : {&s.copied, &s.quantized, &s.returned})   // (waits on them sleep rather than spin)
            if (hipEventCreateWithFlags(e, hipEventDisableTiming | hipEventBlockingSync) != hipSuccess) return false;
    return true;
}

// source bytes a chunk holds at most: GPUQ_STAGE_MB MiB (default 64; a chunk always holds at least one row)
int64_t stage_bytes() {
    const char *e = getenv("GPUQ_STAGE_MB");
    long mb = e ? strtol(e, nullptr, 10) : 64;
    if (mb < 1) mb = 64;
    return (int64_t)mb << 20;
}

// memcpy over up to 16 threads, at least 1 MiB each (pageable <-> pinned staging: one thread moves ~27 GB/s, 16
// about 110 GB/s, while PCIe takes ~57 GB/s each way)
void par_copy(void *dst, const void *src, size_t n) {
    constexpr size_t part_min = (size_t)1 << 20;
    unsigned nt = std::thread::hardware_concurrency();
    nt = nt == 0 ? 1 : (nt > 16 ? 16 : nt);
    if ((size_t)nt > n / part_min) nt = (unsigned)(n / part_min);
    if (nt <= 1) {
        memcpy(dst, src, n);
        return;
    }
    const size_t step = (n / nt + 4095) & ~(size_t)4095;
    std::vector<std::thread> th;
    size_t started = step;   // [0, step) is this thread's part; [step, started) went to other threads
    try {
        for (; started < n; started += step) {
            const size_t b = started, len = n - b < step ? n - b : step;
            th.emplace_back([=] { memcpy((char *)dst + b, (const char *)src + b, len); });
        }
    } catch (...) {   // a thread could not be started: copy what is left here
        memcpy((char *)dst + started, (const char *)src + started, n - started);
    }
    memcpy(dst, src, step);
    for (std::thread &t : th) t.join();
}

// the host API's body: raw bytes of nmat x nrow x n_per_row values (src encoding) -> dst (host); returns once dst
// holds every block, or 0 on an error
size_t quantize_host(int src, const void *raw, int type, void *dst, int64_t nmat, int64_t nrow, int64_t n_per_row,
                     const float *imatrix) {
    if (nmat <= 0 || nrow <= 0 || !type_ok(type, n_per_row, imatrix != nullptr)) return 0;
    const int64_t row_src = src_bytes(src, n_per_row);
    if (!row_src || (n_per_row % 32 && !(type == T_F16 && elementwise_src(src)))) return 0;
    std::lock_guard<std::mutex> lock(g_mu);
    if (!pipe_ready()) return 0;
    const int64_t nb_row = n_per_row / block_len(type), nb_mat = nrow * nb_row, rows = nmat * nrow;
    const int64_t row_out = nb_row * (int64_t)gpuq_block_bytes(type);
    // at least four chunks once the input passes 16 MiB, so that even one matrix overlaps its copies and kernels
    const int64_t budget = std::min(stage_bytes(), std::max<int64_t>((int64_t)4 << 20, (rows * row_src + 3) / 4));
    // chunk i from row r0: whole matrices when it starts at a matrix and its budget holds one, else rows up to the
    // end of the current matrix (so a chunk's blocks map to imatrix rows as in one launch); the first two chunks get
    // a quarter and a half of the budget, so the first kernel starts after a small copy
    auto chunk_end = [&](int64_t r0, int i) {
        const int64_t br = std::max<int64_t>(1, (i == 0 ? budget / 4 : i == 1 ? budget / 2 : budget) / row_src);
        const int64_t r1 = r0 % nrow == 0 && br >= nrow ? r0 + br / nrow * nrow
                                                        : std::min(r0 + br, (r0 / nrow + 1) * nrow);
        return std::min(r1, rows);
    };
    const int64_t max_rows = std::min(rows, std::max<int64_t>(1, budget / row_src));
    for (Slot &s : g_slot) {
        if (!s.in.grow((size_t)(max_rows * row_src) + 16) || !s.out.grow((size_t)(max_rows * row_out) + 16) ||
            !s.pin_in.grow((size_t)(max_rows * row_src)) || !s.pin_out.grow((size_t)(max_rows * row_out)) ||
            (rowsig_type(type) && imatrix && !s.sig.grow((size_t)max_rows * 4)))
            return 0;
        s.used = false;
    }
    const float *qw = nullptr;
    if (imatrix && type != T_Q8_0 && type != T_F16) {
        if (!g_qw.grow((size_t)nmat * n_per_row * 4)) return 0;
        if (hipMemcpy(g_qw.p, imatrix, (size_t)nmat * n_per_row * 4, hipMemcpyHostToDevice) != hipSuccess) return 0;
        qw = (const float *)g_qw.p;
    }
    if (hipMemsetAsync(g_err, 0, sizeof(int), g_st_q) != hipSuccess) return 0;

    bool ok = true;
    int64_t r0 = 0;
    int i = 0;
    auto drain = [&](int chunk) {   // the chunk's blocks: pinned -> dst
        const Slot &s = g_slot[chunk % NSLOT];
        if (hipEventSynchronize(s.returned) != hipSuccess) return false;
        par_copy((uint8_t *)dst + s.r0 * row_out, s.pin_out.p, (size_t)(s.rows * row_out));
        return true;
    };
    while (ok && r0 < rows) {
        const int64_t r1 = chunk_end(r0, i), cr = r1 - r0;
        const size_t in_bytes = (size_t)(cr * row_src), out_bytes = (size_t)(cr * row_out);
        Slot &s = g_slot[i % NSLOT];
        // source bytes -> pinned, once the slot's previous H2D copy has read them; -> device, once the slot's
        // previous kernels have read its device buffers
        if (s.used && hipEventSynchronize(s.copied) != hipSuccess) { ok = false; break; }
        par_copy(s.pin_in.p, (const uint8_t *)raw + r0 * row_src, in_bytes);
        if (s.used) ok = hipStreamWaitEvent(g_st_in, s.quantized, 0) == hipSuccess;
        ok = ok && hipMemcpyAsync(s.in.p, s.pin_in.p, in_bytes, hipMemcpyHostToDevice, g_st_in) == hipSuccess &&
             hipEventRecord(s.copied, g_st_in) == hipSuccess;
        // quantize (the source decoded in registers), once the bytes are in and the slot's previous blocks have left
        ok = ok && hipStreamWaitEvent(g_st_q, s.copied, 0) == hipSuccess;
        if (ok && s.used) ok = hipStreamWaitEvent(g_st_q, s.returned, 0) == hipSuccess;
        if (ok) {
            const float *cqw = qw ? qw + (r0 / nrow) * n_per_row : nullptr;
            const QParams p = params_for(type, s.in.p, s.out.p, cr * nb_row, cqw, nb_mat, nb_row, 1);
            ok = launch_rows(type, src, p, cr, n_per_row, (float *)s.sig.p, g_st_q) &&
                 hipEventRecord(s.quantized, g_st_q) == hipSuccess;
        }
        // blocks -> pinned (the slot's previous blocks were taken out of pin_out by the last iteration)
        ok = ok && hipStreamWaitEvent(g_st_out, s.quantized, 0) == hipSuccess &&
             hipMemcpyAsync(s.pin_out.p, s.out.p, out_bytes, hipMemcpyDeviceToHost, g_st_out) == hipSuccess &&
             hipEventRecord(s.returned, g_st_out) == hipSuccess;
        s.used = true;
        s.r0 = r0;
        s.rows = cr;
        if (ok && i >= NSLOT - 1) ok = drain(i - (NSLOT - 1));   // frees the pinned blocks of the slot used next
        r0 = r1;
        ++i;
    }
    for (int c = std::max(0, i - (NSLOT - 1)); ok && c < i; ++c) ok = drain(c);
    // every stream is idle before the call returns (the buffers are reused by the next call)
    bool idle = true;
    for (hipStream_t st : {g_st_in, g_st_q, g_st_out}) idle = hipStreamSynchronize(st) == hipSuccess && idle;
    if (!ok || !idle) return 0;
    int err = 0;
    if (hipMemcpy(&err, g_err, sizeof(int), hipMemcpyDeviceToHost) != hipSuccess || err) return 0;
    return (size_t)(rows * row_out);
}

// the LDLQ loop's side stream and its events (created once, on the library's device; default priority); g_ev_done
// marks the end of the last gpuq_ldlq_dev call's launches (g_ldlq_pending: one was recorded)
hipStream_t g_st2 = nullptr;
hipEvent_t g_ev_start = nullptr, g_ev_solved = nullptr, g_ev_rest = nullptr, g_ev_done = nullptr;
bool g_ldlq_pending = false;
bool side_stream_ready() {
    if (g_st2) return true;
    for (hipEvent_t *e : {&g_ev_start, &g_ev_solved, &g_ev_rest, &g_ev_done})
        if (hipEventCreateWithFlags(e, hipEventDisableTiming) != hipSuccess) return false;
    return hipStreamCreateWithFlags(&g_st2, hipStreamNonBlocking) == hipSuccess;
}

// W -= Es . U[c0 .. c0+255][cb .. ce) for every matrix
bool launch_update(float *W, const double *Es, const double *U, int64_t u_stride, int64_t nmat, int64_t ne1,
                   int64_t ne0, int64_t c0, int64_t cb, int64_t ce, hipStream_t st) {
    const int64_t nt = ((ce - cb + LDLQ_TN - 1) / LDLQ_TN) * ((ne1 + LDLQ_TM - 1) / LDLQ_TM) * nmat;
    const unsigned grid = (unsigned)((nt + 7) / 8 * 8);   // (a multiple of the 8 XCDs; see ldlq_tile)
    hipLaunchKernelGGL(k_ldlq_update, dim3(grid), dim3(256), 0, st, W, Es, U, u_stride, nmat, ne1, ne0, c0, cb, ce);
    return hipGetLastError() == hipSuccess;
}

// the 256-weight types whose quantizer is closed per super-block and that have a device dequantizer (the
// reference's LDLQ_TYPES, tools/requant_experts.py:195-196, plus Q2_K / Q3_K)
bool ldlq_type(int t) {
    return t == T_IQ2_XXS || t == T_IQ2_XS || t == T_IQ2_S || t == T_IQ3_XXS || t == T_IQ3_S || t == T_IQ1_S ||
           t == T_IQ1_M || t == T_IQ4_XS || t == T_Q2_K || t == T_Q3_K || t == T_Q4_K || t == T_Q5_K || t == T_Q6_K;
}

bool launch_solve(int type, const float *W, const uint8_t *q, int64_t q_stride, int64_t q_off, const double *U,
                  int64_t u_stride, int64_t nmat, int64_t ne1, int64_t ne0, int64_t c0, double *Es, hipStream_t st) {
    const dim3 grid((unsigned)((ne1 + 63) / 64), (unsigned)nmat);
    const uint64_t *dq = tab_of(type).dq;
#define KSOLVE(T) hipLaunchKernelGGL((k_ldlq_solve<T>), grid, dim3(64), 0, st, W, q, q_stride, q_off, U, u_stride, \
                                     ne1, ne0, c0, Es, dq)
    switch (type) {
        case T_IQ2_XXS: KSOLVE(T_IQ2_XXS); break;
        case T_IQ2_XS: KSOLVE(T_IQ2_XS); break;
        case T_IQ2_S: KSOLVE(T_IQ2_S); break;
        case T_IQ3_XXS: KSOLVE(T_IQ3_XXS); break;
        case T_IQ3_S: KSOLVE(T_IQ3_S); break;
        case T_IQ1_S: KSOLVE(T_IQ1_S); break;
        case T_IQ1_M: KSOLVE(T_IQ1_M); break;
        case T_IQ4_XS: KSOLVE(T_IQ4_XS); break;
        case T_Q2_K: KSOLVE(T_Q2_K); break;
        case T_Q3_K: KSOLVE(T_Q3_K); break;
        case T_Q4_K: KSOLVE(T_Q4_K); break;
        case T_Q5_K: KSOLVE(T_Q5_K); break;
        case T_Q6_K: KSOLVE(T_Q6_K); break;
        default: return false;
    }
#undef KSOLVE
    return hipGetLastError() == hipSuccess;
}

}  // namespace

// ------------------------------------------------------------------ the C ABI
extern "C" int gpuq_init(const char *tables, int device) {
    std::lock_guard<std::mutex> lock(g_mu);
    if (hipSetDevice(device) != hipSuccess) return 1;
    if (device >= 0 && device < 64 && !g_scratch[device]) {     // (the device is current)
        void *ptr = nullptr;
        if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || !ptr) return 4;
        g_scratch[device] = (double *)ptr;
        ptr = nullptr;
        if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(tile_ctr)) != hipSuccess || !ptr) return 4;
        g_tile_ctr[device] = (unsigned long long *)ptr;
    }
    int ncu = 0;
    if (hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, device) == hipSuccess && ncu > 0) g_ncu = ncu;
    if (!g_err && hipMalloc((void **)&g_err, sizeof(int)) != hipSuccess) return 4;
    FILE *f = fopen(tables, "rb");
    if (!f) return 2;
    struct Rec {
        int type;
        std::vector<uint64_t> grid;
        std::vector<int32_t> map;
        std::vector<uint16_t> neigh;
        std::vector<int32_t> m3;        // (search types) the staged map and the lists it reaches: pack_search
        std::vector<uint16_t> nb;
    };
    std::vector<Rec> recs;
    int32_t hdr[4];
    while (fread(hdr, sizeof hdr, 1, f) == 1) {
        if (hdr[1] < 0 || hdr[2] < 0 || hdr[3] < 0 || hdr[1] > (1 << 20) || hdr[2] > (1 << 20) || hdr[3] > (1 << 26)) {
            fclose(f);
            return 3;
        }
        Rec r{hdr[0], std::vector<uint64_t>(hdr[1]), std::vector<int32_t>(hdr[2]), std::vector<uint16_t>(hdr[3]), {}, {}};
        if (fread(r.grid.data(), 8, hdr[1], f) != (size_t)hdr[1] || fread(r.map.data(), 4, hdr[2], f) != (size_t)hdr[2] ||
            fread(r.neigh.data(), 2, hdr[3], f) != (size_t)hdr[3]) {
            fclose(f);
            return 3;
        }
        recs.push_back(std::move(r));
    }
    fclose(f);
    // validate everything before touching the device tables
    bool synthetic = false;
    for (Rec &r : recs) {
        if (r.type == SYNTHETIC_MARK) {
            synthetic = true;
        } else if (r.type >= 1000) {
            const int t = r.type - 1000;
            if (t < 0 || t >= 64 || !is_search_type(t) || (int)r.grid.size() != expected_grid(t)) return 6;
        } else if (r.type >= 0 && r.type < 64 && is_search_type(r.type)) {
            if (!valid_search(r.type, r.grid, r.map, r.neigh)) return 6;
            if (!pack_search(r.type, r.map, r.neigh, r.m3, r.nb)) return 6;
        }
    }
    // the tables of an earlier call are replaced but stay allocated until the process ends: launches still in flight
    // and graphs captured before this call keep the old pointers in their parameters and go on reading them
    for (Tabs &t : g_tabs) {
        for (void *p : {(void *)t.grid, (void *)t.map, (void *)t.map3, (void *)t.neigh, (void *)t.npt, (void *)t.dq})
            if (p) g_retired.push_back(p);
        t = Tabs();
    }
    // stand-in codebooks (the file carries the mark) are loaded only where the caller asks for them: quantizing
    // with them writes grid indices llama.cpp would read against ggml's own grids
    const char *allow = getenv("GPUQ_ALLOW_SYNTHETIC_TABLES");
    if (synthetic && !(allow && allow[0] == '1')) recs.clear();
    for (const Rec &r : recs) {
        if (r.type == SYNTHETIC_MARK) continue;
        if (r.type >= 1000) {
            Tabs &t = g_tabs[r.type - 1000];
            if (!upload(&t.dq, r.grid)) return 4;
            t.dq_size = (int)r.grid.size();
        } else if (r.type >= 0 && r.type < 64 && is_search_type(r.type)) {
            Tabs &t = g_tabs[r.type];
            if (!upload(&t.grid, r.grid) || !upload(&t.map, r.map) || !upload(&t.neigh, r.nb) ||
                !upload(&t.map3, r.m3))
                return 4;
            if (!eight_values(r.type)) {    // the lists' points (the searches read them with the list entries)
                std::vector<uint32_t> npt(r.nb.size(), 0u);
                for (size_t off = 0; off < r.nb.size(); off += 1 + (size_t)r.nb[off])
                    for (size_t j = 1; j <= r.nb[off]; ++j) npt[off + j] = (uint32_t)r.grid[r.nb[off + j]];
                if (!upload(&t.npt, npt)) return 4;
            }
            t.grid_size = (int)r.grid.size();
            t.map_size = (int)r.map.size();
            t.neigh_len = (int)r.nb.size();
            t.ok = true;
        }
    }
    g_device = device;
    return 0;
}

extern "C" size_t gpuq_block_bytes(int type) {
    switch (type) {
        case T_IQ2_XXS: return 66;
        case T_IQ2_S: return 82;
        case T_IQ1_S: return 50;
        case T_IQ1_M: return 56;
        case T_IQ2_XS: return 74;
        case T_IQ3_XXS: return 98;
        case T_IQ3_S: return 110;
        case T_IQ4_NL: return 18;
        case T_IQ4_XS: return 136;
        case T_Q2_K: return 84;
        case T_Q3_K: return 110;
        case T_Q4_K: return 144;
        case T_Q5_K: return 176;
        case T_Q6_K: return 210;
        case T_Q8_0: return 34;
        case T_Q4_0: return 18;
        case T_Q5_0: return 22;
        case T_Q5_1: return 24;
        case T_F16: return 2;
        default: return 0;
    }
}

extern "C" int gpuq_can_quantize(int type, int with_imatrix) {
    return type_ok(type, block_len(type), with_imatrix != 0) ? 1 : 0;
}

extern "C" size_t gpuq_quantize_batch(int type, const float *src, void *dst, int64_t nmat, int64_t nrow,
                                      int64_t n_per_row, const float *imatrix) {
    return quantize_host(T_F32, src, type, dst, nmat, nrow, n_per_row, imatrix);
}

extern "C" size_t gpuq_quantize(int type, const float *src, void *dst, int64_t nrow, int64_t n_per_row,
                                const float *imatrix) {
    return quantize_host(T_F32, src, type, dst, 1, nrow, n_per_row, imatrix);
}

extern "C" int gpuq_can_dequantize(int src) { return src_bytes(src, 32) > 0 ? 1 : 0; }

extern "C" size_t gpuq_requantize_batch(int src, const void *raw, int type, void *dst, int64_t nmat, int64_t nrow,
                                        int64_t n_per_row, const float *imatrix) {
    return quantize_host(src, raw, type, dst, nmat, nrow, n_per_row, imatrix);
}

extern "C" size_t gpuq_requantize(int src, const void *raw, int type, void *dst, int64_t nrow, int64_t n_per_row,
                                  const float *imatrix) {
    return quantize_host(src, raw, type, dst, 1, nrow, n_per_row, imatrix);
}

extern "C" size_t gpuq_quantize_dev(int type, const float *d_x, void *d_dst, int64_t nblocks, const float *d_qw,
                                    int64_t qw_mod, int64_t qw_div, void *stream) {
    if (block_len(type) != QK || !type_ok(type, QK, d_qw != nullptr) || nblocks <= 0 || qw_mod <= 0 || qw_div <= 0)
        return 0;
    if (((uintptr_t)d_x & 15) || (d_qw && ((uintptr_t)d_qw & 15)) || ((uintptr_t)d_dst & 1)) return 0;
    const QParams p = params_for(type, d_x, d_dst, nblocks, d_qw, INT64_MAX, qw_mod, qw_div);
    if (!dispatch(type, T_F32, p, (hipStream_t)stream)) return 0;
    return (size_t)nblocks * gpuq_block_bytes(type);
}

extern "C" int gpuq_can_dequantize_type(int type) {
    switch (type) {
        case T_IQ2_XXS: case T_IQ2_XS: case T_IQ2_S: case T_IQ3_XXS: case T_IQ3_S: case T_IQ1_S: case T_IQ1_M:
            return g_device >= 0 && tab_of(type).dq != nullptr;
        case T_IQ4_XS: case T_Q2_K: case T_Q3_K: case T_Q4_K: case T_Q5_K: case T_Q6_K:
            return g_device >= 0 ? 1 : 0;
        default: return 0;
    }
}

extern "C" size_t gpuq_dequantize_dev(int type, const void *d_q, float *d_out, int64_t nblocks, void *stream) {
    if (!gpuq_can_dequantize_type(type) || nblocks <= 0 || ((uintptr_t)d_q & 1) || ((uintptr_t)d_out & 15)) return 0;
    const hipStream_t st = (hipStream_t)stream;
    const unsigned grid = (unsigned)((nblocks * 8 + 255) / 256);
    const uint64_t *dq = tab_of(type).dq;
    const uint8_t *q = (const uint8_t *)d_q;
#define KDQ(T, BB) hipLaunchKernelGGL((k_dequant<T, BB>), dim3(grid), dim3(256), 0, st, q, d_out, nblocks, dq)
    switch (type) {
        case T_IQ2_XXS: KDQ(T_IQ2_XXS, 66); break;
        case T_IQ2_XS: KDQ(T_IQ2_XS, 74); break;
        case T_IQ2_S: KDQ(T_IQ2_S, 82); break;
        case T_IQ3_XXS: KDQ(T_IQ3_XXS, 98); break;
        case T_IQ3_S: KDQ(T_IQ3_S, 110); break;
        case T_IQ1_S: KDQ(T_IQ1_S, 50); break;
        case T_IQ1_M: KDQ(T_IQ1_M, 56); break;
        case T_IQ4_XS: KDQ(T_IQ4_XS, 136); break;
        case T_Q2_K: KDQ(T_Q2_K, 84); break;
        case T_Q3_K: KDQ(T_Q3_K, 110); break;
        case T_Q4_K: KDQ(T_Q4_K, 144); break;
        case T_Q5_K: KDQ(T_Q5_K, 176); break;
        case T_Q6_K: KDQ(T_Q6_K, 210); break;
        default: return 0;
    }
#undef KDQ
    return hipGetLastError() == hipSuccess ? (size_t)nblocks * QK * 4 : 0;
}

extern "C" size_t gpuq_dequantize_src_dev(int src, const void *d_raw, float *d_out, int64_t n, void *stream) {
    if (!src_bytes(src, 32) || n <= 0 || n % 32 || ((uintptr_t)d_out & 15)) return 0;
    if ((src == T_F32 || src == T_F16 || src == T_BF16) && ((uintptr_t)d_raw & 15)) return 0;
    if (src == T_Q8_0 && ((uintptr_t)d_raw & 1)) return 0;
    if (!launch_decode(src, d_raw, d_out, n, (hipStream_t)stream)) return 0;
    return (size_t)n * 4;
}

// Device-pointer requantize (no counterpart in the reference): nmat matrices of nrow x n_per_row values stored as
// src (F32 / F16 / BF16 / Q8_0 / MXFP4, decoded in registers inside the quantize kernel) -> d_dst, matrix m
// weighted by d_imatrix + m * n_per_row (or no imatrix). Asynchronous on `stream`. Returns the bytes the launch will
// write.
extern "C" size_t gpuq_requantize_dev(int src, const void *d_raw, int type, void *d_dst, int64_t nmat, int64_t nrow,
                                      int64_t n_per_row, const float *d_imatrix, void *stream) {
    if (nmat <= 0 || nrow <= 0 || !fused_src(src) || !type_ok(type, n_per_row, d_imatrix != nullptr)) return 0;
    if (type == T_F16) {    // value by value: any row length from F32 / F16 / BF16, element-aligned
        const uintptr_t am = src == T_F32 ? 3 : src == T_MXFP4 ? 0 : 1;
        if ((n_per_row % 32 && !elementwise_src(src)) || ((uintptr_t)d_raw & am)) return 0;
    } else if (n_per_row % 32 || !src_aligned(src, d_raw, n_per_row)) {
        return 0;
    }
    if ((d_imatrix && ((uintptr_t)d_imatrix & 15)) || ((uintptr_t)d_dst & 1)) return 0;
    const hipStream_t st = (hipStream_t)stream;
    const int bs = block_len(type);
    const int64_t nb_row = n_per_row / bs, nb_mat = nrow * nb_row, nunits = nmat * nb_mat, rows = nmat * nrow;
    const QParams p = params_for(type, d_raw, d_dst, nunits, d_imatrix, nb_mat, nb_row, 1);
    if (rowsig_type(type) && d_imatrix) {
        // the rows' sigma2 in a stream-ordered allocation, released on the stream after the launch (not under
        // capture: the allocation would become part of the graph)
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        if (hipStreamIsCapturing(st, &cs) != hipSuccess) return 0;
        if (cs != hipStreamCaptureStatusNone) {
            fprintf(stderr, "gpuq_requantize_dev: Q4_0 / Q5_0 / Q5_1 with an imatrix refused under stream capture\n");
            return 0;
        }
        void *sig = nullptr;
        if (hipMallocAsync(&sig, (size_t)rows * 4, st) != hipSuccess) return 0;
        const bool ok = launch_rows(type, src, p, rows, n_per_row, (float *)sig, st);
        if (hipFreeAsync(sig, st) != hipSuccess || !ok) return 0;
    } else if (!launch_rows(type, src, p, rows, n_per_row, nullptr, st)) {
        return 0;
    }
    return (size_t)nunits * gpuq_block_bytes(type);
}

// Reads and clears the search-failure flag (no counterpart in the reference, whose kernels trap instead): 1 when a
// device-API launch since the last call found a key with no candidate point (non-finite input or a bad table).
extern "C" int gpuq_take_error(void) {
    if (!g_err) return 0;
    int err = 0;
    if (hipDeviceSynchronize() != hipSuccess) return 1;
    if (hipMemcpy(&err, g_err, sizeof(int), hipMemcpyDeviceToHost) != hipSuccess) return 1;
    (void)hipMemset(g_err, 0, sizeof(int));
    return err;
}

// The LDLQ error-feedback loop on the device (tools/ldlq.py:71-107 quantize_matrix / 391-431 quantize_matrix_torch;
// no single counterpart symbol in the reference, which drives gpuq_quantize_dev / gpuq_dequantize_dev and torch from
// Python). d_wp: nmat matrices [ne1][ne0] f32 in permuted column order, updated in place; d_u: the upper Cholesky
// factor of the permuted inverse Hessian, [ne0][ne0] f64 row-major, matrix m's at d_u + m*u_stride (0: shared);
// d_qw: [nmat][ne0] f32 importances in permuted order; blk_order (host, ne0/256 entries): the output slot of permuted
// block k; d_out: [nmat][ne1][ne0/256 blocks]. feedback = 0 quantizes every block as is. Asynchronous on `stream`.
namespace {

// the argument checks both LDLQ entry points share
bool ldlq_args_ok(int type, const float *d_wp, const double *d_u, int64_t u_stride, const float *d_qw, int64_t nmat,
                  int64_t ne1, int64_t ne0, const int64_t *blk_order, const void *d_out) {
    if (!ldlq_type(type) || !gpuq_can_dequantize_type(type) || !type_ok(type, ne0, d_qw != nullptr)) return false;
    if (nmat <= 0 || ne1 <= 0 || ne0 <= 0 || ne0 % QK || u_stride < 0 || !blk_order) return false;
    if (((uintptr_t)d_wp & 15) || (d_qw && ((uintptr_t)d_qw & 15)) || ((uintptr_t)d_u & 7) || ((uintptr_t)d_out & 1))
        return false;
    const int64_t nblk = ne0 / QK;
    for (int64_t k = 0; k < nblk; ++k)
        if (blk_order[k] < 0 || blk_order[k] >= nblk) return false;
    return true;
}

// The loop's launches on `st`, with es holding two blocks of Es (2 * rows * 256 doubles; the update of block k's
// later columns still reads Es(k) while Es(k+1) is solved). side: block k's update is split, the next block's 256
// columns on `st` (they gate quantizing block k+1) and the rest on the library's side stream, where it runs beside
// block k+1's quantization and solve; every column still receives its updates in block order (the next-block part of
// update k waits for the side stream's update k-1), and `st` joins the side stream at the end. Without side, every
// launch is on `st`. Launches only: allocates nothing.
bool ldlq_loop(int type, float *d_wp, const double *d_u, int64_t u_stride, const float *d_qw, int64_t nmat,
               int64_t ne1, int64_t ne0, const int64_t *blk_order, bool fb, void *d_out, hipStream_t st, double *es2,
               bool side) {
    const int64_t nblk = ne0 / QK, bb = (int64_t)gpuq_block_bytes(type), rows = nmat * ne1;
    if (fb && side) {
        if (hipEventRecord(g_ev_start, st) != hipSuccess || hipStreamWaitEvent(g_st2, g_ev_start, 0) != hipSuccess)
            return false;
    }
    bool rest_pending = false;      // a side-stream update not yet waited for by the caller's stream
    for (int64_t k = 0; k < nblk; ++k) {
        const int64_t c0 = k * QK;
        QParams p = params_for(type, d_wp, d_out, rows, d_qw, ne1, 1, 1);
        p.sb_stride = ne0;
        p.sb_off = c0;
        p.qw_stride = ne0;
        p.qw_off = c0;
        p.out_stride = nblk * bb;
        p.out_off = blk_order[k] * bb;
        if (!dispatch(type, T_F32, p, st)) return false;
        if (!fb || k + 1 >= nblk) continue;
        double *es = es2 + (size_t)(k & 1) * rows * QK;
        if (!launch_solve(type, d_wp, (const uint8_t *)d_out, nblk * bb, blk_order[k] * bb, d_u, u_stride, nmat, ne1,
                          ne0, c0, es, st))
            return false;
        const int64_t cn = side && c0 + 2 * QK < ne0 ? c0 + 2 * QK : ne0;
        if (side) {
            if (hipEventRecord(g_ev_solved, st) != hipSuccess) return false;
            if (rest_pending) {
                if (hipStreamWaitEvent(st, g_ev_rest, 0) != hipSuccess) return false;
                rest_pending = false;
            }
        }
        if (!launch_update(d_wp, es, d_u, u_stride, nmat, ne1, ne0, c0, c0 + QK, cn, st)) return false;
        if (cn < ne0) {
            if (hipStreamWaitEvent(g_st2, g_ev_solved, 0) != hipSuccess ||
                !launch_update(d_wp, es, d_u, u_stride, nmat, ne1, ne0, c0, cn, ne0, g_st2) ||
                hipEventRecord(g_ev_rest, g_st2) != hipSuccess)
                return false;
            rest_pending = true;
        }
    }
    if (fb && side) {   // the caller's stream joins the side stream
        if (hipEventRecord(g_ev_rest, g_st2) != hipSuccess || hipStreamWaitEvent(st, g_ev_rest, 0) != hipSuccess)
            return false;
    }
    return true;
}

}  // namespace

extern "C" size_t gpuq_ldlq_dev(int type, float *d_wp, const double *d_u, int64_t u_stride, const float *d_qw,
                                int64_t nmat, int64_t ne1, int64_t ne0, const int64_t *blk_order, int feedback,
                                void *d_out, void *stream) {
    if (!ldlq_args_ok(type, d_wp, d_u, u_stride, d_qw, nmat, ne1, ne0, blk_order, d_out)) return 0;
    const hipStream_t st = (hipStream_t)stream;
    const int64_t nblk = ne0 / QK, bb = (int64_t)gpuq_block_bytes(type), rows = nmat * ne1;
    // not capturable: its Es buffer grows, it is shared with eager calls through an event that a capture would only
    // record as a node, and it forks onto the library's side stream; under capture, gpuq_ldlq_dev_noalloc
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(st, &cs) != hipSuccess) return 0;
    if (cs != hipStreamCaptureStatusNone) {
        fprintf(stderr, "gpuq_ldlq_dev: refused under stream capture (use gpuq_ldlq_dev_noalloc)\n");
        return 0;
    }
    std::lock_guard<std::mutex> lock(g_mu);
    const bool fb = feedback && nblk > 1;
    if (fb && (!g_es.grow((size_t)2 * rows * QK * 8) || !side_stream_ready())) return 0;
    // calls share Es and the side stream: each call's launches wait for the previous call's (on whatever stream it
    // ran), so calls from several streams never run over each other's Es
    if (fb && g_ldlq_pending && hipStreamWaitEvent(st, g_ev_done, 0) != hipSuccess) return 0;
    if (!ldlq_loop(type, d_wp, d_u, u_stride, d_qw, nmat, ne1, ne0, blk_order, fb, d_out, st, (double *)g_es.p, true))
        return 0;
    if (fb) {
        if (hipEventRecord(g_ev_done, st) != hipSuccess) return 0;
        g_ldlq_pending = true;
    }
    return (size_t)(rows * nblk * bb);
}

// gpuq_ldlq_dev for callers that cannot allocate (code under HIP graph capture, serving loops): the same loop with
// the same bytes, its Es in the library's static `scratch` array instead of a buffer it grows, every launch on
// `stream` (no side stream), no event, lock or allocation. At most LDLQ_SCRATCH_ROWS rows (nmat * ne1) with feedback;
// a larger call is refused before any launch. Calls share the device's array: calls that overlap on one GPU race.
extern "C" size_t gpuq_ldlq_dev_noalloc(int type, float *d_wp, const double *d_u, int64_t u_stride, const float *d_qw,
                                        int64_t nmat, int64_t ne1, int64_t ne0, const int64_t *blk_order,
                                        int feedback, void *d_out, void *stream) {
    if (!ldlq_args_ok(type, d_wp, d_u, u_stride, d_qw, nmat, ne1, ne0, blk_order, d_out)) return 0;
    const int64_t nblk = ne0 / QK, bb = (int64_t)gpuq_block_bytes(type), rows = nmat * ne1;
    const bool fb = feedback && nblk > 1;
    double *es = g_device >= 0 && g_device < 64 ? g_scratch[g_device] : nullptr;
    if (fb && !es) return 0;
    if (fb && rows > LDLQ_SCRATCH_ROWS) {
        fprintf(stderr, "gpuq_ldlq_dev_noalloc: %lld rows (nmat x ne1) exceed the scratch maximum of %lld\n",
                (long long)rows, (long long)LDLQ_SCRATCH_ROWS);
        return 0;
    }
    if (!ldlq_loop(type, d_wp, d_u, u_stride, d_qw, nmat, ne1, ne0, blk_order, fb, d_out, (hipStream_t)stream, es,
                   false))
        return 0;
    return (size_t)(rows * nblk * bb);
}

// ------------------------------------------------------------------ the Hessian preparation and the host LDLQ loop
namespace {

// rocBLAS / rocSOLVER, opened on first use (the quantizer never needs them): the copies the process already loaded
// when the caller's framework brought them (same sonames), else ROCm's
struct Lapack {
    bool tried = false, ok = false;
    decltype(&rocblas_create_handle) create = nullptr;
    decltype(&rocblas_set_stream) set_stream = nullptr;
    decltype(&rocsolver_dpotrf) potrf = nullptr;
    decltype(&rocsolver_dpotri) potri = nullptr;
    rocblas_handle h = nullptr;
};
Lapack g_lp;
std::mutex g_mu_h;   // the Hessian preparation's handle and buffers
Buf g_hd;            // device: diag (f64) | perm (i64) | dead (u8) | factorization info

bool lapack_ready() {
    if (g_lp.tried) return g_lp.ok;
    g_lp.tried = true;
    void *blas = dlopen("librocblas.so.5", RTLD_NOW | RTLD_GLOBAL);
    void *sol = dlopen("librocsolver.so.0", RTLD_NOW | RTLD_GLOBAL);
    if (!blas || !sol) return false;
    g_lp.create = (decltype(g_lp.create))dlsym(blas, "rocblas_create_handle");
    g_lp.set_stream = (decltype(g_lp.set_stream))dlsym(blas, "rocblas_set_stream");
    g_lp.potrf = (decltype(g_lp.potrf))dlsym(sol, "rocsolver_dpotrf");
    g_lp.potri = (decltype(g_lp.potri))dlsym(sol, "rocsolver_dpotri");
    if (!g_lp.create || !g_lp.set_stream || !g_lp.potrf || !g_lp.potri) return false;
    if (hipSetDevice(g_device) != hipSuccess || g_lp.create(&g_lp.h) != rocblas_status_success) return false;
    g_lp.ok = true;
    return true;
}

// a factorization's info (0: done; > 0: not positive definite), -1 when it cannot be read
int read_info(const int *d_info, hipStream_t st) {
    int v = -1;
    if (hipMemcpyAsync(&v, d_info, sizeof(int), hipMemcpyDeviceToHost, st) != hipSuccess ||
        hipStreamSynchronize(st) != hipSuccess)
        return -1;
    return v;
}

std::mutex g_mu_l;   // the host LDLQ loop's buffers and stream
Buf g_lH, g_lU, g_lW, g_lWp, g_lqw, g_lout, g_lperm;
hipStream_t g_st_l = nullptr;

}  // namespace

// H += X^T X on the device (the Hessian sum of tools/hessian_from_dump.py:73-79 of the reference, there a float32
// GEMM a chunk of rows added into float64): X [nrows][ne0] f32, H [ne0][ne0] f64 (symmetric, kept so); here every
// product is exact in f64 and each sum runs over the rows in order on the f64 matrix cores. Asynchronous on stream.
// Returns 0, 1 for bad arguments (ne0 a multiple of 256, at most 65280), 4 on a HIP error.
extern "C" int gpuq_hessian_accumulate_dev(const float *d_X, int64_t nrows, int64_t ne0, double *d_H, void *stream) {
    if (g_device < 0 || !d_X || !d_H || nrows <= 0 || ne0 <= 0 || ne0 % QK || ne0 > 65535) return 1;
    if (((uintptr_t)d_X & 3) || ((uintptr_t)d_H & 7)) return 1;
    const hipStream_t st = (hipStream_t)stream;
    const unsigned nt = (unsigned)(ne0 / 128);
    hipLaunchKernelGGL(k_xtx, dim3(nt, nt), dim3(256), 0, st, d_X, nrows, ne0, d_H);
    hipLaunchKernelGGL(k_hess_mirror, dim3((unsigned)((ne0 + 255) / 256), (unsigned)ne0), dim3(256), 0, st, d_H, ne0);
    return hipGetLastError() == hipSuccess ? 0 : 4;
}

// The LDLQ factor on the device: prepare_hessian (tools/ldlq.py:34-68 of the reference) on a device H [ne0][ne0]
// (f64, row-major, symmetric: the sum of x x^T over n inputs). Writes d_U (row-major, upper: U^T U is the inverse of
// Hp = Hn[perm][:, perm] + damp * mean(diag) * I, Hn = H / max(n, 1) with dead columns (diag <= 0) replaced by unit
// rows; one retry with 10x more ridge when Hp does not factor), and on the host perm (ne0 column indices, whole
// 256-blocks: order 0 'seq' keeps them in order, 1 'act' sorts them by descending energy, ties in order), diag_n
// (diag(Hn)[perm]) and dead (ne0 flags, original order); either of the last two may be NULL. Returns 0, or 1 for bad
// arguments, 2 when rocBLAS / rocSOLVER cannot be loaded, 3 when the matrix does not factor, 4 on a HIP error.
extern "C" int gpuq_prepare_hessian_dev(const double *d_H, int64_t ne0, double n, double damp, int order, double *d_U,
                                        int64_t *perm, double *diag_n, uint8_t *dead, void *stream) {
    if (g_device < 0 || !d_H || !d_U || !perm || ne0 <= 0 || ne0 % QK || ne0 > 65535) return 1;   // (grid rows)
    if ((order != 0 && order != 1) || !(damp >= 0) || ((uintptr_t)d_H & 7) || ((uintptr_t)d_U & 7)) return 1;
    std::lock_guard<std::mutex> lock(g_mu_h);
    if (!lapack_ready()) return 2;
    const hipStream_t st = (hipStream_t)stream;
    if (g_lp.set_stream(g_lp.h, st) != rocblas_status_success) return 4;
    const size_t o_perm = (size_t)ne0 * 8, o_dead = o_perm + (size_t)ne0 * 8, o_info = (o_dead + ne0 + 15) & ~15ull;
    if (!g_hd.grow(o_info + 16)) return 4;
    double *dd = (double *)g_hd.p;
    int64_t *dp = (int64_t *)((uint8_t *)g_hd.p + o_perm);
    uint8_t *dz = (uint8_t *)g_hd.p + o_dead;
    int *dinfo = (int *)((uint8_t *)g_hd.p + o_info);
    const double nd = 1.0 > n ? 1.0 : n;                       // max(n, 1)
    const unsigned g1 = (unsigned)((ne0 + 255) / 256);
    const dim3 g2(g1, (unsigned)ne0);
    hipLaunchKernelGGL(k_hess_diag, dim3(g1), dim3(256), 0, st, d_H, ne0, nd, dd);
    std::vector<double> d((size_t)ne0);
    if (hipMemcpyAsync(d.data(), dd, (size_t)ne0 * 8, hipMemcpyDeviceToHost, st) != hipSuccess ||
        hipStreamSynchronize(st) != hipSuccess)
        return 4;
    std::vector<uint8_t> zd((size_t)ne0);
    for (int64_t i = 0; i < ne0; ++i) {
        zd[i] = d[i] <= 0;
        if (zd[i]) d[i] = 1.0;
    }
    const int64_t nblk = ne0 / QK;
    std::vector<int64_t> bo((size_t)nblk);
    for (int64_t b = 0; b < nblk; ++b) bo[b] = b;
    if (order == 1) {
        std::vector<double> key((size_t)nblk);          // -energy; NaN sorts last, as numpy's argsort puts it
        for (int64_t b = 0; b < nblk; ++b) {
            double e = 0;
            for (int i = 0; i < QK; ++i) e += d[b * QK + i];
            key[b] = e != e ? HUGE_VAL : -e;
        }
        std::stable_sort(bo.begin(), bo.end(), [&](int64_t a, int64_t b) { return key[a] < key[b]; });
    }
    std::vector<int64_t> pm((size_t)ne0);
    double mean = 0;
    for (int64_t i = 0; i < ne0; ++i) {
        pm[i] = bo[i / QK] * QK + i % QK;
        mean += d[pm[i]];
    }
    mean /= (double)ne0;
    if (hipMemcpyAsync(dp, pm.data(), (size_t)ne0 * 8, hipMemcpyHostToDevice, st) != hipSuccess ||
        hipMemcpyAsync(dz, zd.data(), (size_t)ne0, hipMemcpyHostToDevice, st) != hipSuccess)
        return 4;
    const double r1 = damp * mean;
    const rocblas_int nn = (rocblas_int)ne0;
    hipLaunchKernelGGL(k_hess_perm, g2, dim3(256), 0, st, d_H, ne0, nd, (const int64_t *)dp, (const uint8_t *)dz, r1,
                       d_U);
    if (g_lp.potrf(g_lp.h, rocblas_fill_lower, nn, d_U, nn, dinfo) != rocblas_status_success) return 4;
    int info = read_info(dinfo, st);
    if (info > 0) {                                       // more ridge until it factors
        hipLaunchKernelGGL(k_hess_perm, g2, dim3(256), 0, st, d_H, ne0, nd, (const int64_t *)dp,
                           (const uint8_t *)dz, r1, d_U);
        hipLaunchKernelGGL(k_diag_add, dim3(g1), dim3(256), 0, st, d_U, ne0, 10 * damp * mean);
        if (g_lp.potrf(g_lp.h, rocblas_fill_lower, nn, d_U, nn, dinfo) != rocblas_status_success) return 4;
        info = read_info(dinfo, st);
    }
    if (info != 0) return info > 0 ? 3 : 4;
    // Hp^-1 from the factor (lower triangle), made symmetric, then its own lower factor: read row-major, U
    if (g_lp.potri(g_lp.h, rocblas_fill_lower, nn, d_U, nn, dinfo) != rocblas_status_success) return 4;
    if ((info = read_info(dinfo, st)) != 0) return info > 0 ? 3 : 4;
    hipLaunchKernelGGL(k_sym_from_lower, g2, dim3(256), 0, st, d_U, ne0);
    if (g_lp.potrf(g_lp.h, rocblas_fill_lower, nn, d_U, nn, dinfo) != rocblas_status_success) return 4;
    if ((info = read_info(dinfo, st)) != 0) return info > 0 ? 3 : 4;
    hipLaunchKernelGGL(k_zero_upper, g2, dim3(256), 0, st, d_U, ne0);
    if (hipGetLastError() != hipSuccess || hipStreamSynchronize(st) != hipSuccess) return 4;
    for (int64_t i = 0; i < ne0; ++i) {
        perm[i] = pm[i];
        if (diag_n) diag_n[i] = d[pm[i]];
        if (dead) dead[i] = zd[i];
    }
    return 0;
}

// The 'schur' importance of every 256-column block of a factor (tools/ldlq.py:90-93; no single counterpart symbol in
// the reference, which computes it in numpy or torch): d_u [ne0][ne0] f64 upper factor (device) -> d_w [nrep][ne0]
// f32 (device), the same ne0 values in each of the nrep rows. Fixed summation order (k_schur_weights). Asynchronous
// on `stream`. Returns 0, 1 for bad arguments, 4 on a HIP error.
extern "C" int gpuq_schur_weights_dev(const double *d_u, int64_t ne0, float *d_w, int64_t nrep, void *stream) {
    if (g_device < 0 || !d_u || !d_w || ne0 <= 0 || ne0 % QK || ne0 > 65535 * (int64_t)QK || nrep <= 0) return 1;
    if (((uintptr_t)d_u & 7) || ((uintptr_t)d_w & 3)) return 1;
    hipLaunchKernelGGL(k_schur_weights, dim3(QK, (unsigned)(ne0 / QK)), dim3(64), 0, (hipStream_t)stream, d_u, ne0,
                       d_w, nrep);
    return hipGetLastError() == hipSuccess ? 0 : 4;
}

// The LDLQ loop from host memory, with no framework on the caller's side (tools/ldlq.py:71-107 of the reference,
// quantize_matrix with the factor from prepare_hessian): W [nmat][ne1][ne0] f32 (original column order), H the
// Hessian sum over n inputs, [ne0][ne0] f64, one for all matrices (h_stride 0) or one a matrix (h_stride ne0*ne0).
// weights: the importance each block's quantizer gets, 0 'imatrix' (imatrix [nmat][ne0] permuted; NULL only for a
// type that takes none), 1 'diag' (diag(H)/n, permuted), 2 'schur' (diag((U_BB^T U_BB)^-1) of each block). Writes
// the GGUF bytes of every matrix to dst and returns their count, or 0 on an error (a factor that cannot be built
// included).
extern "C" size_t gpuq_ldlq(int type, const float *W, const double *H, int64_t h_stride, double n, double damp,
                            int order, int weights, const float *imatrix, int64_t nmat, int64_t ne1, int64_t ne0,
                            void *dst) {
    if (!W || !H || !dst || nmat <= 0 || ne1 <= 0 || ne0 <= 0 || ne0 % QK) return 0;
    if (h_stride != 0 && h_stride != ne0 * ne0) return 0;
    if (weights < 0 || weights > 2 || (weights != 0 && imatrix)) return 0;
    const bool with_qw = weights != 0 || imatrix;
    if (!ldlq_type(type) || !gpuq_can_dequantize_type(type) || !type_ok(type, ne0, with_qw)) return 0;
    std::lock_guard<std::mutex> lock(g_mu_l);
    if (!g_st_l && hipStreamCreateWithFlags(&g_st_l, hipStreamNonBlocking) != hipSuccess) return 0;
    const hipStream_t st = g_st_l;
    const int64_t nblk = ne0 / QK, row_bytes = nblk * (int64_t)gpuq_block_bytes(type);
    const int64_t gsz = h_stride ? 1 : nmat;            // matrices that share a factor
    const size_t wbytes = (size_t)gsz * ne1 * ne0 * 4, obytes = (size_t)gsz * ne1 * row_bytes;
    if (!g_lH.grow((size_t)ne0 * ne0 * 8) || !g_lU.grow((size_t)ne0 * ne0 * 8) || !g_lW.grow(wbytes) ||
        !g_lWp.grow(wbytes) || !g_lqw.grow((size_t)gsz * ne0 * 4) || !g_lout.grow(obytes + 16) ||
        !g_lperm.grow((size_t)ne0 * 8))
        return 0;
    if (hipMemsetAsync(g_err, 0, sizeof(int), st) != hipSuccess) return 0;
    std::vector<int64_t> perm((size_t)ne0), slots((size_t)nblk);
    std::vector<double> diag_n((size_t)ne0);
    std::vector<float> qw(weights != 2 && with_qw ? (size_t)gsz * ne0 : 0);
    const unsigned gy = (unsigned)std::min<int64_t>(gsz * ne1, 65535);
    for (int64_t m0 = 0; m0 < nmat; m0 += gsz) {
        if (hipMemcpyAsync(g_lH.p, H + (h_stride ? m0 * h_stride : 0), (size_t)ne0 * ne0 * 8, hipMemcpyHostToDevice,
                           st) != hipSuccess ||
            gpuq_prepare_hessian_dev((const double *)g_lH.p, ne0, n, damp, order, (double *)g_lU.p, perm.data(),
                                     diag_n.data(), nullptr, st) != 0)
            return 0;
        for (int64_t k = 0; k < nblk; ++k) slots[k] = perm[k * QK] / QK;
        if (weights == 0 && imatrix) {
            for (int64_t m = 0; m < gsz; ++m)
                for (int64_t c = 0; c < ne0; ++c) qw[m * ne0 + c] = imatrix[(m0 + m) * ne0 + perm[c]];
        } else if (weights == 1) {
            for (int64_t m = 0; m < gsz; ++m)
                for (int64_t c = 0; c < ne0; ++c) qw[m * ne0 + c] = (float)diag_n[c];
        }
        if (hipMemcpyAsync(g_lW.p, W + m0 * ne1 * ne0, wbytes, hipMemcpyHostToDevice, st) != hipSuccess ||
            hipMemcpyAsync(g_lperm.p, perm.data(), (size_t)ne0 * 8, hipMemcpyHostToDevice, st) != hipSuccess ||
            (!qw.empty() && hipMemcpyAsync(g_lqw.p, qw.data(), (size_t)gsz * ne0 * 4, hipMemcpyHostToDevice, st) !=
                                hipSuccess))
            return 0;
        if (weights == 2 && gpuq_schur_weights_dev((const double *)g_lU.p, ne0, (float *)g_lqw.p, gsz, st) != 0)
            return 0;
        hipLaunchKernelGGL(k_gather_cols, dim3((unsigned)((ne0 + 255) / 256), gy), dim3(256), 0, st,
                           (const float *)g_lW.p, (float *)g_lWp.p, (const int64_t *)g_lperm.p, gsz * ne1, ne0);
        if (hipGetLastError() != hipSuccess) return 0;
        if (!gpuq_ldlq_dev(type, (float *)g_lWp.p, (const double *)g_lU.p, 0, with_qw ? (const float *)g_lqw.p : nullptr,
                           gsz, ne1, ne0, slots.data(), 1, g_lout.p, st))
            return 0;
        if (hipMemcpyAsync((uint8_t *)dst + m0 * ne1 * row_bytes, g_lout.p, obytes, hipMemcpyDeviceToHost, st) !=
                hipSuccess ||
            hipStreamSynchronize(st) != hipSuccess)
            return 0;
    }
    int err = 0;
    if (hipMemcpy(&err, g_err, sizeof(int), hipMemcpyDeviceToHost) != hipSuccess || err) return 0;
    return (size_t)(nmat * ne1 * row_bytes);
}
