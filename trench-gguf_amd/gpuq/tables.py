"""Search and dequantization tables for the i-quants, in the gpuq_tables.bin layout.

File layout (the reference's gpuq/gpuq_tables.c:5-8, read by gpuq_init, gpuq/gpuq.hip:2059-2080): a sequence of
records, each `int32 type, grid_size, map_size, neigh_len`, then `uint64 grid[grid_size]`, `int32 map[map_size]`,
`uint16 neighbours[neigh_len]`. Search records carry ggml type ids 16, 17, 19, 22 (IQ2_XXS, IQ2_XS, IQ1_S, IQ2_S: 8
values a point, 2-bit keys, map of 43692) and 18, 21 (IQ3_XXS, IQ3_S: 4 values a point in the low 4 bytes, 3-bit keys,
map of 4096). A search point stores 2l+1 for each level l. map[u] >= 0 is the index of the point whose key is u;
map[u] < 0 means neighbours[-map[u]-1] is a count n followed by n point indices. Dequantizer grids are records of type
1000 + t with no map and no neighbours.

ggml builds these tables in iq2xs_init_impl / iq3xs_init_impl from its own codebooks (ggml-common.h), which are not
available here. `synthetic_tables()` therefore builds self-consistent stand-ins of the same shapes with a documented
rule, so that every consumer (the HIP library, the CPU oracle, the reference library built from source) searches the
same tables:
  - grid: the `grid_size` level vectors of lowest cost sum(c[l_i]) (ties broken by a fixed integer hash of the key),
    among those whose key fits the map;
  - neighbours of an off-grid key: every grid point within the `nwant` smallest distinct squared distances between
    the key's 2l+1 vector and the point's, ordered by (distance, index) - the rule ggml's init functions apply;
  - dequantizer grids: IQ2 levels -> {8, 25, 43, 59}, IQ3_XXS levels -> {4, 12, 20, 28, 36, 44, 52, 62}, IQ3_S
    levels -> {1, 3, ..., 15}, IQ1 levels -> {-1, 0, 1}: what each to_float's scale arithmetic expects.
A gpuq_tables.bin written by the reference's gpuq_tables.c from ggml's own code replaces this file one for one.

The file written here ends with one more record, the stand-in mark: type 0x53594e54 with one grid entry (the bytes
"SYNTHTAB") and no map or neighbours. The reference's loader keeps it as a table of a type nothing asks for; libgpuq's
gpuq_init loads the stand-in IQ1/IQ2/IQ3 tables of a marked file only when GPUQ_ALLOW_SYNTHETIC_TABLES=1 is set
(tests and benchmarks), so that no model file is written with grid indices into stand-in codebooks by accident.
"""
import hashlib
import struct

import numpy as np

IQ2_XXS, IQ2_XS, IQ3_XXS, IQ1_S, IQ3_S, IQ2_S = 16, 17, 18, 19, 21, 22
MAP2 = 43692    # 2-bit keys of 8 levels up to the all-2 key 0xAAAA (+ slack), ggml's kmap_size
MAP3 = 4096     # 3-bit keys of 4 levels
MARK = 0x53594E54                                   # the stand-in mark's record type
MARK_GRID = np.frombuffer(b"SYNTHTAB", dtype="<u8")  # its one grid entry

# (type, grid points, levels a coordinate, values a point, neighbour distance shells)
SPECS = [
    (IQ2_XXS, 256, 4, 8, 2),
    (IQ2_XS, 512, 4, 8, 2),
    (IQ1_S, 2048, 3, 8, 3),
    (IQ2_S, 1024, 4, 8, 1),
    (IQ3_XXS, 256, 8, 4, 2),
    (IQ3_S, 512, 8, 4, 3),
]
DQ_VALUES = {
    IQ2_XXS: [8, 25, 43, 59], IQ2_XS: [8, 25, 43, 59], IQ2_S: [8, 25, 43, 59],
    IQ3_XXS: [4, 12, 20, 28, 36, 44, 52, 62], IQ3_S: [1, 3, 5, 7, 9, 11, 13, 15],
    IQ1_S: [-1, 0, 1],
}


def _hash32(v):
    v = (np.asarray(v, dtype=np.uint64) * np.uint64(0x9E3779B97F4A7C15)) & np.uint64(0xFFFFFFFFFFFFFFFF)
    return (v >> np.uint64(40)).astype(np.int64)


def _levels_of_keys(keys, nval, bits):
    keys = np.asarray(keys, dtype=np.int64)
    return np.stack([(keys >> (bits * i)) & ((1 << bits) - 1) for i in range(nval)], axis=1)


def _grid(n, nlev, nval, bits, map_size):
    """the n lowest-cost level vectors whose key fits the map"""
    if nlev == 3:
        cost = np.array([1.0, 0.0, 1.0])            # IQ1: levels -1, 0, +1
    elif nlev == 4:
        cost = np.array([0.0, 1.0, 2.6, 4.5])
    else:
        cost = np.arange(nlev, dtype=np.float64) ** 1.25
    keys = np.arange(map_size if bits == 2 else 1 << (bits * nval), dtype=np.int64)
    lv = _levels_of_keys(keys, nval, bits)
    ok = (lv < nlev).all(axis=1) & (keys < map_size)
    keys, lv = keys[ok], lv[ok]
    score = (cost[lv].sum(axis=1) * 1e6).astype(np.int64) * (1 << 24) + (_hash32(keys) & 0xFFFFFF)
    pick = np.sort(keys[np.argsort(score, kind="stable")[:n]])
    return pick, _levels_of_keys(pick, nval, bits)


def _neighbours(grid_lv, map_size, nval, bits, nwant, on_grid):
    """ggml's neighbour rule for every off-grid key of the map"""
    gpos = (2 * grid_lv + 1).astype(np.float64)                  # [G, nval]
    g2 = (gpos * gpos).sum(axis=1)
    keys = np.nonzero(~on_grid)[0]
    lists = []
    for c0 in range(0, len(keys), 4096):
        kk = keys[c0:c0 + 4096]
        kp = (2 * _levels_of_keys(kk, nval, bits) + 1).astype(np.float64)        # [K, nval]
        # squared distances |k|^2 + |g|^2 - 2 k.g: small integers, exact in float64
        d2 = ((kp * kp).sum(axis=1)[:, None] + g2[None, :] - 2.0 * (kp @ gpos.T)).astype(np.int32)
        sd = np.sort(d2, axis=1)
        new = np.ones_like(sd, dtype=bool)
        new[:, 1:] = sd[:, 1:] != sd[:, :-1]
        shell = np.cumsum(new, axis=1)                                           # 1-based distinct-distance rank
        cnt = (shell <= nwant).sum(axis=1)
        thr = sd[np.arange(len(kk)), cnt - 1]                                    # the nwant-th distinct distance
        rows, cols = np.nonzero(d2 <= thr[:, None])
        o = np.lexsort((cols, d2[rows, cols], rows))                             # (row, distance, index) order
        cols = cols[o]
        ends = np.cumsum(cnt)
        lists.extend(np.split(cols, ends[:-1]))
    return keys, lists


# the extreme set: the same grids and rule with more distance shells, so lists run long (up to 490 points) and the
# file's list offsets pass 2^21 (IQ1_S: 3.2M entries), bounding how the search's cost and the loader's packing depend
# on the tables' shape
EXTREME_SHELLS = {IQ2_XXS: 5, IQ2_XS: 4, IQ1_S: 4, IQ2_S: 4, IQ3_XXS: 5, IQ3_S: 6}


def synthetic_tables(shells=None):
    """[(type, grid uint64[G], map int32[M], neighbours uint16[N])] in the reference writer's record order; shells:
    {type: distance shells} replacing SPECS' (EXTREME_SHELLS for the extreme set)"""
    recs = []
    for typ, n, nlev, nval, nwant in SPECS:
        nwant = (shells or {}).get(typ, nwant)
        bits = 2 if nval == 8 else 3
        map_size = MAP2 if nval == 8 else MAP3
        gkeys, glv = _grid(n, nlev, nval, bits, map_size)
        pts = (2 * glv + 1).astype(np.uint64)
        grid = np.zeros(n, dtype=np.uint64)
        for i in range(nval):
            grid |= pts[:, i] << np.uint64(8 * i)
        kmap = np.full(map_size, -1, dtype=np.int64)
        kmap[gkeys] = np.arange(n)
        keys, lists = _neighbours(glv, map_size, nval, bits, nwant, kmap >= 0)
        lens = np.array([len(lst) for lst in lists], dtype=np.int64)
        offs = np.concatenate([[0], np.cumsum(lens + 1)[:-1]])
        kmap[keys] = -(offs + 1)
        neigh = np.concatenate([np.concatenate([[n_], lst]) for n_, lst in zip(lens, lists)]).astype(np.uint16)
        recs.append((typ, grid, kmap.astype(np.int32), neigh))
    order_dq = [IQ2_XXS, IQ2_XS, IQ2_S, IQ3_XXS, IQ3_S, IQ1_S]
    by_type = {r[0]: r for r in recs}
    for typ in order_dq:
        grid = by_type[typ][1]
        nval = 8 if typ in (IQ2_XXS, IQ2_XS, IQ2_S, IQ1_S) else 4
        vals = np.asarray(DQ_VALUES[typ], dtype=np.int64)
        dq = np.zeros(len(grid), dtype=np.uint64)
        for i in range(nval):
            lev = ((grid >> np.uint64(8 * i)) & np.uint64(0xFF)).astype(np.int64)
            v = vals[(lev - 1) // 2] & 0xFF
            dq |= v.astype(np.uint64) << np.uint64(8 * i)
        recs.append((1000 + typ, dq, np.zeros(0, dtype=np.int32), np.zeros(0, dtype=np.uint16)))
    return recs


def mark_record():
    return (MARK, MARK_GRID.copy(), np.zeros(0, dtype=np.int32), np.zeros(0, dtype=np.uint16))


def write_tables(path, recs=None, mark=True):
    """recs (default: the stand-ins) in the file layout, followed by the stand-in mark unless mark=False"""
    recs = list(synthetic_tables() if recs is None else recs)
    if mark:
        recs.append(mark_record())
    with open(path, "wb") as f:
        for typ, grid, kmap, neigh in recs:
            f.write(struct.pack("<4i", typ, len(grid), len(kmap), len(neigh)))
            f.write(np.ascontiguousarray(grid, dtype="<u8").tobytes())
            f.write(np.ascontiguousarray(kmap, dtype="<i4").tobytes())
            f.write(np.ascontiguousarray(neigh, dtype="<u2").tobytes())
    return path


def read_tables(path):
    """{type: (grid uint64, map int32, neighbours uint16)}"""
    out = {}
    with open(path, "rb") as f:
        data = f.read()
    o = 0
    while o + 16 <= len(data):
        typ, g, m, n = struct.unpack_from("<4i", data, o)
        o += 16
        grid = np.frombuffer(data, dtype="<u8", count=g, offset=o); o += 8 * g
        kmap = np.frombuffer(data, dtype="<i4", count=m, offset=o); o += 4 * m
        neigh = np.frombuffer(data, dtype="<u2", count=n, offset=o); o += 2 * n
        out[typ] = (grid, kmap, neigh)
    return out


def is_synthetic(path):
    """the file carries the stand-in mark"""
    return MARK in read_tables(path)


def content_sha(path):
    """sha256 of the table records without the stand-in mark (the mark is written last, so this is the hash of the
    file as it was before the mark existed)"""
    data = open(path, "rb").read()
    tail = 16 + 8
    if len(data) >= tail and struct.unpack_from("<4i", data, len(data) - tail) == (MARK, 1, 0, 0):
        data = data[:-tail]
    return hashlib.sha256(data).hexdigest()


if __name__ == "__main__":
    import sys
    args = [a for a in sys.argv[1:] if a != "--extreme"]
    write_tables(args[0] if args else "gpuq_tables.bin",
                 synthetic_tables(EXTREME_SHELLS) if "--extreme" in sys.argv else None)
