"""The oracle's fallback types (oracle/gq_oracle.c: o_q0, o_q5_1, quant_row_legacy and F16 in gqo_quantize_chunk):
llama-quantize's Q4_0 / Q5_0 / Q5_1 / F16 for rows that are not whole 256-weight super-blocks
(tools/requant_experts.py:180-192). The reference writes them through ggml on the CPU and holds no vectors for them,
and ggml is not part of it, so the oracle is pinned here by what ggml's rules fix:

- F16: IEEE round-to-nearest-even of every finite value (numpy's conversion), NaN to 0x7E00 with the value's sign;
- the plain rules (quantize_row_q4_0_ref / q5_0_ref / q5_1_ref): the stored scale is fp16(max / -nmax) (Q4_0 / Q5_0,
  max the first value of largest magnitude) or fp16((max - min) / 31) and fp16(min) (Q5_1); every level is the
  nearest of its grid (within half a step of the value, ties upward), the largest-magnitude value's level is 0, and
  only values past the last step are clamped to the top level;
- the imatrix rules (quantize_row_*_impl), weights qw * sqrt(sigma2 + x^2) with sigma2 the mean of x^2 over the
  whole row: the levels are those of one of make_qx_quants' trial scales, the stored scale is the weighted
  least-squares scale of those levels, and no trial scores higher (Q4_0 / Q5_0); the stored (d, m) are the weighted
  least-squares fit of the levels with m <= 0, or the start (max - min) / 31, min (Q5_1); a block's bytes depend on
  the rest of its row.

Each check is shown to catch a planted mistake: nibbles swapped, the scale's sign flipped, block-wide sigma2."""
import numpy as np
import pytest

Q4_0, Q5_0, Q5_1, F16 = 2, 6, 7, 1
NMAX = {Q4_0: 8, Q5_0: 16}
BB = {Q4_0: 18, Q5_0: 22, Q5_1: 24}


def rows(rng, nrow, ncol):
    x = (rng.standard_normal((nrow, ncol)) * rng.uniform(0.005, 0.05, (nrow, 1))).astype(np.float32)
    x[0] = 0                                                    # an all-zero row
    x[1, ::7] *= 40                                             # spikes
    x[2] = np.abs(x[2])                                         # one-signed
    x[3] *= np.float32(1e-18)                                   # x^2 subnormal
    return x


def h16(v):
    return np.float32(v).astype(np.float16).view(np.uint16)


def levels(typ, blk):
    """(levels [32], fp16 d bits, fp16 m bits or None) of one block"""
    d = int(blk[0]) | int(blk[1]) << 8
    if typ == Q4_0:
        qs = blk[2:18]
        return np.concatenate([qs & 15, qs >> 4]).astype(np.int64), d, None
    qh_at, qs_at = (2, 6) if typ == Q5_0 else (4, 8)
    qh = int.from_bytes(bytes(blk[qh_at:qh_at + 4]), "little")
    qs = blk[qs_at:qs_at + 16]
    lv = np.concatenate([qs & 15, qs >> 4]).astype(np.int64)
    lv |= ((qh >> np.arange(32)) & 1) << 4
    return lv, d, (int(blk[2]) | int(blk[3]) << 8) if typ == Q5_1 else None


def f16f(bits):
    return np.float64(np.uint16(bits).view(np.float16))


def check_plain(typ, xb, blk):
    """the plain rule's facts for one block; returns a reason string when one fails"""
    lv, d, m = levels(typ, blk)
    if typ in NMAX:
        nm = NMAX[typ]
        k = int(np.argmax(np.abs(xb)))                       # (first of the largest magnitudes)
        d32 = np.float32(xb[k]) / np.float32(-nm)
        if d != int(h16(d32)):
            return "scale"
        if d32 == 0:
            return None if np.all(lv == nm) else "zero block"
        if lv[k] != 0:
            return "largest value's level"
        pos = (xb.astype(np.float64) / np.float64(d32)) + nm    # the value on the level grid
        top = lv == 2 * nm - 1
        off = np.abs(pos - lv)
        if np.any(off[~top] > 0.5 + 1e-5) or np.any(pos[top] < 2 * nm - 1.5 - 1e-5):
            return "levels"
        return None
    mn, mx = np.float32(xb.min()), np.float32(xb.max())
    d32 = (mx - mn) / np.float32(31)
    if d != int(h16(d32)) or m != int(h16(mn)):
        return "scale / min"
    if d32 == 0:
        return None if np.all(lv == 0) else "flat block"
    pos = (xb.astype(np.float64) - np.float64(mn)) / np.float64(d32)
    if np.any(np.abs(pos - lv) > 0.5 + 1e-5) or lv[int(np.argmin(xb))] != 0 or lv[int(np.argmax(xb))] != 31:
        return "levels"
    return None


@pytest.mark.parametrize("typ", [Q4_0, Q5_0, Q5_1], ids=["q4_0", "q5_0", "q5_1"])
def test_plain_rule_facts(oracle_lib, typ):
    rng = np.random.default_rng(typ)
    x = rows(rng, 24, 160)
    out = oracle_lib.quantize(typ, x).reshape(24, 5, BB[typ])
    bad = [(r, b, why) for r in range(24) for b in range(5)
           if (why := check_plain(typ, x[r, 32 * b:32 * b + 32], out[r, b])) is not None]
    assert not bad, bad[:5]
    # planted: nibbles swapped (Q4_0 / Q5_0 / Q5_1), or the scale's sign flipped
    blk = out[4, 0].copy()
    qs_at = {Q4_0: 2, Q5_0: 6, Q5_1: 8}[typ]
    blk[qs_at:qs_at + 16] = ((blk[qs_at:qs_at + 16] & 15) << 4) | (blk[qs_at:qs_at + 16] >> 4)
    assert check_plain(typ, x[4, :32], blk) is not None
    if typ in NMAX:
        blk = out[4, 0].copy()
        blk[1] ^= 0x80
        assert check_plain(typ, x[4, :32], blk) is not None


def weights(x_row, qw_row, block_wide=False):
    """qw * sqrt(sigma2 + x^2), sigma2 the mean of x^2 over the row (float32, ggml's serial sum)"""
    if block_wide:
        s2 = np.repeat(np.mean((x_row.astype(np.float64) ** 2).reshape(-1, 32), axis=1), 32)
    else:
        s = np.float32(0)
        for v in x_row:
            s = np.float32(s + np.float32(v * v))
        s2 = np.float32(s / np.float32(x_row.size))
    return (qw_row.astype(np.float64) * np.sqrt(s2 + x_row.astype(np.float64) ** 2))


def check_imatrix_q0(typ, xb, wb, blk):
    """make_qx_quants' facts for one block (wb: its weights); None when they hold"""
    nm = NMAX[typ]
    lv, d, _ = levels(typ, blk)
    if np.max(np.abs(xb)) < 1e-15:
        return None if d == 0 and np.all(lv == 0) else "negligible block"
    l = lv - nm
    x64 = xb.astype(np.float64)
    k = int(np.argmax(np.abs(xb)))
    iscales = [-np.float32(nm) / xb[k]] + [-(np.float32(nm) + np.float32(0.1) * np.float32(i)) / xb[k]
                                           for i in range(-9, 10) if i]
    trials = [np.clip(np.floor(np.float32(s) * xb + 0.5), -nm, nm - 1) for s in iscales]
    if not any(np.array_equal(t, l) for t in trials):
        return "levels of no trial scale"
    sl2 = float(np.sum(wb * l * l))
    if sl2 <= 0:
        return None
    scale = float(np.sum(wb * x64 * l)) / sl2
    if abs(f16f(d) - scale) > 1e-3 * abs(scale) + 1e-30:
        return "least-squares scale %g vs %g" % (f16f(d), scale)
    scores = [float(np.sum(wb * x64 * t)) ** 2 / max(float(np.sum(wb * t * t)), 1e-300) for t in trials]
    if float(np.sum(wb * x64 * l)) ** 2 / sl2 < max(scores) * (1 - 1e-4):
        return "a trial scores higher"
    return None


def check_imatrix_q51(xb, wb, blk):
    lv, d, m = levels(Q5_1, blk)
    x64 = xb.astype(np.float64)
    sw, sx, sl = np.sum(wb), np.sum(wb * x64), np.sum(wb * lv)
    sl2, sxl = np.sum(wb * lv * lv), np.sum(wb * x64 * lv)
    D = sw * sl2 - sl * sl
    fits = []
    if D > 0:
        sc, mn = (sw * sxl - sx * sl) / D, (sl2 * sx - sl * sxl) / D
        if mn > 0:
            sc, mn = sxl / sl2, 0.0
        fits.append((sc, mn))
    mn32, mx32 = np.float32(xb.min()), np.float32(xb.max())
    fits.append((float((mx32 - mn32) / np.float32(31)), float(mn32)))          # (no trial beat the start)
    ok = any(abs(f16f(d) - sc) <= 2e-3 * abs(sc) + 1e-30 and abs(f16f(m) - mn) <= 2e-3 * abs(mn) + 1e-6 * abs(sc)
             for sc, mn in fits)
    return None if ok else "d, m %g %g vs %s" % (f16f(d), f16f(m), fits)


@pytest.mark.parametrize("typ", [Q4_0, Q5_0, Q5_1], ids=["q4_0", "q5_0", "q5_1"])
def test_imatrix_rule_facts(oracle_lib, typ):
    rng = np.random.default_rng(10 + typ)
    x = rows(rng, 16, 160)[4:]                              # (rows with negligible blocks are checked apart)
    x = (x * np.repeat(np.array([1.0, 10.0, 0.1, 3.0, 0.3], np.float32), 32)).astype(np.float32)   # block scales
    qw = rng.lognormal(0.0, 1.5, 160).astype(np.float32)
    out = oracle_lib.quantize(typ, x, qw).reshape(x.shape[0], 5, BB[typ])

    def fails(block_wide):
        n = 0
        for r in range(x.shape[0]):
            w = weights(x[r], qw, block_wide)
            for b in range(5):
                sl = slice(32 * b, 32 * b + 32)
                why = (check_imatrix_q0(typ, x[r, sl], w[sl], out[r, b]) if typ in NMAX
                       else check_imatrix_q51(x[r, sl], w[sl], out[r, b]))
                n += why is not None
        return n
    assert fails(False) == 0
    assert fails(True) > 0                                  # planted: sigma2 of the block instead of the row


@pytest.mark.parametrize("typ", [Q4_0, Q5_0, Q5_1], ids=["q4_0", "q5_0", "q5_1"])
def test_imatrix_block_depends_on_its_row(oracle_lib, typ):
    rng = np.random.default_rng(20 + typ)
    x = (rng.standard_normal((64, 96)) * 0.02).astype(np.float32)
    y = x.copy()
    y[:, 32:] *= 3                                          # the rest of each row changed, block 0 kept
    qw = rng.lognormal(0.0, 1.5, 96).astype(np.float32)
    a = oracle_lib.quantize(typ, x, qw).reshape(64, 3, BB[typ])[:, 0]
    b = oracle_lib.quantize(typ, y, qw).reshape(64, 3, BB[typ])[:, 0]
    assert np.any(a != b)
    pa = oracle_lib.quantize(typ, x).reshape(64, 3, BB[typ])[:, 0]
    pb = oracle_lib.quantize(typ, y).reshape(64, 3, BB[typ])[:, 0]
    assert np.array_equal(pa, pb)                           # (the plain rule is block-local)


def test_f16_is_ieee_rounding(oracle_lib):
    rng = np.random.default_rng(3)
    x = np.concatenate([rng.standard_normal(4000) * 10.0 ** rng.uniform(-9, 6, 4000),
                        [0.0, -0.0, 65504.0, 65519.99, 65520.0, 1e9, -1e9, 5.96e-8, 2.98e-8, 2.99e-8, 1e-10,
                         np.inf, -np.inf]]).astype(np.float32)
    x = x[:x.size // 37 * 37].reshape(-1, 37)                   # (rows of 37: any length)
    got = oracle_lib.quantize(F16, x).view(np.uint16).reshape(x.shape)
    with np.errstate(over="ignore"):                            # (values past 65519.99 round to inf)
        assert np.array_equal(got, x.astype(np.float16).view(np.uint16))
    nan = np.array([[np.nan, -np.nan, np.float32(1.0)]], np.float32)
    g = oracle_lib.quantize(F16, nan).view(np.uint16).reshape(-1)
    assert g[0] == 0x7E00 and g[1] == 0xFE00 and g[2] == 0x3C00
