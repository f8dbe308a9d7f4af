"""Re-quantize the tensors of a (split) GGUF that a rules file names, on the MI355X, and copy the rest byte for byte.

    python requant.py <in shard 1> <out dir> <rules file> [--imatrix=<imatrix.gguf>] [--check] [--gpu=N]
                      [--only-matched] [--hessian=<dir> [--damp=0.01] [--damp-iq1=D] [--order=seq|act] [--gated]
                      [--weights=imatrix|diag|schur]] [--allow-synthetic-tables]

This is the plan-and-write part of the reference's tools/requant_experts.py (rules: 171-177; fallback types:
180-192; imatrix normalization: 280-293; the per-shard plan: 420-470; the writer: 471-500) with its quantizer
calls going to libgpuq's host entry point `gpuq_requantize_batch`, which decodes the STORED source bytes (F32, F16,
BF16, Q8_0, MXFP4) on the GPU and quantizes every expert with its own imatrix row. GGUF files are read and written
by gguf_io (no gguf-py). The rules file holds one "<tensor name regex> <type>" a line (# comments); the first rule
whose regex matches anywhere in the name wins.

--hessian=<dir> turns on error-feedback (LDLQ) rounding for the expert tensors the folder has a Hessian for, as the
reference's driver does (tools/requant_experts.py:200-212, 520-600): blk.L.in.npy [n_expert, ne0, ne0] for
ffn_gate/up_exps, blk.L.mid.npy for ffn_down_exps (blk.L.in_g / mid_g with --gated), blk.L.counts.npy the rows
each expert's Hessian summed. Each expert runs libgpuq's whole LDLQ path (gpuq_ldlq: the factor and the loop on the
device); the importance a super-block's quantizer gets is --weights (the imatrix row by default, 'diag' for diag(H)/n
or 'schur'); a tensor without imatrix data, and an expert with fewer than LDLQ_MIN_ROWS (64) rows, are rounded plain
(tools/requant_experts.py:551-552). Sources for it: F32, F16 and BF16 (widened to f32 exactly on the host).

--allow-synthetic-tables: the package's own gpuq_tables.bin holds stand-in IQ1/IQ2/IQ3 codebooks (ggml's are not
part of this repository) and carries a mark that makes libgpuq refuse those types, because llama.cpp would read the
grid indices against ggml's own grids. This flag lifts that refusal for test runs. A gpuq_tables.bin written from
ggml by the reference's gpuq_tables.c needs no flag.

llama-quantize's fallback types for rows that are not whole blocks of the asked type (Q4_0, Q5_0, Q5_1, IQ4_NL, Q8_0,
F16: FALLBACK below) are quantized by libgpuq too, with the tensor's imatrix where ggml takes one; the reference writes
these through ggml on the CPU (tools/requant_experts.py:732-747).

Not here (the reference's other paths): --dump / --dense-dump Hessians, --sub, the CPU quantizer and sources in other
stored types. A tensor that needs one of these stops the run with its name and the reason; nothing falls back to the
CPU.
"""
import os
import re
import sys
import time

import numpy as np

if __package__ in (None, ""):
    sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
import gpuq  # noqa: E402
from gpuq import gguf_io, tables  # noqa: E402

T = gguf_io.TYPE_BY_NAME
# llama-quantize's tensor_type_fallback for rows that are not whole blocks of the asked type
FALLBACK = {T["IQ1_S"]: T["IQ4_NL"], T["IQ1_M"]: T["IQ4_NL"], T["IQ2_XXS"]: T["IQ4_NL"], T["IQ2_XS"]: T["IQ4_NL"],
            T["IQ2_S"]: T["IQ4_NL"], T["IQ3_XXS"]: T["IQ4_NL"], T["IQ3_S"]: T["IQ4_NL"], T["IQ4_XS"]: T["IQ4_NL"],
            T["Q2_K"]: T["Q4_0"], T["Q3_K"]: T["Q4_0"], T["Q4_K"]: T["Q5_0"], T["Q5_K"]: T["Q5_1"],
            T["Q6_K"]: T["Q8_0"]}
# the types ggml refuses to quantize without importance data
NEEDS_IMATRIX = {T["IQ1_S"], T["IQ1_M"], T["IQ2_XXS"], T["IQ2_XS"], T["IQ2_S"]}
SOURCES = (gpuq.F32, gpuq.F16, gpuq.BF16, gpuq.Q8_0, gpuq.MXFP4)   # stored types the library decodes
# types whose quantizer is closed per 256-weight super-block: the LDLQ loop can feed back between super-blocks
LDLQ_TYPES = {T["IQ1_S"], T["IQ1_M"], T["IQ2_XXS"], T["IQ2_XS"], T["IQ2_S"], T["IQ3_XXS"], T["IQ3_S"], T["IQ4_XS"],
              T["Q4_K"], T["Q5_K"], T["Q6_K"]}
MIN_ROWS = int(os.environ.get("LDLQ_MIN_ROWS", 64))   # an expert with fewer calibration rows is rounded plain


class RequantError(RuntimeError):
    pass


def read_rules(path):
    """[(compiled regex, ggml type)] in file order"""
    rules = []
    with open(path, encoding="utf-8") as f:
        for n, line in enumerate(f, 1):
            line = line.split("#", 1)[0].strip()
            if not line:
                continue
            parts = line.rsplit(None, 1)
            if len(parts) != 2 or parts[1].upper() not in T:
                raise RequantError("%s:%d: expected '<regex> <type>', got %r" % (path, n, line))
            rules.append((re.compile(parts[0]), T[parts[1].upper()]))
    return rules


def rule_type(rules, name):
    return next((typ for pat, typ in rules if pat.search(name)), None)


def fit_type(typ, ne0):
    """the type llama-quantize writes for rows of ne0 weights when asked for typ: typ, its fallback, or F16"""
    if ne0 % gguf_io.GGML_TYPES[typ][1] == 0:
        return typ
    fb = FALLBACK.get(typ, typ)
    return fb if ne0 % gguf_io.GGML_TYPES[fb][1] == 0 else T["F16"]


def read_imatrix(path):
    """{tensor name: [rows, ne0] float32}: in_sum2 / counts per row, 1.0 for a row the calibration never reached
    (llama-quantize's normalization; one row per expert)"""
    r = gguf_io.GGUFReader(path)
    sums, counts = {}, {}
    for t in r.tensors:
        if t.name.endswith(".in_sum2"):
            sums[t.name[:-len(".in_sum2")]] = np.asarray(t.f32(), dtype=np.float32)
        elif t.name.endswith(".counts"):
            counts[t.name[:-len(".counts")]] = np.asarray(t.f32(), dtype=np.float32).reshape(-1)
    out = {}
    for name, s in sums.items():
        if name not in counts:
            raise RequantError("%s: %s.in_sum2 without %s.counts" % (path, name, name))
        c = counts[name]
        s = s.reshape(len(c), -1)
        out[name] = np.where(c[:, None] > 0, s / np.maximum(c, 1)[:, None], 1.0).astype(np.float32)
    return out


def shard_paths(shard1):
    """every shard of a split named <prefix>-0000k-of-0000n.gguf, or the one file"""
    m = re.match(r"(.*)-(\d{5})-of-(\d{5})\.gguf$", os.path.basename(shard1))
    if m is None:
        return [shard1]
    d = os.path.dirname(shard1)
    return [os.path.join(d, "%s-%05d-of-%s.gguf" % (m.group(1), i, m.group(3))) for i in range(1, int(m.group(3)) + 1)]


def hess_file(hess_dir, name, gated=False):
    """(Hessian .npy, counts .npy) of an expert tensor, or None when the folder has none for it"""
    m = re.match(r"blk\.(\d+)\.ffn_(gate|up|down)_exps\.weight$", name)
    if m is None:
        return None
    h = os.path.join(hess_dir, "blk.%s.%s%s.npy" % (m.group(1), "mid" if m.group(2) == "down" else "in",
                                                   "_g" if gated else ""))
    c = os.path.join(hess_dir, "blk.%s.counts.npy" % m.group(1))
    return (h, c) if os.path.exists(h) and os.path.exists(c) else None


class Step:
    """one tensor of the plan: kept (new_type None) or re-quantized to new_type, with or without its imatrix rows"""
    __slots__ = ("tensor", "new_type", "nbytes", "imatrix", "note", "hessian")

    def __init__(self, tensor, new_type=None, nbytes=0, imatrix=None, note="", hessian=None):
        self.tensor, self.new_type, self.nbytes, self.imatrix, self.note = tensor, new_type, nbytes, imatrix, note
        self.hessian = hessian          # (Hessian .npy, counts .npy) for error-feedback rounding, or None


TABLE_TYPES = {T["IQ1_S"], T["IQ1_M"], T["IQ2_XXS"], T["IQ2_XS"], T["IQ2_S"], T["IQ3_XXS"], T["IQ3_S"]}


def plan_shard(reader, rules, imat, can_quantize=None, hess=None, can_ldlq=None):
    """the plan of one shard (tools/requant_experts.py:420-470): the rule's type, fitted to the row length; an
    i-quant that needs an imatrix the file does not hold, or one of the wrong shape, leaves the tensor as it is; a
    type that takes one quantizes without it then. can_quantize(type, with_imatrix) -> bool is libgpuq's
    gpuq_can_quantize (None: plan only). hess: {"dir", "gated"} for error-feedback rounding, or None; can_ldlq(type)
    -> bool is libgpuq's gpuq_can_dequantize_type (the loop reads each block back; None: plan only)."""
    plan = []
    for t in reader.tensors:
        typ = rule_type(rules, t.name)
        note = ""
        if typ is not None and len(t.shape) not in (2, 3):
            typ, note = None, "not a matrix: left as is"
        im = None
        if typ is not None:
            ne0, ne1 = t.shape[0], t.shape[1]
            ne2 = t.shape[2] if len(t.shape) == 3 else 1
            fit = fit_type(typ, ne0)
            if fit != typ:
                note = "rows of %d do not fit %s: %s instead (llama-quantize's fallback)" % (
                    ne0, gguf_io.type_name(typ), gguf_io.type_name(fit))
                typ = fit
            im = imat.get(t.name)
            if im is not None and im.shape != (ne2, ne0):
                if typ in NEEDS_IMATRIX:
                    typ, note = None, "imatrix %s does not fit [%d x %d experts]: left as is" % (im.shape, ne0, ne2)
                else:
                    note = "imatrix %s does not fit [%d x %d]: quantized without it" % (im.shape, ne0, ne2)
                im = None
            elif im is None and typ in NEEDS_IMATRIX:
                typ, note = None, "no imatrix data, which %s needs: left as is" % gguf_io.type_name(typ)
        if typ is not None and typ == t.tensor_type:
            typ = None
        if typ is None:
            plan.append(Step(t, note=note))
            continue
        if typ not in gpuq.TYPE_NAMES or (can_quantize is not None and not can_quantize(typ, im is not None)):
            why = ""
            if typ in TABLE_TYPES and os.path.exists(gpuq.tables_path()) and tables.is_synthetic(gpuq.tables_path()):
                why = (" (%s holds the package's stand-in codebooks, refused outside tests: use a table file written "
                       "from ggml, or --allow-synthetic-tables for a test run)" % gpuq.tables_path())
            raise RequantError("%s: libgpuq does not quantize %s%s%s" % (
                t.name, gguf_io.type_name(typ), "" if im is not None else " without an imatrix", why))
        if t.tensor_type not in SOURCES:
            raise RequantError("%s: stored as %s, which libgpuq does not decode (F32, F16, BF16, Q8_0, MXFP4)" % (
                t.name, gguf_io.type_name(t.tensor_type)))
        hf = None
        if hess is not None and len(t.shape) == 3:
            hf = hess_file(hess["dir"], t.name, hess.get("gated", False))
            if hf is not None:
                shp = np.load(hf[0], mmap_mode="r").shape
                why = ("Hessian %s does not fit [%d x %d x %d]" % (shp, t.shape[2], t.shape[0], t.shape[0])
                       if shp != (t.shape[2], t.shape[0], t.shape[0]) else
                       "no imatrix" if im is None else
                       "%s is not rounded per 256-weight super-block" % gguf_io.type_name(typ)
                       if typ not in LDLQ_TYPES or t.shape[0] % 256 else
                       "libgpuq cannot read %s back" % gguf_io.type_name(typ)
                       if can_ldlq is not None and not can_ldlq(typ) else
                       "stored as %s (error feedback reads F32 / F16 / BF16)" % gguf_io.type_name(t.tensor_type)
                       if t.tensor_type not in (gpuq.F32, gpuq.F16, gpuq.BF16) else None)
                if why is not None:
                    note = (note + "; " if note else "") + why + ": plain rounding"
                    hf = None
        plan.append(Step(t, typ, gguf_io.tensor_bytes(typ, t.shape), im, note, hf))
    return plan


def quantize_tensor(gq, step, batch_floats, hess=None):
    """the re-quantized bytes of one tensor: gpuq_requantize_batch over groups of whole experts (source bytes as
    stored, each expert with its own imatrix row)"""
    t = step.tensor
    ne0, ne1 = t.shape[0], t.shape[1]
    ne2 = t.shape[2] if len(t.shape) == 3 else 1
    out = np.empty(step.nbytes, dtype=np.uint8)
    src_mat = t.n_bytes // ne2
    dst_mat = step.nbytes // ne2
    per = max(1, min(ne2, batch_floats // (ne0 * ne1)))
    if step.hessian is not None:
        return quantize_tensor_ldlq(gq, step, hess or {}, out)
    src = np.ascontiguousarray(t.data)        # (a view of the mapped file: read as the library copies it in)
    for e0 in range(0, ne2, per):
        n = min(per, ne2 - e0)
        im = None
        if step.imatrix is not None:
            im = np.ascontiguousarray(step.imatrix[e0:e0 + n], dtype=np.float32)
        got = gq.gpuq_requantize_batch(t.tensor_type, src.ctypes.data + e0 * src_mat, step.new_type,
                                       out.ctypes.data + e0 * dst_mat, n, ne1, ne0,
                                       None if im is None else im.ctypes.data)
        if got != n * dst_mat:
            raise RequantError("%s: gpuq_requantize_batch returned %d bytes for experts %d..%d (%d expected)" % (
                t.name, got, e0, e0 + n - 1, n * dst_mat))
    return out


def quantize_tensor_ldlq(gq, step, hess, out):
    """error-feedback rounding, expert by expert: the expert's Hessian and row count from the folder, the whole LDLQ
    path on the device (gpuq_ldlq), the importance hess["weights"] (the expert's imatrix row by default); plain
    rounding for an expert with fewer than MIN_ROWS rows"""
    from gpuq import ldlq
    t = step.tensor
    ne0, ne1, ne2 = t.shape
    typ = step.new_type
    damp = hess.get("damp", 0.01)
    if hess.get("damp_iq1") is not None and typ in (T["IQ1_S"], T["IQ1_M"]):
        damp = hess["damp_iq1"]
    H_all = np.load(step.hessian[0], mmap_mode="r")
    counts = np.asarray(np.load(step.hessian[1])).reshape(-1)
    weights = hess.get("weights", "imatrix")
    per = t.n_bytes // ne2
    dst = out.reshape(ne2, -1)
    for e in range(ne2):
        n = float(counts[e])
        w = np.ascontiguousarray(gguf_io.widen(t.tensor_type, t.data[e * per:(e + 1) * per], t.name).reshape(ne1, ne0))
        im = np.ascontiguousarray(step.imatrix[e], dtype=np.float32)
        if n < MIN_ROWS:
            got = gq.gpuq_quantize(typ, w.ctypes.data, dst[e].ctypes.data, ne1, ne0, im.ctypes.data)
            if got != dst.shape[1]:
                raise RequantError("%s: gpuq_quantize failed for expert %d" % (t.name, e))
            continue
        H = np.asarray(H_all[e], dtype=np.float64)
        try:
            dst[e] = ldlq.quantize_matrix_host(gq, typ, w, H, n, im, damp=damp, order=hess.get("order", "seq"),
                                               weights=weights).reshape(-1)
        except RuntimeError as err:
            raise RequantError("%s, expert %d: %s" % (t.name, e, err)) from err
    return out


def write_shard(path, reader, plan, gq, batch_floats, only_matched=False, kv_src=None, log=print, hess=None):
    """the output GGUF: the source's key/values as stored (kv_src's for only_matched, split keys dropped), then
    every tensor of the plan in the source's order, re-quantized or copied"""
    steps = [s for s in plan if s.new_type is not None] if only_matched else plan
    w = gguf_io.GGUFWriter(path, alignment=reader.alignment)
    for kv in (kv_src or reader).fields.values():
        if only_matched and kv.name.startswith("split."):
            continue
        w.add_raw_kv(kv)
    for s in steps:
        w.add_tensor_info(s.tensor.name, s.tensor.shape, s.new_type if s.new_type is not None else s.tensor.tensor_type)
    with w:
        w.write_header()
        for s in steps:
            if s.new_type is None:
                w.write_tensor_data(s.tensor.data)
            else:
                t0 = time.time()
                w.write_tensor_data(quantize_tensor(gq, s, batch_floats, hess))
                log("  %-34s %s -> %s%s  %.2f s" % (s.tensor.name, gguf_io.type_name(s.tensor.tensor_type),
                                                    gguf_io.type_name(s.new_type),
                                                    " (error feedback)" if s.hessian else "", time.time() - t0))


def run(shard1, out_dir, rules_path, imatrix_path=None, check=False, device=0, only_matched=False, gq=None,
        log=print, hess=None):
    """re-quantize every shard; returns (source bytes, output bytes) of the re-quantized tensors"""
    rules = read_rules(rules_path)
    imat = read_imatrix(imatrix_path) if imatrix_path else {}
    if gq is None and not check:
        gq = gpuq.load_gpuq(device)
    can = None if gq is None else (lambda typ, with_im: gq.gpuq_can_quantize(typ, 1 if with_im else 0) == 1)
    can_ldlq = None if gq is None else (lambda typ: gq.gpuq_can_dequantize_type(typ) == 1)
    batch_floats = int(os.environ.get("GPUQ_BATCH_MB", "2048")) << 20
    paths = shard_paths(shard1)
    if not check:
        os.makedirs(out_dir, exist_ok=True)
    first = gguf_io.GGUFReader(paths[0]) if os.path.isfile(paths[0]) else None
    old = new = 0
    for sh in paths:
        if not os.path.isfile(sh):
            log("%s is not there: skipped" % sh)
            continue
        r = first if sh == paths[0] else gguf_io.GGUFReader(sh)
        out = os.path.join(out_dir, os.path.basename(sh))
        log("%s -> %s" % (sh, out))
        plan = plan_shard(r, rules, imat, can, hess, can_ldlq)
        for s in plan:
            if s.note:
                log("  %s: %s" % (s.tensor.name, s.note))
            if s.new_type is not None:
                old += s.tensor.n_bytes
                new += s.nbytes
                log("  %-34s %-7s %8.3f GiB -> %-7s %8.3f GiB" % (
                    s.tensor.name, gguf_io.type_name(s.tensor.tensor_type), s.tensor.n_bytes / 2**30,
                    gguf_io.type_name(s.new_type), s.nbytes / 2**30))
        if check:
            continue
        if only_matched and not any(s.new_type is not None for s in plan):
            log("  nothing re-quantized in this shard: no file (--only-matched)")
            continue
        write_shard(out, r, plan, gq, batch_floats, only_matched, first if only_matched else None, log, hess)
    log("re-quantized tensors: %.3f GiB -> %.3f GiB" % (old / 2**30, new / 2**30))
    return old, new


def main(argv=None):
    argv = sys.argv[1:] if argv is None else argv
    flags = [a for a in argv if a.startswith("--")]
    args = [a for a in argv if not a.startswith("--")]
    known = ("--imatrix=", "--gpu=", "--check", "--only-matched", "--hessian=", "--damp=", "--damp-iq1=",
             "--order=", "--gated", "--weights=", "--allow-synthetic-tables")
    bad = [f for f in flags if not f.startswith(known)]
    if len(args) != 3 or bad:
        print(__doc__.split("\n\n")[1], file=sys.stderr)
        if bad:
            print("not supported here: %s" % " ".join(bad), file=sys.stderr)
        return 2
    imat = next((f.split("=", 1)[1] for f in flags if f.startswith("--imatrix=")), None)
    dev = int(next((f.split("=", 1)[1] for f in flags if f.startswith("--gpu=")), "0"))
    opt = {f.split("=", 1)[0]: f.split("=", 1)[1] for f in flags if "=" in f}
    hess = None
    if "--hessian" in opt:
        hess = {"dir": opt["--hessian"], "damp": float(opt.get("--damp", 0.01)), "gated": "--gated" in flags,
                "damp_iq1": float(opt["--damp-iq1"]) if "--damp-iq1" in opt else None,
                "order": opt.get("--order", "seq"), "weights": opt.get("--weights", "imatrix")}
        if hess["order"] not in ("seq", "act"):
            print("--order is seq or act", file=sys.stderr)
            return 2
        if hess["weights"] not in ("imatrix", "diag", "schur"):
            print("--weights is imatrix, diag or schur", file=sys.stderr)
            return 2
    if "--allow-synthetic-tables" in flags:
        os.environ["GPUQ_ALLOW_SYNTHETIC_TABLES"] = "1"
    try:
        run(args[0], args[1], args[2], imat, "--check" in flags, dev, "--only-matched" in flags, hess=hess)
    except (RequantError, RuntimeError, OSError) as e:
        print("error: %s" % e, file=sys.stderr)
        return 1
    return 0


if __name__ == "__main__":
    sys.exit(main())
