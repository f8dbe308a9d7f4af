#!/usr/bin/env python3
"""bench.py - throughput of the MI355X GGUF quantizer on the configured synthetic workloads.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-host] [--only NAME,...] [--experts N]
    python bench.py --only experts16      (not in the default run: five search types on 16 BF16 experts)

One "step" is one pass of the quantizer over one workload tensor already resident in HBM (the device entry point
gpuq_requantize_dev: source bytes decoded in registers, quantized, blocks written to HBM). The headline line is
IQ2_XXS with imatrix on 256 stacked BF16 experts of 2048 x 7168 (expert e ~ N(0, s_e), s_e ~ U[0.01, 0.03], a
log-normal(0, 1.5) imatrix a expert). `per_type` adds Q8_0 on a 4096 x 4096 F32 tensor (and on 64 of them, 4.3 GB, where launch
and ramp time no longer weigh), Q4_K and Q6_K on a
2048 x 7168 BF16 tensor (N(0, 0.02) plus 0.1% outliers at +-8 sigma, a log-normal imatrix), IQ1_S / IQ1_M on 384 x
2048 x 7168 MXFP4 experts, IQ2_S with LDLQ error feedback on 64 BF16 experts, and ggml's to_float of the headline's own
IQ2_XXS blocks (gpuq_dequantize_dev, 16 experts' worth, HBM-bound); `other_types` the remaining nine
types on the 2048 x 7168 tensor (GPU rate, roofline, byte spot check on 64 rows). `--only experts16` runs Q3_K,
IQ2_XS, IQ2_S, IQ3_XXS and IQ3_S on 16 of the BF16 experts: launches long enough that neither the tile queue's last
round (that tensor gives 2,048 resident waves 3.5 tiles each) nor the write-back of each resident wave's register
spill area, once a launch, weighs on the rate or the traffic. Kernel time comes from HIP events
on the launch stream; inputs that fit the 256 MB Infinity Cache are rotated over enough copies that every launch
reads HBM.

Each entry carries a roofline and a CPU baseline:
- roofline: HBM bytes for Q8_0 against 8 TB/s; for the searches, the sequential algorithm's VALU operations (each
  add, mul, compare, select, convert one; the oracle's op-counting build run on a sample of the same tensor) against
  78.6 T operations/s, MI355X's published FP32 vector peak of 157.3 TFLOP/s counted per instruction (an FMA is two
  flops): two wave64 VALU instructions per SIMD per four clocks, 1,024 SIMDs, 2.4 GHz. `traffic` (HBM bytes a launch)
  and `valu_issue` (instructions issued per SIMD per clock, rocprof's VALUBusy) come from the committed rocprofv3
  counter summaries under profiles/;
- cpu_baseline: the oracle (a C restatement of ggml_quantize_chunk, -O2 without FMA) on all the host cores this
  process may use, timed on a bounded sample of the same tensor whose bytes are also compared with the GPU's; for
  LDLQ the reference's CPU loop order (numpy LU solve and BLAS product a block, tools/ldlq.py:103-106, one expert a
  thread) around the oracle's quantizer.
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "trench-gguf_amd"))
sys.path.insert(0, os.path.join(ROOT, "oracle"))

METRIC = "Mweights/s per type (Q8_0, Q4_K, IQ2_XXS, IQ1_M) on 1 MI355X; % VALU/HBM peak"
HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, GB/s
VALU_PEAK_TOPS = 78.6          # 157.3 TFLOP/s FP32 vector / 2 flops an FMA: 2 wave64 instr / SIMD / 4 clk, 2.4 GHz
FP64_PEAK_TFLOPS = 78.6        # MI355X FP64 (vector and matrix)
MALL_BYTES = 256 << 20         # Infinity Cache
CPU_MIN_S = 10.0               # the CPU baseline repeats its sample until this much CPU time has run
ENTRIES = ["IQ2_XXS", "Q8_0", "Q8_0_large", "Q4_K", "Q6_K", "IQ1_S", "IQ1_M", "LDLQ", "other", "experts16"]
OTHER = ["Q2_K", "Q3_K", "Q5_K", "IQ4_NL", "IQ4_XS", "IQ2_XS", "IQ2_S", "IQ3_XXS", "IQ3_S"]
EXPERTS16 = ["Q3_K", "IQ2_XS", "IQ2_S", "IQ3_XXS", "IQ3_S"]     # (run only when asked for: --only experts16)


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def profile_value(fname, tag, key):
    """the value of a line `<tag>[<key>] = <value>` in profiles/<fname> (a committed rocprofv3 summary), or None"""
    try:
        with open(os.path.join(ROOT, "profiles", fname)) as f:
            for line in f:
                line = line.strip().strip("`")
                if line.startswith("%s[%s] = " % (tag, key)):
                    return line.split("=", 1)[1].strip()
    except OSError:
        pass
    return None


KEY_SUFFIX = ""        # appended to the profile keys of a run on other tables than the regular ones


def pmc_traffic(key):
    """HBM bytes a launch from rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE on this workload, scaled by the same counters'
    reading for a copy kernel of known size (profiles/hbm_traffic_pmc.md), or None when not measured"""
    v = profile_value("hbm_traffic_pmc.md", "traffic", key)
    return None if v is None else int(v)


def pmc_valu(key):
    """{issue_per_simd_clk, valu_busy_pct, lane_util} from profiles/valu_counters_pmc.md, or None"""
    v = profile_value("valu_counters_pmc.md", "valu", key)
    if v is None:
        return None
    issue, busy, util = v.split()
    return {"issue_per_simd_clk": float(issue), "valu_busy_pct": float(busy), "lane_util": float(util),
            "source": "profiles/valu_counters_pmc.md"}


def cpu_threads():
    try:
        return max(1, min(len(os.sched_getaffinity(0)), 64))
    except AttributeError:
        return os.cpu_count() or 1


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


class Workload:
    """a synthetic tensor in HBM (source bytes, imatrix) plus its host-side sample for the CPU leg"""

    def __init__(self, name, key, src, nmat, nrow, ncol, raw, imatrix):
        self.name, self.key, self.src, self.nmat, self.nrow, self.ncol = name, key, src, nmat, nrow, ncol
        self.raw, self.imatrix = raw, imatrix
        self.n = nmat * nrow * ncol


def make_f32(torch, gen, shape, sigma):
    return (torch.randn(shape, device="cuda", generator=gen) * sigma).contiguous()


def wl_c1(torch, gpuq):
    g = torch.Generator(device="cuda").manual_seed(0)
    x = make_f32(torch, g, (4096, 4096), 0.02)
    return Workload("F32 4096x4096 N(0,0.02), seed 0", "F32 4096x4096", gpuq.F32, 1, 4096, 4096, x, None)


def wl_q8_large(torch, gpuq, nmat=64):
    """Q8_0's streaming rate away from launch and ramp time: nmat F32 matrices of 4096 x 4096 (4.3 GB at 64)"""
    g = torch.Generator(device="cuda").manual_seed(4)
    x = torch.empty((nmat, 4096, 4096), dtype=torch.float32, device="cuda")
    for e in range(0, nmat, 8):
        x[e:e + 8] = torch.randn((min(8, nmat - e), 4096, 4096), device="cuda", generator=g) * 0.02
    return Workload("F32 %dx4096x4096 N(0,0.02), seed 4" % nmat, "F32 %dx4096x4096" % nmat, gpuq.F32, nmat, 4096,
                    4096, x.reshape(-1), None)


def wl_c2(torch, gpuq):
    g = torch.Generator(device="cuda").manual_seed(1)
    x = make_f32(torch, g, (2048, 7168), 0.02).reshape(-1)
    nout = x.numel() // 1000                                     # 0.1% outliers at +-8 sigma
    pos = torch.randperm(x.numel(), device="cuda", generator=g)[:nout]
    sgn = torch.randint(0, 2, (nout,), device="cuda", generator=g).float() * 2 - 1
    x[pos] = sgn * 0.16
    raw = x.to(torch.bfloat16).contiguous()                       # RNE to BF16
    im = torch.exp(torch.randn(1, 7168, device="cuda", generator=g) * 1.5).contiguous()
    return Workload("BF16 2048x7168 N(0,0.02) + 0.1% outliers at +-8 sigma, log-normal(0,1.5) imatrix",
                    "BF16 2048x7168", gpuq.BF16, 1, 2048, 7168, raw, im)


def wl_c3(torch, gpuq, nexp=256):
    g = torch.Generator(device="cuda").manual_seed(2)
    sig = torch.rand(nexp, 1, 1, device="cuda", generator=g) * 0.02 + 0.01
    raw = torch.empty((nexp, 2048, 7168), dtype=torch.bfloat16, device="cuda")
    for e in range(0, nexp, 16):                                  # (bounded temporaries)
        raw[e:e + 16] = (torch.randn((min(16, nexp - e), 2048, 7168), device="cuda", generator=g)
                         * sig[e:e + 16]).to(torch.bfloat16)
    im = torch.exp(torch.randn(nexp, 7168, device="cuda", generator=g) * 1.5).contiguous()
    return Workload("BF16 %dx2048x7168 experts, N(0, s_e), s_e ~ U[0.01,0.03], per-expert log-normal(0,1.5) imatrix"
                    % nexp, "BF16 %dx2048x7168" % nexp, gpuq.BF16, nexp, 2048, 7168, raw.reshape(-1), im)


def wl_c4(torch, gpuq, nexp=384):
    g = torch.Generator(device="cuda").manual_seed(3)
    nblk = nexp * 2048 * 7168 // 32
    raw = torch.randint(0, 256, (nblk, 17), dtype=torch.uint8, device="cuda", generator=g)
    raw[:, 0] = (127 + torch.randint(-8, -3, (nblk,), device="cuda", generator=g)).to(torch.uint8)
    im = torch.exp(torch.randn(nexp, 7168, device="cuda", generator=g) * 1.5).contiguous()
    return Workload("MXFP4 %dx2048x7168 experts, e8m0 exponents U{-8..-4}, uniform e2m1 codes, per-expert "
                    "log-normal(0,1.5) imatrix" % nexp, "MXFP4 %dx2048x7168" % nexp, gpuq.MXFP4, nexp, 2048, 7168,
                    raw.reshape(-1), im)


def wl_c5(torch, gpuq, ldlq, nexp=64, ncal=8192):
    """64 BF16 experts of 2048 x 7168, N(0, 0.02); each with its own SPD Hessian H = X^T X / n + 1e-2 mean(diag) I
    from X [8192 x 7168] of Student-t (nu = 4) activations, factored with prepare_hessian(H, n=1, damp=0.01, seq)
    and a log-normal(0, 1.5) imatrix (IQ2_S needs one)"""
    ne1, ne0 = 2048, 7168
    g = torch.Generator(device="cuda").manual_seed(5)
    W = (torch.randn((nexp, ne1, ne0), device="cuda", generator=g) * 0.02).to(torch.bfloat16).float().contiguous()
    Us = torch.empty((nexp, ne0, ne0), dtype=torch.float64, device="cuda")
    perm = None
    for e in range(nexp):
        z = torch.randn((ncal, ne0), device="cuda", generator=g)
        chi = (torch.randn((4, ncal, ne0), device="cuda", generator=g) ** 2).sum(0) / 4
        X = z / torch.sqrt(chi)
        H = (X.T @ X).double() / ncal
        H.diagonal().add_(1e-2 * float(torch.diagonal(H).mean()))
        U, perm, _, _ = ldlq.prepare_hessian_torch(H, 1, damp=0.01, order="seq")
        Us[e] = U
        del z, chi, X, H, U
    im = torch.exp(torch.randn(nexp, ne0, device="cuda", generator=g) * 1.5).contiguous()
    return W, Us, perm, im


def blas_ldlq_rows(orc, typ, Wp, U, qw):
    """the reference's CPU loop (tools/ldlq.py:71-107) in numpy's order on permuted rows Wp [rows, ne0]: the oracle
    quantizes and reads back each block, np.linalg.solve gives E U_BB^-1, a BLAS product the update. Returns the
    bytes of each permuted block"""
    Wp = Wp.copy()
    rows, ne0 = Wp.shape
    nblk = ne0 // 256
    out = []
    for k in range(nblk):
        cols = slice(256 * k, 256 * (k + 1))
        blk = np.ascontiguousarray(Wp[:, cols])
        raw = orc.quantize(typ, blk, qw[cols])
        out.append(raw)
        if k + 1 < nblk:
            q = orc.dequantize(typ, raw, rows * 256).reshape(rows, 256)
            Es = np.linalg.solve(U[cols, cols].T, (blk - q).T).T
            Wp[:, 256 * (k + 1):] -= (Es @ U[cols, 256 * (k + 1):]).astype(np.float32)
    return out


def bench_ldlq(torch, gq, gpuq, orc, steps, want_cpu, nexp):
    """IQ2_S with LDLQ error feedback over 64 experts; one step = the whole loop (gpuq_ldlq_dev)"""
    from gpuq import ldlq
    t0 = time.time()
    W, Us, perm, im = wl_c5(torch, gpuq, ldlq, nexp)
    log("LDLQ workload ready in %.1f s" % (time.time() - t0))
    nexp_, ne1, ne0 = W.shape
    slots = np.ascontiguousarray(ldlq.slot_order(perm), dtype=np.int64)
    pt = torch.as_tensor(perm, device="cuda")
    Wp0 = W.index_select(2, pt).contiguous()
    qw = im.index_select(1, pt).contiguous()
    tsize = gq.gpuq_block_bytes(gpuq.IQ2_S)
    out = torch.empty((nexp_, ne1, ne0 // 256 * tsize), dtype=torch.uint8, device="cuda")
    stream = torch.cuda.current_stream()
    times = []
    for it in range(steps + 1):
        Wp = Wp0.clone()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        got = gq.gpuq_ldlq_dev(gpuq.IQ2_S, Wp.data_ptr(), Us.data_ptr(), ne0 * ne0, qw.data_ptr(), nexp_, ne1, ne0,
                               slots.ctypes.data, 1, out.data_ptr(), stream.cuda_stream)
        e1.record(stream)
        torch.cuda.synchronize()
        if got != out.numel():
            raise RuntimeError("gpuq_ldlq_dev failed")
        if it:                                            # (the first call is the warm-up)
            times.append(e0.elapsed_time(e1))
        del Wp
    ms = sum(times) / len(times)
    n = nexp_ * ne1 * ne0
    flops = 2.0 * nexp_ * ne1 * 256 * sum(ne0 - 256 * (k + 1) for k in range(ne0 // 256))
    e = {"workload": "IQ2_S with LDLQ error feedback (seq order, imatrix weights), %d BF16 experts of 2048x7168, "
                     "per-expert H from 8192 Student-t(4) activations" % nexp_,
         "value": round(n / (ms / 1e3) / 1e6, 1), "unit": "Mweights/s", "ms_per_step": round(ms, 2),
         "steps": steps,
         "roofline": {"bound": "fp64", "achieved": round(flops / (ms / 1e3) / 1e12, 2), "peak": FP64_PEAK_TFLOPS,
                      "unit": "TFLOP/s", "frac": round(flops / (ms / 1e3) / 1e12 / FP64_PEAK_TFLOPS, 4),
                      "traffic": None, "algorithmic_flops_per_step": flops,
                      "note": "the update's f64 flops over the whole loop's time (quantize + solve + update)"}}
    # byte check: rows are independent in the loop, so rows of expert 0 through the oracle's fixed-order loop are
    # exact; the CPU baseline: the reference's CPU loop order, one expert's row sample a thread
    nthr = cpu_threads()
    check_rows = 16
    U0 = Us[0].cpu().numpy()
    qw_h = qw.cpu().numpy()
    want = orc.ldlq(gpuq.IQ2_S, Wp0[0:1, :check_rows].cpu().numpy(), U0, qw_h[0:1], slots)[0]
    e["sample_identical_to_oracle"] = bool(np.array_equal(out[0:1, :check_rows].cpu().numpy(), want))
    if want_cpu:
        import concurrent.futures
        from threadpoolctl import threadpool_limits
        nexp_s = min(nexp_, nthr)
        Uh = [U0] + [Us[i].cpu().numpy() for i in range(1, nexp_s)]

        def cpu_pass(rows):
            Ws = [Wp0[i, :rows].cpu().numpy() for i in range(nexp_s)]
            t0 = time.time()
            with threadpool_limits(limits=1), concurrent.futures.ThreadPoolExecutor(nthr) as ex:
                res = list(ex.map(lambda i: blas_ldlq_rows(orc, gpuq.IQ2_S, Ws[i], Uh[i], qw_h[i]), range(nexp_s)))
            return res, time.time() - t0
        rows = 32
        parts, cpu_s = cpu_pass(rows)
        if cpu_s < CPU_MIN_S:                     # (a sample of about CPU_MIN_S: a stable rate)
            rows = int(min(ne1, max(rows, rows * CPU_MIN_S / max(cpu_s, 1e-3))) // 16 * 16)
            parts, cpu_s = cpu_pass(rows)
        same = []
        gpu_h = out[:nexp_s, :rows].cpu().numpy().reshape(nexp_s, rows, ne0 // 256, tsize)
        for i, blocks in enumerate(parts):
            for k, b in enumerate(blocks):
                same.append((gpu_h[i][:, slots[k]] == b).all(axis=1))
        share = float(np.concatenate(same).mean())
        e["cpu_baseline"] = {"value": round(nexp_s * rows * ne0 / cpu_s / 1e6, 3), "unit": "Mweights/s",
                             "cores": nthr, "cpu": cpu_model(), "kind": "port",
                             "sample": "%d experts x %d rows (the loop's rows are independent), one expert a thread, "
                                       "numpy LU solve + BLAS product a block (1 BLAS thread each) around the oracle's "
                                       "IQ2_S quantizer and reader, %.1f s" % (nexp_s, rows, cpu_s)}
        e["cpu_loop_identical_superblocks"] = round(share, 4)
        e["speedup_vs_cpu"] = round(e["value"] / e["cpu_baseline"]["value"], 1)
    del W, Us, Wp0, out
    torch.cuda.empty_cache()
    return e


_sleep_per_ms = []


def hold_gpu(torch, ms):
    """keep the current stream busy for about `ms` (torch's spin kernel, calibrated once), so that launches timed
    after it run back to back instead of waiting for the host to issue each (a Q8_0 launch takes ~20 us)"""
    if not _sleep_per_ms:
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda._sleep(1000)
        e0.record()
        torch.cuda._sleep(1 << 20)
        e1.record()
        torch.cuda.synchronize()
        _sleep_per_ms.append((1 << 20) / max(e0.elapsed_time(e1), 1e-3))
    torch.cuda._sleep(int(ms * _sleep_per_ms[0]))


def time_gpu(torch, gq, gpuq, wl, typ, steps, warmup):
    """average kernel time (ms) of gpuq_requantize_dev over `steps` launches, HIP events on the launch stream"""
    bpw = {gpuq.F32: 4.0, gpuq.BF16: 2.0, gpuq.MXFP4: 17 / 32}[wl.src]
    in_bytes = wl.n * bpw
    copies = 1
    if in_bytes < 2 * MALL_BYTES:                                 # rotate copies so each launch reads HBM
        copies = int(2 * MALL_BYTES // in_bytes) + 1
    raws = [wl.raw] + [wl.raw.clone() for _ in range(copies - 1)]
    out_bytes = wl.n // gpuq.BLOCK[typ] * gq.gpuq_block_bytes(typ)
    outs = [torch.empty(out_bytes, dtype=torch.uint8, device="cuda") for _ in range(min(copies, 4))]
    stream = torch.cuda.current_stream()
    im = None if (wl.imatrix is None or typ == gpuq.Q8_0) else wl.imatrix.data_ptr()

    def launch(i):
        got = gq.gpuq_requantize_dev(wl.src, raws[i % copies].data_ptr(), typ, outs[i % len(outs)].data_ptr(),
                                     wl.nmat, wl.nrow, wl.ncol, im, stream.cuda_stream)
        if got != out_bytes:
            raise RuntimeError("gpuq_requantize_dev failed for %s" % gpuq.TYPE_NAMES[typ])

    for i in range(warmup):
        launch(i)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    hold_gpu(torch, 2.0 + 0.05 * steps)     # the host enqueues every timed launch before the GPU reaches e0
    e0.record(stream)
    for i in range(steps):
        launch(warmup + i)
    e1.record(stream)
    if e0.query():
        log("note: the GPU reached the timed launches before the host had enqueued them all")
    torch.cuda.synchronize()
    if gq.gpuq_take_error():
        raise RuntimeError("a search reported no candidate (%s)" % gpuq.TYPE_NAMES[typ])
    ms = e0.elapsed_time(e1) / steps
    result = outs[(warmup + steps - 1) % len(outs)]
    del raws[1:]
    return ms, result


def bench_to_float(torch, gq, gpuq, orc, q, typ, nblk, steps, warmup):
    """gpuq_dequantize_dev (ggml's to_float) over nblk blocks already in HBM (the quantizer's own output), HIP events
    on the launch stream: HBM bytes (blocks read, f32 written) against 8 TB/s and a device copy of as many bytes; the
    first 64 blocks' values against the oracle's to_float, bit for bit"""
    bb = gq.gpuq_block_bytes(typ)
    qv = q[: nblk * bb]
    # the blocks rotated over copies (twice the 256 MB Infinity Cache between two reads of one copy), so every launch
    # reads them from HBM as the output goes to it
    srcs = [qv] + [qv.clone() for _ in range(max(0, -(-2 * MALL_BYTES // (nblk * bb)) - 1))]
    outs = [torch.empty(nblk * 256, dtype=torch.float32, device="cuda") for _ in range(2)]
    stream = torch.cuda.current_stream()

    def launch(i):
        src = srcs[i % len(srcs)]
        if gq.gpuq_dequantize_dev(typ, src.data_ptr(), outs[i % 2].data_ptr(), nblk, stream.cuda_stream) != nblk * 1024:
            raise RuntimeError("gpuq_dequantize_dev failed for %s" % gpuq.TYPE_NAMES[typ])

    for i in range(warmup):
        launch(i)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    hold_gpu(torch, 2.0 + 0.05 * steps)
    e0.record(stream)
    for i in range(steps):
        launch(warmup + i)
    e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    got = outs[(warmup + steps - 1) % 2][: 64 * 256].cpu().numpy()
    want = orc.dequantize(typ, qv[: 64 * bb].cpu().numpy(), 64 * 256)
    nbytes = nblk * bb + nblk * 256 * 4
    achieved = nbytes / (ms / 1e3) / 1e9
    copy_gbs = copy_reference(torch, nbytes)
    return {"workload": "%s blocks of %d BF16 experts of 2048x7168 (the headline's output) -> f32" %
                        (gpuq.TYPE_NAMES[typ], nblk // (2048 * 7168 // 256)),
            "entry_point": "gpuq_dequantize_dev", "value": round(nblk * 256 / (ms / 1e3) / 1e6, 1),
            "unit": "Mweights/s", "ms_per_step": round(ms, 4), "steps": steps, "source_copies": len(srcs),
            "sample_identical_to_oracle": bool(np.array_equal(got.view(np.uint32), want.view(np.uint32))),
            "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(achieved / HBM_PEAK_GBS, 4), "algorithmic_bytes": nbytes,
                         "traffic": pmc_traffic("IQ2_XXS to_float 16x2048x7168"),
                         "device_copy_same_bytes_GBps": round(copy_gbs, 1),
                         "frac_of_device_copy": round(achieved / copy_gbs, 4)}}


def copy_reference(torch, total_bytes, steps=20):
    """GB/s of a torch device copy that moves `total_bytes` (half read, half written), timed as time_gpu times a
    kernel (HIP events, sources rotated past the Infinity Cache): what a plain streaming kernel of that size reaches"""
    half = int(total_bytes // 2)
    copies = int(2 * MALL_BYTES // half) + 1
    srcs = [torch.empty(half, dtype=torch.uint8, device="cuda").fill_(1) for _ in range(copies)]
    dsts = [torch.empty(half, dtype=torch.uint8, device="cuda") for _ in range(min(copies, 4))]
    for i in range(3):
        dsts[i % len(dsts)].copy_(srcs[i % copies])
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    hold_gpu(torch, 2.0 + 0.05 * steps)
    e0.record(stream)
    for i in range(steps):
        dsts[i % len(dsts)].copy_(srcs[i % copies])
    e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    del srcs, dsts
    return 2 * half / (ms / 1e3) / 1e9


def host_api(torch, gq, gpuq, wl, typ, nmat, dev_out, reps=3):
    """PCIe-inclusive rate of the host entry point gpuq_requantize_batch on the first `nmat` matrices of the workload:
    source bytes in pageable host memory, blocks back into host memory (copies overlapped with the kernels); its bytes
    must equal the device entry point's"""
    u8 = wl.raw.view(torch.uint8).reshape(-1)
    per_src = u8.numel() // wl.nmat
    raw = u8[:nmat * per_src].cpu().numpy()
    im = None if wl.imatrix is None else np.ascontiguousarray(wl.imatrix[:nmat].cpu().numpy())
    per_out = wl.nrow * wl.ncol // gpuq.BLOCK[typ] * gq.gpuq_block_bytes(typ)
    out = np.empty(nmat * per_out, dtype=np.uint8)

    def call():
        got = gq.gpuq_requantize_batch(wl.src, raw.ctypes.data, typ, out.ctypes.data, nmat, wl.nrow, wl.ncol,
                                       None if im is None else im.ctypes.data)
        if got != out.nbytes:
            raise RuntimeError("gpuq_requantize_batch failed for %s" % gpuq.TYPE_NAMES[typ])
    call()                                                        # (grows the staging buffers)
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        call()
        ts.append(time.perf_counter() - t0)
    ms = 1e3 * sorted(ts)[len(ts) // 2]
    same = bool(np.array_equal(out, dev_out.reshape(-1)[:out.nbytes].cpu().numpy()))
    nw = nmat * wl.nrow * wl.ncol
    return {"entry_point": "gpuq_requantize_batch", "matrices": nmat, "value": round(nw / (ms / 1e3) / 1e6, 1),
            "unit": "Mweights/s", "ms_per_call": round(ms, 3), "calls": reps,
            "host_bytes_in": int(raw.nbytes), "host_bytes_out": int(out.nbytes),
            "identical_to_device_entry_point": same}


def host_sample(torch, wl, rows):
    """the first `rows` rows of every sampled matrix as host source bytes (the exact bytes the GPU read)"""
    per_row = {0: 4, 30: 2}.get(wl.src)
    if per_row is not None:
        b = wl.raw.reshape(-1).view(torch.uint8)
        return b[: rows * wl.ncol * per_row].cpu().numpy()
    return wl.raw.reshape(-1)[: rows * wl.ncol // 32 * 17].cpu().numpy()


def cpu_and_roofline(torch, gq, gpuq, orc, orc_ops, wl, typ, ms, out_dev, sample_rows, want_cpu):
    """the CPU baseline on a sample, the op count per weight, and a byte spot check of the GPU output"""
    nthr = cpu_threads()
    raw = host_sample(torch, wl, sample_rows)
    n = sample_rows * wl.ncol
    im = None
    if wl.imatrix is not None and typ != gpuq.Q8_0:
        nm = (sample_rows + wl.nrow - 1) // wl.nrow
        im = wl.imatrix[:nm].cpu().numpy()
    nmat_s, nrow_s = (sample_rows // wl.nrow, wl.nrow) if sample_rows >= wl.nrow else (1, sample_rows)
    entry = {}
    # byte spot check: the GPU's blocks of the sampled rows against the oracle's
    rb = wl.ncol // gpuq.BLOCK[typ] * gq.gpuq_block_bytes(typ)
    t0 = time.time()
    want = orc.requantize_mt(wl.src, raw, typ, nmat_s, nrow_s, wl.ncol, im, unit_rows=16, nthreads=nthr)
    cpu_s = time.time() - t0
    got = out_dev[: sample_rows * rb].cpu().numpy()
    entry["sample_identical_to_oracle"] = bool(np.array_equal(got, want))
    if want_cpu:
        passes = 1
        while cpu_s < CPU_MIN_S and passes < 10000:            # (at least CPU_MIN_S of CPU work: a stable rate)
            t0 = time.time()
            orc.requantize_mt(wl.src, raw, typ, nmat_s, nrow_s, wl.ncol, im, unit_rows=16, nthreads=nthr)
            cpu_s += time.time() - t0
            passes += 1
        entry["cpu_baseline"] = {"value": round(passes * n / cpu_s / 1e6, 2), "unit": "Mweights/s", "cores": nthr,
                                 "cpu": cpu_model(), "kind": "port",
                                 "sample": "%d rows x %d of the same tensor (%.1f M weights), %d passes, %.1f s on %d "
                                           "threads" % (sample_rows, wl.ncol, n / 1e6, passes, cpu_s, nthr)}
    # roofline (the counters in profiles/ are for the regular tables only)
    key = "%s %s%s" % (gpuq.TYPE_NAMES[typ], wl.key, KEY_SUFFIX)
    traffic = pmc_traffic(key)
    if typ == gpuq.Q8_0:
        bpw = {0: 4.0, 30: 2.0}.get(wl.src, 17 / 32) + 34 / 32
        achieved = bpw * wl.n / (ms / 1e3) / 1e9
        copy_gbs = copy_reference(torch, bpw * wl.n)
        entry["roofline"] = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                             "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                             "algorithmic_bytes_per_weight": bpw, "algorithmic_bytes": round(bpw * wl.n),
                             "device_copy_same_bytes_GBps": round(copy_gbs, 1),
                             "frac_of_device_copy": round(achieved / copy_gbs, 4)}
    else:
        ops_rows = min(sample_rows, 64)
        sub = raw[: (ops_rows * wl.ncol) * {0: 4, 30: 2}.get(wl.src, 0)] if wl.src in (0, 30) else \
            raw[: ops_rows * wl.ncol // 32 * 17]
        f = orc_ops.decode_src(wl.src, sub, ops_rows * wl.ncol).reshape(ops_rows, wl.ncol)
        orc_ops.ops_read_reset()
        orc_ops.quantize(typ, f, None if im is None else im[0])
        opw = orc_ops.ops_read_reset() / (ops_rows * wl.ncol)
        achieved = opw * wl.n / (ms / 1e3) / 1e12
        entry["roofline"] = {"bound": "valu", "achieved": round(achieved, 3), "peak": VALU_PEAK_TOPS,
                             "unit": "Tops/s", "frac": round(achieved / VALU_PEAK_TOPS, 4), "traffic": traffic,
                             "algorithmic_ops_per_weight": round(opw, 1)}
        valu = pmc_valu(key)
        if valu is not None:
            entry["roofline"]["valu_issue"] = valu
    return entry


def type_entry(torch, gq, gpuq, orc, orc_ops, wl, typ, steps, warmup, sample_rows, want_cpu):
    ms, out = time_gpu(torch, gq, gpuq, wl, typ, steps, warmup)
    e = {"workload": wl.name, "value": round(wl.n / (ms / 1e3) / 1e6, 1), "unit": "Mweights/s",
         "ms_per_step": round(ms, 4), "steps": steps}
    e.update(cpu_and_roofline(torch, gq, gpuq, orc, orc_ops, wl, typ, ms, out, sample_rows, want_cpu))
    if "cpu_baseline" in e:
        e["speedup_vs_cpu"] = round(e["value"] / e["cpu_baseline"]["value"], 1)
    return e, out


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baselines")
    ap.add_argument("--no-host", action="store_true",
                    help="skip the host entry point timings (their chunked launches would mix into a kernel profile)")
    ap.add_argument("--only", default="", help="comma list of entries to run (%s, or an other type)" %
                    ", ".join(ENTRIES))
    ap.add_argument("--experts", type=int, default=0, help="cap the expert count of the MoE workloads (profiling)")
    ap.add_argument("--tables", choices=["regular", "extreme"], default="regular",
                    help="search tables: the regular stand-ins, or the extreme set (more neighbour shells: lists up to "
                         "490 points) that bounds how the i-quant rates depend on the tables' shape")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: there is no multi-GPU path (experts would shard across GPUs with no "
              "exchange step, each GPU writing disjoint byte ranges). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)
    only = [s.strip() for s in args.only.split(",") if s.strip()]
    bad = [s for s in only if s not in ENTRIES + OTHER]
    if bad:
        ap.error("unknown --only entries: %s" % ", ".join(bad))

    def want(name):
        return not only or name in only

    import torch
    torch.cuda.init()
    import gpuq
    from oracle import Oracle
    os.environ["GPUQ_ALLOW_SYNTHETIC_TABLES"] = "1"      # the repository's stand-in IQ tables (a benchmark run)
    gq = gpuq.load_gpuq(0)
    tpath = gpuq.tables_path()
    if args.tables == "extreme":
        global KEY_SUFFIX
        KEY_SUFFIX = " extreme tables"
        tpath = os.path.join(os.path.dirname(tpath), "gpuq_tables_extreme.bin")
        rc = gq.gpuq_init(tpath.encode(), 0)
        if rc != 0:
            sys.exit("gpuq_init %d on %s (built by __graft_entry__.build())" % (rc, tpath))
    orc = Oracle(tables=tpath)
    orc_ops = Oracle("liboracle_ops.so", tables=tpath)
    nthr = cpu_threads()
    ksteps = max(1, min(args.steps, 5))
    want_cpu = not args.no_cpu
    line = {"metric": METRIC, "value": None, "unit": "Mweights/s", "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "ms_per_step": None, "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": "f32", "data": "synthetic"}
    if args.tables == "extreme":
        line["tables"] = "gpuq_tables_extreme.bin (the stand-in grids with more neighbour shells)"
    host = {"note": "PCIe-inclusive, pageable host memory in and out; not the value"}
    per = {}

    # headline: IQ2_XXS with imatrix on 256 BF16 experts of 2048 x 7168
    if want("IQ2_XXS"):
        nexp_c3 = args.experts or 256
        c3 = wl_c3(torch, gpuq, nexp_c3)
        log("headline: IQ2_XXS on %s" % c3.name)
        srows = c3.nrow * min(nexp_c3, max(2, nthr))
        e, out = type_entry(torch, gq, gpuq, orc, orc_ops, c3, gpuq.IQ2_XXS, args.steps, args.warmup, srows,
                            want_cpu)
        line["value"] = e["value"]
        line["ms_per_step"] = e["ms_per_step"]
        line["config"] = {"workload": "IQ2_XXS with imatrix, " + c3.name, "type": "IQ2_XXS",
                          "shape": [nexp_c3, 2048, 7168], "source": "BF16", "entry_point": "gpuq_requantize_dev"}
        for k in ("roofline", "cpu_baseline", "speedup_vs_cpu", "sample_identical_to_oracle"):
            if k in e:
                line[k] = e[k]
        if not args.no_host:
            log("host entry point: IQ2_XXS on 16 experts")
            host["IQ2_XXS"] = host_api(torch, gq, gpuq, c3, gpuq.IQ2_XXS, min(16, c3.nmat), out)
        nblk16 = min(16, c3.nmat) * (2048 * 7168 // 256)
        log("to_float: IQ2_XXS blocks of %d experts" % (nblk16 // (2048 * 7168 // 256)))
        per["IQ2_XXS_to_float"] = bench_to_float(torch, gq, gpuq, orc, out, gpuq.IQ2_XXS, nblk16, args.steps,
                                                 args.warmup)
        del c3, out
        torch.cuda.empty_cache()
    if want("Q8_0"):
        c1 = wl_c1(torch, gpuq)
        log("per type: Q8_0 on %s" % c1.name)
        per["Q8_0"], _ = type_entry(torch, gq, gpuq, orc, orc_ops, c1, gpuq.Q8_0, args.steps, args.warmup, c1.nrow,
                                    want_cpu)
        del c1
    if want("Q8_0_large"):
        ql = wl_q8_large(torch, gpuq)
        log("per type: Q8_0 on %s (the streaming rate at a size launch time does not weigh on)" % ql.name)
        per["Q8_0_large"], _ = type_entry(torch, gq, gpuq, orc, orc_ops, ql, gpuq.Q8_0, args.steps, args.warmup,
                                          64, False)
        del ql
        torch.cuda.empty_cache()
    c2 = None
    if want("Q4_K") or want("Q6_K") or any(want(t) for t in OTHER) or want("other"):
        c2 = wl_c2(torch, gpuq)
    for name in ("Q4_K", "Q6_K"):
        if want(name):
            log("per type: %s on %s" % (name, c2.name))
            per[name], out = type_entry(torch, gq, gpuq, orc, orc_ops, c2, getattr(gpuq, name), args.steps,
                                        args.warmup, c2.nrow, want_cpu)
            if name == "Q4_K" and not args.no_host:
                log("host entry point: Q4_K on %s" % c2.name)
                host["Q4_K"] = host_api(torch, gq, gpuq, c2, gpuq.Q4_K, 1, out)
            del out
    other = {}
    for name in OTHER:
        if want(name) or (not only) or "other" in only:
            log("other type: %s on %s" % (name, c2.name))
            e, out = type_entry(torch, gq, gpuq, orc, orc_ops, c2, getattr(gpuq, name), ksteps, 1, 64, False)
            del e["workload"]
            other[name] = e
            del out
    if other:
        line["other_types"] = {"workload": c2.name, "types": other}
    del c2
    if want("IQ1_S") or want("IQ1_M"):
        nexp_c4 = args.experts or 384
        c4 = wl_c4(torch, gpuq, nexp_c4)
        for name in ("IQ1_S", "IQ1_M"):
            if want(name):
                log("per type: %s on %s" % (name, c4.name))
                srows = c4.nrow * min(nexp_c4, max(2, nthr))
                per[name], _ = type_entry(torch, gq, gpuq, orc, orc_ops, c4, getattr(gpuq, name), ksteps, 1, srows,
                                          want_cpu)
        del c4
        torch.cuda.empty_cache()
    if "experts16" in only:
        c16 = wl_c3(torch, gpuq, 16)
        for name in EXPERTS16:
            log("experts16: %s on %s" % (name, c16.name))
            e, out = type_entry(torch, gq, gpuq, orc, orc_ops, c16, getattr(gpuq, name), ksteps, 1, 64, False)
            per["%s_16_experts" % name] = e
            del out
        del c16
        torch.cuda.empty_cache()
    if want("LDLQ"):
        log("per type: IQ2_S LDLQ")
        per["IQ2_S_LDLQ"] = bench_ldlq(torch, gq, gpuq, orc, min(args.steps, 2), want_cpu, args.experts or 64)
    if per:
        line["per_type"] = per
    if len(host) > 1:
        line["host_api"] = host
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
