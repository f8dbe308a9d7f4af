"""GGUF files and the requant driver (gpuq/gguf_io.py, gpuq/requant.py).

CPU: the writer's bytes against a file assembled by hand from the GGUF v3 layout, reader/writer round trips (every
value type, non-default alignment, metadata copied bit for bit), the rules / fallback / imatrix / plan logic of the
reference's tools/requant_experts.py:171-192, 280-293, 420-470, and the --check plan with no GPU.
GPU: a small multi-tensor GGUF re-quantized through gpuq_requantize_batch, every re-quantized tensor compared byte
for byte with the oracle (per expert, each with its imatrix row) and every other tensor with the source.
"""
import os
import struct

import numpy as np
import pytest

from gpuq import gguf_io, requant
import gpuq

T = gguf_io.TYPE_BY_NAME


def _s(b):
    return struct.pack("<Q", len(b)) + b


def test_writer_bytes_match_the_file_layout(tmp_path):
    p = str(tmp_path / "a.gguf")
    x = np.arange(6, dtype=np.float32)
    with gguf_io.GGUFWriter(p) as w:
        w.add_kv("general.architecture", gguf_io.STRING, "llama")
        w.add_kv("n", gguf_io.UINT32, 7)
        w.add_tensor_info("t", (3, 2), T["F32"])
        w.write_header()
        w.write_tensor_data(x)
    # magic, version 3, 1 tensor, 2 key/values; string = u64 length + bytes; the value type is a u32 (8: string,
    # 4: uint32); tensor info = name, u32 n_dims, u64 ne0, ne1, u32 type (0: F32), u64 offset 0; then zeros to the
    # 32-byte alignment, the data, and zeros to the next multiple of 32
    head = (b"GGUF" + struct.pack("<IQQ", 3, 1, 2) + _s(b"general.architecture") + struct.pack("<I", 8) +
            _s(b"llama") + _s(b"n") + struct.pack("<II", 4, 7) + _s(b"t") + struct.pack("<IQQIQ", 2, 3, 2, 0, 0))
    head += b"\0" * (-len(head) % 32)
    want = head + x.tobytes() + b"\0" * 8
    assert open(p, "rb").read() == want


def _sample_file(path, alignment=64):
    rng = np.random.default_rng(3)
    tensors = {
        "blk.0.ffn_down_exps.weight": (T["BF16"], (512, 64, 4), rng.integers(0, 2**16, 512 * 64 * 4, dtype=np.uint16)),
        "blk.0.attn_norm.weight": (T["F32"], (512,), rng.standard_normal(512).astype(np.float32)),
        "blk.0.attn_q.weight": (T["Q8_0"], (512, 3), rng.integers(0, 256, 3 * 16 * 34, dtype=np.uint8)),
        "tok.weight": (T["F16"], (96, 5), rng.standard_normal(480).astype(np.float16)),
    }
    with gguf_io.GGUFWriter(path, alignment=alignment) as w:
        w.add_kv("general.architecture", gguf_io.STRING, "qwen3moe")
        w.add_kv("general.alignment", gguf_io.UINT32, alignment)
        for vt, v in ((gguf_io.UINT8, 200), (gguf_io.INT8, -5), (gguf_io.UINT16, 60000), (gguf_io.INT16, -3000),
                      (gguf_io.UINT32, 4_000_000_000), (gguf_io.INT32, -7), (gguf_io.FLOAT32, 1e-6),
                      (gguf_io.BOOL, True), (gguf_io.UINT64, 2**63 + 5), (gguf_io.INT64, -2**40),
                      (gguf_io.FLOAT64, 0.1)):
            w.add_kv("v.%d" % vt, vt, v)
        w.add_kv("a.i32", gguf_io.ARRAY, [1, -2, 3], sub=gguf_io.INT32)
        w.add_kv("a.f32", gguf_io.ARRAY, [0.5, -0.25], sub=gguf_io.FLOAT32)
        w.add_kv("a.str", gguf_io.ARRAY, ["a", "bé", ""], sub=gguf_io.STRING)
        w.add_kv("a.bool", gguf_io.ARRAY, [True, False], sub=gguf_io.BOOL)
        for name, (tt, shape, data) in tensors.items():
            w.add_tensor_info(name, shape, tt)
        w.write_header()
        for name, (tt, shape, data) in tensors.items():
            w.write_tensor_data(data)
    return tensors


def test_round_trip_values_tensors_and_raw_copy(tmp_path):
    p, q = str(tmp_path / "a.gguf"), str(tmp_path / "b.gguf")
    tensors = _sample_file(p)
    r = gguf_io.GGUFReader(p)
    assert r.alignment == 64 and r.data_offset % 64 == 0
    assert r.get("general.architecture") == "qwen3moe"
    assert r.get("v.%d" % gguf_io.UINT64) == 2**63 + 5 and r.get("v.%d" % gguf_io.INT16) == -3000
    assert r.get("v.%d" % gguf_io.FLOAT32) == np.float32(1e-6) and r.get("v.%d" % gguf_io.BOOL) is True
    assert r.get("a.i32") == [1, -2, 3] and r.get("a.f32") == [0.5, -0.25] and r.get("a.str") == ["a", "bé", ""]
    assert r.get("a.bool") == [True, False] and r.fields["a.str"].sub == gguf_io.STRING
    assert [t.name for t in r.tensors] == list(tensors)
    for t in r.tensors:
        tt, shape, data = tensors[t.name]
        assert t.tensor_type == tt and t.shape == shape and t.offset % 64 == 0
        assert np.array_equal(t.data, np.frombuffer(data.tobytes(), dtype=np.uint8))
    assert np.array_equal(r.tensor("tok.weight").f32(), tensors["tok.weight"][2].astype(np.float32).reshape(5, 96))
    # a copy through add_raw_kv and the stored tensor bytes is the same file
    with gguf_io.GGUFWriter(q) as w:
        for kv in r.fields.values():
            w.add_raw_kv(kv)
        for t in r.tensors:
            w.add_tensor_info(t.name, t.shape, t.tensor_type)
        w.write_header()
        for t in r.tensors:
            w.write_tensor_data(t.data)
    assert open(p, "rb").read() == open(q, "rb").read()


def test_reader_rejects_bad_files(tmp_path):
    p = tmp_path / "bad.gguf"
    p.write_bytes(b"GGUX" + b"\0" * 60)
    with pytest.raises(ValueError, match="not a GGUF"):
        gguf_io.GGUFReader(str(p))
    q = str(tmp_path / "a.gguf")
    _sample_file(q)
    cut = tmp_path / "cut.gguf"
    cut.write_bytes(open(q, "rb").read()[:-100])
    with pytest.raises(ValueError, match="runs past the end"):
        gguf_io.GGUFReader(str(cut))


def test_writer_checks_sizes_and_counts(tmp_path):
    p = str(tmp_path / "w.gguf")
    w = gguf_io.GGUFWriter(p)
    w.add_tensor_info("t", (32, 2), T["Q8_0"])
    w.add_tensor_info("u", (4,), T["F32"])
    w.write_header()
    with pytest.raises(ValueError, match="68 declared"):
        w.write_tensor_data(np.zeros(64, np.uint8))
    w.write_tensor_data(np.zeros(68, np.uint8))
    with pytest.raises(RuntimeError, match="1 of 2"):
        w.close()
    assert not os.path.exists(p)
    with pytest.raises(ValueError, match="not whole Q4_K blocks"):
        gguf_io.GGUFWriter(p).add_tensor_info("t", (100, 2), T["Q4_K"])


def test_ggml_type_sizes():
    # bytes a block from the blocks' layouts: fp16 scale(s) plus packed codes
    assert gguf_io.GGML_TYPES[T["Q8_0"]][1:] == (32, 2 + 32)
    assert gguf_io.GGML_TYPES[T["Q4_K"]][1:] == (256, 2 + 2 + 12 + 128)
    assert gguf_io.GGML_TYPES[T["Q6_K"]][1:] == (256, 128 + 64 + 16 + 2)
    assert gguf_io.GGML_TYPES[T["IQ2_XXS"]][1:] == (256, 2 + 64)
    assert gguf_io.GGML_TYPES[T["IQ1_M"]][1:] == (256, 32 + 16 + 8)
    assert gguf_io.GGML_TYPES[T["MXFP4"]][1:] == (32, 1 + 16)
    # and the library's own answers for every type it quantizes (symbols only: no device work)
    if os.path.exists(gpuq.lib_path()):
        lib = gpuq.open_lib()
        for t in gpuq.TYPE_NAMES:
            assert gguf_io.GGML_TYPES[t][2] == lib.gpuq_block_bytes(t), gpuq.TYPE_NAMES[t]
            assert gguf_io.GGML_TYPES[t][1] == gpuq.BLOCK[t]


def test_rules_fallback_and_imatrix(tmp_path):
    rp = tmp_path / "rules.txt"
    rp.write_text("# experts\nblk\\.0\\.ffn_(gate|up)_exps\\.weight  iq2_xxs\nffn_down_exps iq1_m # down\n"
                  "attn_q q8_0\n.*exps q4_k\n")
    rules = requant.read_rules(str(rp))
    assert [t for _, t in rules] == [T["IQ2_XXS"], T["IQ1_M"], T["Q8_0"], T["Q4_K"]]
    assert requant.rule_type(rules, "blk.0.ffn_up_exps.weight") == T["IQ2_XXS"]
    assert requant.rule_type(rules, "blk.1.ffn_up_exps.weight") == T["Q4_K"]      # first match wins
    assert requant.rule_type(rules, "output.weight") is None
    rp.write_text("x q9_9\n")
    with pytest.raises(requant.RequantError, match="rules.txt:1"):
        requant.read_rules(str(rp))
    # fallback: 640-long rows fit 32-weight blocks only; 100 fits none
    assert requant.fit_type(T["IQ2_XXS"], 640) == T["IQ4_NL"] and requant.fit_type(T["IQ2_XXS"], 512) == T["IQ2_XXS"]
    assert requant.fit_type(T["Q4_K"], 640) == T["Q5_0"] and requant.fit_type(T["Q6_K"], 640) == T["Q8_0"]
    assert requant.fit_type(T["IQ1_S"], 100) == T["F16"] and requant.fit_type(T["Q8_0"], 100) == T["F16"]
    # imatrix: in_sum2 / counts per expert row, 1.0 where the count is 0
    ip = str(tmp_path / "im.gguf")
    s = np.arange(12, dtype=np.float32).reshape(3, 4) + 1
    c = np.array([2, 0, 4], dtype=np.float32)
    with gguf_io.GGUFWriter(ip) as w:
        w.add_tensor_info("blk.0.ffn_down_exps.weight.in_sum2", (12,), T["F32"])
        w.add_tensor_info("blk.0.ffn_down_exps.weight.counts", (3,), T["F32"])
        w.write_header()
        w.write_tensor_data(s)
        w.write_tensor_data(c)
    im = requant.read_imatrix(ip)["blk.0.ffn_down_exps.weight"]
    assert np.array_equal(im, np.array([s[0] / 2, [1, 1, 1, 1], s[2] / 4], dtype=np.float32))


def test_plan_and_check_mode(tmp_path, capsys):
    p = str(tmp_path / "m.gguf")
    _sample_file(p)
    r = gguf_io.GGUFReader(p)
    rules = [(requant.re.compile("ffn_down_exps"), T["IQ2_XXS"]), (requant.re.compile("attn_norm"), T["Q8_0"]),
             (requant.re.compile("attn_q"), T["Q8_0"]), (requant.re.compile("tok"), T["Q4_K"])]
    plan = {s.tensor.name: s for s in requant.plan_shard(r, rules[:3], {})}
    assert plan["blk.0.ffn_down_exps.weight"].new_type is None            # IQ2_XXS needs an imatrix
    assert "no imatrix" in plan["blk.0.ffn_down_exps.weight"].note
    assert plan["blk.0.attn_norm.weight"].new_type is None and "not a matrix" in plan["blk.0.attn_norm.weight"].note
    assert plan["blk.0.attn_q.weight"].new_type is None                   # already Q8_0
    s = requant.plan_shard(r, rules[3:], {})[-1]                          # 96-long rows: Q4_K -> Q5_0
    assert s.new_type == T["Q5_0"] and "fallback" in s.note and s.nbytes == 5 * 3 * 22
    with pytest.raises(requant.RequantError, match="does not quantize Q5_0"):   # (a library without it)
        requant.plan_shard(r, rules[3:], {}, can_quantize=lambda typ, with_im: typ != T["Q5_0"])
    im = {"blk.0.ffn_down_exps.weight": np.ones((4, 512), np.float32)}
    s = requant.plan_shard(r, rules[:1], im)[0]
    assert s.new_type == T["IQ2_XXS"] and s.nbytes == 4 * 64 * 2 * 66 and s.imatrix is im[s.tensor.name]
    s = requant.plan_shard(r, rules[:1], {"blk.0.ffn_down_exps.weight": np.ones((3, 512), np.float32)})[0]
    assert s.new_type is None and "does not fit" in s.note
    s = requant.plan_shard(r, [(requant.re.compile("down"), T["Q4_K"])],
                           {"blk.0.ffn_down_exps.weight": np.ones((3, 512), np.float32)})[0]
    assert s.new_type == T["Q4_K"] and s.imatrix is None and "without it" in s.note
    # the command line's --check: the plan, no GPU, no files
    rp = tmp_path / "rules.txt"
    rp.write_text("attn_q q4_k\n")
    assert requant.main([p, str(tmp_path / "out"), str(rp), "--check"]) == 0
    assert "Q8_0" in capsys.readouterr().out and not os.path.exists(tmp_path / "out")
    assert requant.main([p, str(tmp_path / "out"), str(rp), "--dump=x"]) == 2


def test_hessian_files_and_plan(tmp_path):
    """which tensors take error feedback: an expert tensor with a Hessian of its shape, an imatrix, a type rounded per
    256-weight super-block and a float source; anything else is rounded plain, with the reason"""
    hd = tmp_path / "h"
    hd.mkdir()
    assert requant.hess_file(str(hd), "blk.0.ffn_down_exps.weight") is None
    np.save(hd / "blk.0.mid.npy", np.zeros((4, 512, 512)))
    np.save(hd / "blk.0.counts.npy", np.full(4, 100.0))
    np.save(hd / "blk.0.in_g.npy", np.zeros((4, 256, 256)))
    assert requant.hess_file(str(hd), "blk.0.ffn_down_exps.weight") == (str(hd / "blk.0.mid.npy"),
                                                                       str(hd / "blk.0.counts.npy"))
    assert requant.hess_file(str(hd), "blk.0.ffn_up_exps.weight") is None
    assert requant.hess_file(str(hd), "blk.0.ffn_up_exps.weight", gated=True)[0].endswith("blk.0.in_g.npy")
    assert requant.hess_file(str(hd), "blk.0.attn_q.weight") is None
    p = str(tmp_path / "m.gguf")
    _sample_file(p)
    r = gguf_io.GGUFReader(p)
    im = {"blk.0.ffn_down_exps.weight": np.ones((4, 512), np.float32)}
    hess = {"dir": str(hd)}
    for typ, imat, note in ((T["IQ2_S"], im, None), (T["IQ2_S"], {}, "no imatrix data"),
                            (T["Q8_0"], im, "not rounded per 256-weight super-block"), (T["Q4_K"], im, None),
                            (T["Q6_K"], im, None), (T["Q3_K"], im, "not rounded per 256-weight super-block")):
        s = requant.plan_shard(r, [(requant.re.compile("down"), typ)], imat, None, hess)[0]
        if note is None:
            assert s.hessian is not None and s.new_type == typ
        else:
            assert s.hessian is None and note in s.note
    # a library that cannot read a type back rounds it plain, with the reason (instead of failing mid-run)
    s = requant.plan_shard(r, [(requant.re.compile("down"), T["Q4_K"])], im, None, hess, can_ldlq=lambda t: False)[0]
    assert s.hessian is None and "cannot read Q4_K back" in s.note and s.new_type == T["Q4_K"]
    np.save(hd / "blk.0.mid.npy", np.zeros((3, 512, 512)))
    s = requant.plan_shard(r, [(requant.re.compile("down"), T["IQ2_S"])], im, None, hess)[0]
    assert s.hessian is None and "does not fit" in s.note and s.new_type == T["IQ2_S"]


def test_shard_paths():
    assert requant.shard_paths("/m/x-00001-of-00003.gguf") == ["/m/x-%05d-of-00003.gguf" % i for i in (1, 2, 3)]
    assert requant.shard_paths("/m/x.gguf") == ["/m/x.gguf"]


@pytest.fixture(scope="module")
def gq():
    """the library on device 0, loaded after torch has touched the GPU (torch wheels bundle a HIP runtime of the
    same soname: initialised first, it serves both, and the later test modules' torch calls keep working)"""
    import torch
    torch.cuda.init()
    return gpuq.load_gpuq(0)


@pytest.mark.gpu
def test_requant_gguf_matches_oracle(tmp_path, gq):
    """a two-shard model: BF16 experts -> IQ2_XXS, MXFP4 experts -> IQ1_M, F32 -> Q8_0 and F16 -> Q4_K without an
    imatrix, 640-long rows -> IQ4_NL (the fallback), llama-quantize's other fallbacks (96-long rows asked Q4_K -> Q5_0
    with an imatrix, 160-long F16 rows asked Q5_K -> Q5_1, 100-long BF16 rows asked Q2_K -> F16), the rest copied; the
    second shard also with --only-matched"""
    from oracle import Oracle
    orc = Oracle(tables=gpuq.tables_path())
    rng = np.random.default_rng(11)
    ne0, ne1, nexp = 512, 32, 3
    bf = (rng.standard_normal((nexp, ne1, ne0)).astype(np.float32) * 0.02).view(np.uint32)
    bf16 = ((bf + 0x7FFF + ((bf >> 16) & 1)) >> 16).astype(np.uint16)          # RNE to BF16
    mx = np.empty((nexp, ne1, ne0 // 32, 17), np.uint8)
    mx[..., 0] = rng.integers(119, 124, mx.shape[:3])
    mx[..., 1:] = rng.integers(0, 256, mx.shape[:3] + (16,))
    f32 = (rng.standard_normal((8, ne0)) * 0.02).astype(np.float32)
    f16 = (rng.standard_normal((4, ne0)) * 0.02).astype(np.float16)
    nl = (rng.standard_normal((6, 640)) * 0.02).astype(np.float32)
    q50 = (rng.standard_normal((5, 96)) * 0.02).astype(np.float32)
    q51 = (rng.standard_normal((4, 160)) * 0.02).astype(np.float16)
    b100 = (rng.standard_normal((3, 100)).astype(np.float32) * 0.02).view(np.uint32)
    b100 = ((b100 + 0x7FFF + ((b100 >> 16) & 1)) >> 16).astype(np.uint16)
    norm = rng.standard_normal(ne0).astype(np.float32)
    ims = {n: rng.lognormal(0, 1.5, shp).astype(np.float32) for n, shp in (
        ("blk.0.ffn_up_exps.weight", (nexp, ne0)), ("blk.0.ffn_down_exps.weight", (nexp, ne0)),
        ("blk.1.fallback.weight", (1, 640)), ("blk.1.q50.weight", (1, 96)))}
    shard = [
        [("blk.0.ffn_up_exps.weight", T["BF16"], (ne0, ne1, nexp), bf16), ("blk.0.norm.weight", T["F32"], (ne0,), norm),
         ("blk.0.ffn_down_exps.weight", T["MXFP4"], (ne0, ne1, nexp), mx)],
        [("blk.1.attn_q.weight", T["F32"], (ne0, 8), f32), ("blk.1.attn_k.weight", T["F16"], (ne0, 4), f16),
         ("blk.1.fallback.weight", T["F32"], (640, 6), nl), ("blk.1.keep.weight", T["F32"], (ne0, 8), f32),
         ("blk.1.q50.weight", T["F32"], (96, 5), q50), ("blk.1.q51.weight", T["F16"], (160, 4), q51),
         ("blk.1.f16.weight", T["BF16"], (100, 3), b100)],
    ]
    src = tmp_path / "src"
    src.mkdir()
    for i, tensors in enumerate(shard):
        with gguf_io.GGUFWriter(str(src / ("m-%05d-of-00002.gguf" % (i + 1)))) as w:
            if i == 0:
                w.add_kv("general.architecture", gguf_io.STRING, "qwen3moe")
            w.add_kv("split.no", gguf_io.UINT16, i)
            for name, tt, shp, _ in tensors:
                w.add_tensor_info(name, shp, tt)
            w.write_header()
            for *_, data in tensors:
                w.write_tensor_data(data)
    imp = str(tmp_path / "im.gguf")
    with gguf_io.GGUFWriter(imp) as w:
        for n, a in ims.items():
            w.add_tensor_info(n + ".in_sum2", (a.size,), T["F32"])
            w.add_tensor_info(n + ".counts", (a.shape[0],), T["F32"])
        w.write_header()
        for a in ims.values():
            w.write_tensor_data(a)
            w.write_tensor_data(np.ones(a.shape[0], np.float32))
    rules = tmp_path / "rules.txt"
    rules.write_text("ffn_up_exps iq2_xxs\nffn_down_exps iq1_m\nattn_q q8_0\nattn_k q4_k\nfallback iq2_xxs\n"
                     "q50 q4_k\nq51 q5_k\nf16 q2_k\n")
    out = tmp_path / "out"
    requant.run(str(src / "m-00001-of-00002.gguf"), str(out), str(rules), imp, gq=gq)
    want_types = {"blk.0.ffn_up_exps.weight": T["IQ2_XXS"], "blk.0.ffn_down_exps.weight": T["IQ1_M"],
                  "blk.1.attn_q.weight": T["Q8_0"], "blk.1.attn_k.weight": T["Q4_K"],
                  "blk.1.fallback.weight": T["IQ4_NL"], "blk.1.q50.weight": T["Q5_0"], "blk.1.q51.weight": T["Q5_1"],
                  "blk.1.f16.weight": T["F16"]}
    for i, tensors in enumerate(shard):
        name = "m-%05d-of-00002.gguf" % (i + 1)
        r, s = gguf_io.GGUFReader(str(out / name)), gguf_io.GGUFReader(str(src / name))
        assert [f.raw for f in r.fields.values()] == [f.raw for f in s.fields.values()]
        assert [t.name for t in r.tensors] == [t.name for t in s.tensors]
        for t, st in zip(r.tensors, s.tensors):
            assert t.shape == st.shape
            if t.name not in want_types:
                assert t.tensor_type == st.tensor_type and np.array_equal(t.data, st.data), t.name
                continue
            typ = want_types[t.name]
            assert t.tensor_type == typ, t.name
            n0 = st.shape[0]
            nmat = st.shape[2] if len(st.shape) == 3 else 1
            if st.tensor_type == T["BF16"] and n0 % 32:          # (the oracle's decoder takes 32-value blocks)
                x = (np.ascontiguousarray(st.data).view(np.uint16).astype(np.uint32) << 16).view(np.float32)
                x = x.reshape(nmat, -1, n0)
            else:
                x = orc.decode_src(st.tensor_type, np.ascontiguousarray(st.data), st.n_elements).reshape(nmat, -1, n0)
            im = ims.get(t.name) if typ != T["Q4_K"] else None
            rows = [orc.quantize(typ, x[e], None if im is None or typ == T["Q8_0"] else im[e]) for e in range(nmat)]
            assert np.array_equal(t.data, np.concatenate([a.reshape(-1) for a in rows])), t.name
    # --only-matched: shard 1's metadata minus the split keys, the re-quantized tensors only
    out2 = tmp_path / "out2"
    requant.run(str(src / "m-00001-of-00002.gguf"), str(out2), str(rules), imp, gq=gq, only_matched=True)
    r = gguf_io.GGUFReader(str(out2 / "m-00002-of-00002.gguf"))
    assert list(r.fields) == ["general.architecture"]
    assert [t.name for t in r.tensors] == ["blk.1.attn_q.weight", "blk.1.attn_k.weight", "blk.1.fallback.weight",
                                           "blk.1.q50.weight", "blk.1.q51.weight", "blk.1.f16.weight"]
    full = gguf_io.GGUFReader(str(out / "m-00002-of-00002.gguf"))
    for t in r.tensors:
        assert np.array_equal(t.data, full.tensor(t.name).data)


@pytest.mark.gpu
@pytest.mark.parametrize("tname,weights", [("IQ2_S", "imatrix"), ("Q4_K", "imatrix"), ("IQ2_XXS", "schur")])
def test_requant_hessian_matches_oracle_ldlq(tmp_path, oracle_lib, gq, tname, weights):
    """--hessian: BF16 experts -> an i-quant or k-quant with error feedback, one Hessian per expert from blk.0.in.npy;
    expert 1's row count is below LDLQ_MIN_ROWS (plain rounding). Each expert equals the oracle's LDLQ loop on the
    factor the device builds from that expert's Hessian, with the --weights importance (or the oracle's plain
    quantization for expert 1)."""
    import torch
    from gpuq import ldlq
    from test_ldlq_gpu import design, prepare_dev
    ne0, ne1, nexp, typ = 512, 16, 3, T[tname]
    Hs, ims, ws = [], [], []
    for e in range(nexp):
        H, n, imatrix, W = design(ne1=ne1, ne0=ne0, seed=20 + e)
        Hs.append(H)
        ims.append(imatrix * (1 + e))
        ws.append(W[0])
    counts = np.array([n, 10, n], dtype=np.float64)
    bits = np.stack(ws).view(np.uint32)
    bf16 = ((bits + 0x7FFF + ((bits >> 16) & 1)) >> 16).astype(np.uint16)
    wbf = (bf16.astype(np.uint32) << 16).view(np.float32)                     # the weights the file holds
    hd = tmp_path / "hess"
    hd.mkdir()
    np.save(hd / "blk.0.in.npy", np.stack(Hs))
    np.save(hd / "blk.0.counts.npy", counts)
    src = str(tmp_path / "m.gguf")
    with gguf_io.GGUFWriter(src) as w:
        w.add_tensor_info("blk.0.ffn_up_exps.weight", (ne0, ne1, nexp), T["BF16"])
        w.add_tensor_info("blk.0.ffn_down_exps.weight", (ne0, ne1, nexp), T["BF16"])   # no Hessian: plain
        w.write_header()
        w.write_tensor_data(bf16)
        w.write_tensor_data(bf16)
    imp = str(tmp_path / "im.gguf")
    im_all = np.stack(ims).astype(np.float32)
    with gguf_io.GGUFWriter(imp) as w:
        for nm in ("blk.0.ffn_up_exps.weight", "blk.0.ffn_down_exps.weight"):
            w.add_tensor_info(nm + ".in_sum2", (im_all.size,), T["F32"])
            w.add_tensor_info(nm + ".counts", (nexp,), T["F32"])
        w.write_header()
        for _ in range(2):
            w.write_tensor_data(im_all)
            w.write_tensor_data(np.ones(nexp, np.float32))
    rules = tmp_path / "rules.txt"
    rules.write_text("ffn_(up|down)_exps %s\n" % tname.lower())
    out = tmp_path / "out"
    print("case requant --hessian %s weights=%s" % (tname, weights), flush=True)
    requant.run(src, str(out), str(rules), imp, gq=gq,
                hess={"dir": str(hd), "damp": 0.01, "order": "seq", "weights": weights})
    r = gguf_io.GGUFReader(str(out / "m.gguf"))
    rb = ne0 // 256 * gq.gpuq_block_bytes(typ)
    for e in range(nexp):
        if counts[e] < requant.MIN_ROWS:
            want = oracle_lib.quantize(typ, wbf[e], im_all[e])
        else:
            U, perm, _, _ = prepare_dev(torch, gq, Hs[e], counts[e], "seq")
            qw = im_all[e][perm] if weights == "imatrix" else oracle_lib.schur_weights(U)
            want = oracle_lib.ldlq(typ, wbf[e][None][:, :, perm], U, qw[None], ldlq.slot_order(perm))[0][0]
        got = r.tensor("blk.0.ffn_up_exps.weight").data.reshape(nexp, ne1 * rb)[e]
        assert np.array_equal(got, want.reshape(-1)), "expert %d: %d bytes differ" % (e, int((got != want.reshape(-1)).sum()))
        plain = oracle_lib.quantize(typ, wbf[e], im_all[e])
        assert np.array_equal(r.tensor("blk.0.ffn_down_exps.weight").data.reshape(nexp, -1)[e], plain.reshape(-1))
    # the feedback changed the experts it ran on
    assert not np.array_equal(r.tensor("blk.0.ffn_up_exps.weight").data, r.tensor("blk.0.ffn_down_exps.weight").data)
