"""GGUF loader (gpeed_amd/host/gguf.{h,cpp}) and the device-resident store.

CPU tests drive tests/cpp/host_check (gguf-info / gguf-read, no device use):
files written by our own writer (gpeed_amd/gguf.py, the layout of
make_test_gguf.py:126-205) must parse to exactly what was written, and to what
the reference's own loader (cpp/core/src/gguf.cpp, compiled into oracle/_ref)
parses from the same file: header, every value type, tensor infos,
alignment, data offset, shards, payload bytes. GPU tests load the same files
into glm5::gpu::WeightStore (pin_nonexpert / pin_experts, the residency of
weights.cpp:62-84): the HBM copy reads back bit for bit and by-name products
match the oracle.
"""
import json
import os
import struct
import subprocess

import numpy as np
import pytest

import oracle
from gpeed_amd import gguf, synth
from conftest import ROOT, rel_err

EXE = os.path.join(ROOT, "tests", "cpp", "host_check")
TIGHT = 2e-5


def run(*args, ok=True):
    r = subprocess.run([EXE, *map(str, args)], stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True,
                       timeout=240)
    if ok:
        assert r.returncode == 0, r.stdout
    return r


def info(path):
    return json.loads(run("gguf-info", path).stdout)


def f16(vals):
    return np.asarray(vals, np.float16).tobytes()


def selftest_file(path, alignment=32, extra_tensors=()):
    """The reference's selftest layout (make_test_gguf.py:146-188: f32, f16,
    bf16, q8_0 and iq3_xxs tensors, the same metadata keys) plus every other
    value type, nested arrays, and IQ3_XXS matrices (2-D and a 3-D expert
    tensor)."""
    rng = np.random.default_rng(1234)
    kvs = [
        ("general.architecture", gguf.STRING, "glm5_next"),
        ("general.name", gguf.STRING, "glm5-selftest"),
        ("general.alignment", gguf.UINT32, alignment),
        ("glm5_next.block_count", gguf.UINT32, 45),
        ("glm5_next.expert_count", gguf.UINT32, 288),
        ("test.float", gguf.FLOAT32, 1.5),
        ("test.array", gguf.ARRAY, (gguf.UINT32, [1, 2, 3])),
        ("t.u8", gguf.UINT8, 250), ("t.i8", gguf.INT8, -5), ("t.u16", gguf.UINT16, 65000),
        ("t.i16", gguf.INT16, -30000), ("t.i32", gguf.INT32, -7), ("t.u64", gguf.UINT64, 1 << 40),
        ("t.i64", gguf.INT64, -(1 << 40)), ("t.f64", gguf.FLOAT64, -2.718281828459045),
        ("t.bool", gguf.BOOL, True), ("t.str_utf8", gguf.STRING, "ΔΣ \"quoted\" \\ tab\t"),
        ("t.strs", gguf.ARRAY, (gguf.STRING, ["a", "", "ccc"])),
        ("t.nested", gguf.ARRAY, (gguf.ARRAY, [(gguf.INT16, [-1, 2]), (gguf.INT16, [])])),
        ("t.empty", gguf.ARRAY, (gguf.FLOAT32, [])),
    ]
    iq = synth.iq3xxs_blocks(77, 0, 1)
    tensors = [
        ("test.f32", [4, 2], gguf.F32, np.array([1.5, -2.25, 3.0, 4.5, 0.0, 7.75, -0.5, 100.0], np.float32).tobytes()),
        ("test.f16", [4], gguf.F16, f16([0.5, -1.0, 2.0, -4.0])),
        ("test.bf16", [4], gguf.BF16, bytes.fromhex("003f80bf004080c0")),
        ("test.q8_0", [32], gguf.Q8_0, f16([0.125]) + rng.integers(0, 256, 32, dtype=np.uint8).tobytes()),
        ("test.iq3_xxs", [256], gguf.IQ3_XXS, iq.tobytes()),
        ("blk.0.attn_q_a.weight", [512, 70], gguf.IQ3_XXS, synth.iq3xxs_matrix(77, 1, 70, 512).tobytes()),
        ("blk.0.ffn_gate_exps.weight", [512, 128, 4], gguf.IQ3_XXS,
         synth.iq3xxs_matrix(77, 2, 512, 512).tobytes()),
        *extra_tensors,
    ]
    gguf.write(path, kvs, tensors)
    return kvs, tensors


def test_writer_matches_reference_layout(tmp_path):
    """The writer's bytes, checked by hand against the format: magic,
    version, counts, the first key, alignment padding, data offsets."""
    kvs, tensors = selftest_file(tmp_path / "t.gguf")
    b = (tmp_path / "t.gguf").read_bytes()
    assert b[:4] == b"GGUF" and struct.unpack("<IQQ", b[4:24]) == (3, len(tensors), len(kvs))
    assert struct.unpack("<Q", b[24:32])[0] == len("general.architecture")
    lay = gguf.layout(kvs, tensors)
    assert all(off % 32 == 0 for off, _ in lay.values())


def test_gguf_info_matches_writer_and_reference(tmp_path):
    path = str(tmp_path / "t.gguf")
    kvs, tensors = selftest_file(path)
    got = info(path)
    assert got["version"] == 3 and got["alignment"] == 32 and got["shards"] == 1
    assert got["data_offset"] % 32 == 0
    assert os.path.getsize(path) == got["data_offset"] + max(off + n for off, n in gguf.layout(kvs, tensors).values())
    for k, vt, v in kvs:
        e = got["kv"][k]
        assert e["type"] == vt, k
        if vt == gguf.ARRAY:
            et, items = v
            assert e["array_type"] == et
            if et == gguf.ARRAY:
                assert e["value"] == [list(x[1]) for x in items]
            else:
                assert e["value"] == list(items), k
        elif vt in (gguf.FLOAT32,):
            assert e["value"] == float(np.float32(v))
        else:
            assert e["value"] == v, k
    lay = gguf.layout(kvs, tensors)
    assert [t["name"] for t in got["tensors"]] == [t[0] for t in tensors]
    for t, (name, dims, dtype, payload) in zip(got["tensors"], tensors):
        assert t["dims"] == list(dims) and t["type"] == dtype and t["offset"] == lay[name][0]
        assert t["n_bytes"] == len(payload)
    ref = oracle.ref()
    if ref is None:
        pytest.skip("oracle/_ref not built: reference loader unavailable")
    want = oracle.ref_gguf_dump(path)
    for field in ("version", "data_offset", "shards", "kv"):
        assert got[field] == want[field], field
    for a, b in zip(got["tensors"], want["tensors"]):
        assert {k: a[k] for k in b} == b


def test_gguf_read_payload_roundtrip(tmp_path):
    path = str(tmp_path / "t.gguf")
    _, tensors = selftest_file(path)
    for name, dims, dtype, payload in tensors:
        run("gguf-read", path, name, tmp_path / "out.bin")
        got = (tmp_path / "out.bin").read_bytes()
        assert got == payload, name
        if oracle.ref() is not None:
            assert oracle.ref_gguf_read(path, name, len(payload)) == payload


def test_gguf_alignment_64_and_shards(tmp_path):
    """general.alignment 64 and a model split over two shard files, found from
    either file's name (GgufModel::discover_shards)."""
    p1, p2 = str(tmp_path / "m-00001-of-00002.gguf"), str(tmp_path / "m-00002-of-00002.gguf")
    kvs1, t1 = selftest_file(p1, alignment=64)
    w2 = synth.iq3xxs_matrix(78, 0, 64, 768)
    kvs2 = [("general.alignment", gguf.UINT32, 64), ("split.no", gguf.UINT16, 1)]
    t2 = [("blk.1.ffn_down.weight", [768, 64], gguf.IQ3_XXS, w2.tobytes()),
          ("test.f32", [2], gguf.F32, np.zeros(2, np.float32).tobytes())]  # duplicate name: the first shard wins
    gguf.write(p2, kvs2, t2)
    for p in (p1, p2):
        got = info(p)
        assert got["shards"] == 2 and got["alignment"] == 64
        names = [t["name"] for t in got["tensors"]]
        assert names == [t[0] for t in t1] + ["blk.1.ffn_down.weight"]
        tdown = got["tensors"][-1]
        assert tdown["shard"] == 1 and tdown["offset"] % 64 == 0
        assert [t for t in got["tensors"] if t["name"] == "test.f32"][0]["shard"] == 0
    run("gguf-read", p2, "blk.1.ffn_down.weight", tmp_path / "o.bin")
    assert (tmp_path / "o.bin").read_bytes() == w2.tobytes()
    if oracle.ref() is not None:
        want = oracle.ref_gguf_dump(p1)
        got = info(p1)
        assert [t["name"] for t in got["tensors"]] == [t["name"] for t in want["tensors"]]
        assert [t["shard"] for t in got["tensors"]] == [t["shard"] for t in want["tensors"]]


@pytest.mark.parametrize("damage,msg", [
    ("magic", "GGUF: bad magic"),
    ("version", "GGUF: unsupported version"),
    ("truncate_header", "GGUF: unexpected end of file"),
    ("truncate_data", "runs past the end"),
    ("alignment0", "GGUF: bad alignment"),
])
def test_gguf_rejects_damaged_files(tmp_path, damage, msg):
    path = tmp_path / "t.gguf"
    if damage == "alignment0":
        gguf.write(path, [("general.alignment", gguf.UINT32, 32)], [], version=3)
    else:
        selftest_file(path)
    b = bytearray(path.read_bytes())
    if damage == "magic":
        b[0:4] = b"GGUX"
    elif damage == "version":
        b[4:8] = struct.pack("<I", 1)
    elif damage == "truncate_header":
        b = b[:200]
    elif damage == "truncate_data":
        b = b[:-100]
    elif damage == "alignment0":
        at = 24 + 8 + len("general.alignment") + 4  # the key's u32 value
        assert struct.unpack("<I", b[at:at + 4])[0] == 32
        b[at:at + 4] = struct.pack("<I", 0)
    path.write_bytes(bytes(b))
    r = run("gguf-info", path, ok=False)
    assert r.returncode == 1 and msg in r.stdout, r.stdout


# ------------------------------------------------------------------ GPU: the resident store

@pytest.mark.gpu
def test_store_pins_and_reads_back(gpu, tmp_path):
    """pin_nonexpert holds, as the reference's (weights.cpp:70-84), every
    tensor but the routed experts, F32 tensors, payloads under 4 KiB and
    (here) types the kernels do not decode; pin_experts adds the experts.
    Each HBM copy (T64 for IQ3_XXS, GGUF rows otherwise) reads back to the
    file's bytes."""
    path = str(tmp_path / "t.gguf")
    wq6 = synth.quant_matrix(78, 0, 14, 16, 512)
    wq8 = synth.quant_matrix(78, 1, 8, 64, 512)
    extra = [("blk.0.attn_output.weight", [512, 16], gguf.Q6_K, wq6.tobytes()),
             ("blk.0.attn_kv_a_mqa.weight", [512, 64], gguf.Q8_0, wq8.tobytes()),
             ("blk.0.attn_norm.weight", [2048], gguf.F32, synth.normal(78, 2, 2048).tobytes()),
             ("blk.0.q4_0.weight", [512, 16], 2, bytes(16 * 16 * 18))]
    _, tensors = selftest_file(path, extra_tensors=extra)
    pinned = {"blk.0.attn_q_a.weight", "blk.0.attn_output.weight", "blk.0.attn_kv_a_mqa.weight"}
    payload = {n: p for n, d, t, p in tensors}
    script = tmp_path / "s.txt"
    lines = ["pin_nonexpert"]
    lines += [f"readback {n} {tmp_path / (n + '.raw')}" for n in sorted(pinned)]
    lines += ["pin_experts", f"readback blk.0.ffn_gate_exps.weight {tmp_path / 'exps.raw'}"]
    script.write_text("\n".join(lines) + "\n")
    out = run("gguf-store", path, script).stdout.split("\n")
    res = [int(l.split()[1]) for l in out if l.startswith("resident")]
    t64 = lambda rows, k: -(-rows // 64) * 64 * k // 256 * 98  # noqa: E731
    assert res[0] == t64(70, 512) + wq6.nbytes + wq8.nbytes
    assert res[1] == res[0] + t64(512, 512)  # + the 4-expert tensor
    for n in pinned:
        assert (tmp_path / (n + ".raw")).read_bytes() == payload[n], n
    assert (tmp_path / "exps.raw").read_bytes() == payload["blk.0.ffn_gate_exps.weight"]


@pytest.mark.gpu
def test_store_products_by_name(gpu, tmp_path):
    """matvec_quant / matmul_quant by tensor name on a store attached to a GGUF
    model (tensors uploaded on first use, IQ3_XXS and other formats) and the
    routed-expert step on the file's 3-D expert tensors, against the
    oracle."""
    H, I, E, T, K = 512, 256, 8, 5, 2
    NH, KVL, DK = 16, 512, 256  # attn_k_b: NH heads of KVL rows over DK
    wq = synth.iq3xxs_matrix(79, 0, 384, 1024)
    wk = synth.iq3xxs_matrix(79, 8, NH * KVL, DK)
    wg = synth.iq3xxs_matrix(79, 1, E * I, H)
    wu = synth.iq3xxs_matrix(79, 2, E * I, H)
    wd = synth.iq3xxs_matrix(79, 3, E * H, I)
    wo = synth.quant_matrix(79, 10, 14, 96, 1024)
    wkv = synth.quant_matrix(79, 11, 8, 80, 1024)
    tensors = [("blk.3.attn_q_b.weight", [1024, 384], gguf.IQ3_XXS, wq.tobytes()),
               ("blk.3.ffn_gate_exps.weight", [H, I, E], gguf.IQ3_XXS, wg.tobytes()),
               ("blk.3.ffn_up_exps.weight", [H, I, E], gguf.IQ3_XXS, wu.tobytes()),
               ("blk.3.ffn_down_exps.weight", [I, H, E], gguf.IQ3_XXS, wd.tobytes()),
               ("blk.3.attn_k_b.weight", [DK, NH * KVL], gguf.IQ3_XXS, wk.tobytes()),
               ("blk.3.attn_output.weight", [1024, 96], gguf.Q6_K, wo.tobytes()),
               ("blk.3.attn_kv_a_mqa.weight", [1024, 80], gguf.Q8_0, wkv.tobytes())]
    path = str(tmp_path / "m.gguf")
    gguf.write(path, [("general.alignment", gguf.UINT32, 32)], tensors)
    x = synth.normal(79, 4, 1024)
    X = synth.normal(79, 5, 12 * 1024).reshape(12, 1024)
    Xm = synth.normal(79, 6, T * H).reshape(T, H)
    logits = synth.normal(79, 7, T * E).reshape(T, E)
    qn = synth.normal(79, 9, NH * DK).reshape(NH, DK)
    for name, a in (("x", x), ("X", X), ("Xm", Xm), ("lg", logits), ("qn", qn)):
        a.astype(np.float32).tofile(tmp_path / f"{name}.bin")
    (tmp_path / "s.txt").write_text(
        f"matvec blk.3.attn_q_b.weight 64 1024 300 {tmp_path / 'x.bin'} {tmp_path / 'y.bin'}\n"
        f"matmul blk.3.attn_q_b.weight 0 1024 384 12 {tmp_path / 'X.bin'} {tmp_path / 'Y.bin'}\n"
        f"moe blk.3.ffn_gate_exps.weight blk.3.ffn_up_exps.weight blk.3.ffn_down_exps.weight {E} {H} {I} {T} {K} "
        f"{tmp_path / 'Xm.bin'} {tmp_path / 'lg.bin'} {tmp_path / 'Ym.bin'}\n"
        f"heads blk.3.attn_k_b.weight 0 {DK} {KVL} {NH} {tmp_path / 'qn.bin'} {tmp_path / 'qa.bin'}\n"
        f"matvec blk.3.attn_output.weight 16 1024 80 {tmp_path / 'x.bin'} {tmp_path / 'yo.bin'}\n"
        f"matmul blk.3.attn_kv_a_mqa.weight 0 1024 80 12 {tmp_path / 'X.bin'} {tmp_path / 'Ykv.bin'}\n")
    run("gguf-store", path, tmp_path / "s.txt")
    y = np.fromfile(tmp_path / "y.bin", np.float32)
    assert rel_err(y, oracle.matvec(wq, 64, 1024, 300, x)) < TIGHT
    Y = np.fromfile(tmp_path / "Y.bin", np.float32).reshape(12, 384)
    ref = oracle.matmul(wq, 0, 1024, 384, X)
    assert max(rel_err(Y[t], ref[t]) for t in range(12)) < TIGHT
    Ym = np.fromfile(tmp_path / "Ym.bin", np.float32).reshape(T, H)
    eptr, tok, wt, _ = oracle.moe_route(logits, K, 1)
    refm = oracle.moe_experts(wg, wu, wd, H, I, Xm, eptr, tok, wt, 10.0)
    assert max(rel_err(Ym[t], refm[t]) for t in range(T)) < TIGHT
    qa = np.fromfile(tmp_path / "qa.bin", np.float32).reshape(NH, KVL)
    for h in range(NH):  # each head: the matvec_quant of model.cpp:640
        assert rel_err(qa[h], oracle.matvec(wk, h * KVL, DK, KVL, qn[h])) < TIGHT, h
    # the other formats by name (Q6_K, Q8_0), uploaded on first use
    yo = np.fromfile(tmp_path / "yo.bin", np.float32)
    assert rel_err(yo, oracle.matmul_rows(14, wo, 16, 1024, 80, x)[0]) < TIGHT
    Ykv = np.fromfile(tmp_path / "Ykv.bin", np.float32).reshape(12, 80)
    assert rel_err(Ykv, oracle.matmul_rows(8, wkv, 0, 1024, 80, X)) < TIGHT
