"""The GGUF reader (vireo_gguf_*, vireo_amd/csrc/gguf.c) on the host.

* Against the reference's own reader (src/gguf.c, compiled into
  oracle/_ref): on synthetic MoE files of several shapes and alignments, the
  two parse the same version, counts, alignment, data offset, every metadata
  entry (key, type, value bits, string, array type/length/position) and every
  tensor (name, dims, type, offset, element and byte counts, data position),
  and the getters agree.
* Against what was written (independent of the reference): every scalar type,
  strings, string/number/nested arrays, tensor bytes.
* Malformed files: every truncation of a file, bad magic or version, a tensor
  reaching past the end, a zero alignment and random corruption return NULL
  (or a context) without reading outside the file.
* The MoE loader's metadata errors (no expert_count, no block_count) come back
  as -EINVAL with a message, before any device work.
"""
import ctypes as C
import errno
import os
import struct

import numpy as np
import pytest

from vireo_amd import _lib
from vireo_amd import gguf as G
from vireo_amd import workloads as W

TINY = W.MoEShape("tiny", 256, 8, 2, 256, True, W.Q4_K, W.Q4_K, W.Q6_K)
TINY_Q8 = W.MoEShape("tiny-q8", 256, 8, 2, 256, False, W.Q8_0, W.Q8_0, W.Q8_0)


@pytest.fixture(scope="module")
def vl():
    return _lib.load()


@pytest.fixture(scope="module")
def reflib():
    from oracle.oracle import Reference
    if not Reference.available():
        pytest.skip("oracle/_ref not built")
    L = C.CDLL(os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "oracle", "_ref",
                            "libvireo_ref.so"))
    P = C.POINTER(_lib.GGUFCtx)
    L.gguf_open.restype, L.gguf_open.argtypes = P, [C.c_char_p]
    L.gguf_close.argtypes = [P]
    L.gguf_get_u64.restype, L.gguf_get_u64.argtypes = C.c_int, [P, C.c_char_p, C.POINTER(C.c_uint64)]
    L.gguf_get_f32.restype, L.gguf_get_f32.argtypes = C.c_int, [P, C.c_char_p, C.POINTER(C.c_float)]
    L.gguf_get_str.restype, L.gguf_get_str.argtypes = C.c_void_p, [P, C.c_char_p, C.POINTER(C.c_uint64)]
    L.gguf_tensor_by_name.restype, L.gguf_tensor_by_name.argtypes = C.POINTER(_lib.GGUFTensor), [P, C.c_char_p]
    return L


def kv_rec(g, i):
    k = g.kv[i]
    base = g.map
    return (k.key.text(), k.type, k.val if k.type not in (G.STRING, G.ARRAY) else None,
            k.str.text() if k.type == G.STRING else None, k.arr_type if k.type == G.ARRAY else None,
            k.arr_len if k.type == G.ARRAY else None, (k.arr_data - base) if k.type == G.ARRAY else None)


def tensor_rec(g, i):
    t = g.tensors[i]
    return (t.name.text(), t.n_dims, tuple(t.dims[:t.n_dims]), t.ggml_type, t.offset, t.n_elems, t.nbytes,
            t.data - g.map)


def summary(p):
    g = p.contents
    return ((g.version, g.n_tensors, g.n_kv, g.alignment, g.data - g.map),
            [kv_rec(g, i) for i in range(g.n_kv)], [tensor_rec(g, i) for i in range(g.n_tensors)])


@pytest.mark.parametrize("shape,layers,vocab,untied,align", [
    (TINY, 2, 300, False, 32), (TINY, 3, 0, False, 64), (TINY_Q8, 2, 128, True, 32), (TINY_Q8, 1, 64, True, 256)])
def test_reader_matches_reference(vl, reflib, tmp_path, shape, layers, vocab, untied, align):
    path = str(tmp_path / "m.gguf")
    G.write_moe_gguf(path, shape, layers, seed=5, vocab=vocab, untied=untied, alignment=align)
    a, b = vl.vireo_gguf_open(path.encode()), reflib.gguf_open(path.encode())
    assert a and b
    sa, sb = summary(a), summary(b)
    assert sa[0] == sb[0]
    assert sa[1] == sb[1]
    assert sa[2] == sb[2]
    arch = G.moe_arch(shape)
    for key in [f"{arch}.block_count", f"{arch}.expert_count", f"{arch}.expert_used_count", "general.alignment",
                f"{arch}.attention.layer_norm_rms_epsilon", "general.architecture", "absent.key"]:
        u1, u2, f1, f2, n1, n2 = C.c_uint64(7), C.c_uint64(7), C.c_float(7), C.c_float(7), C.c_uint64(9), C.c_uint64(9)
        assert vl.vireo_gguf_get_u64(a, key.encode(), C.byref(u1)) == reflib.gguf_get_u64(b, key.encode(), C.byref(u2))
        assert u1.value == u2.value
        assert vl.vireo_gguf_get_f32(a, key.encode(), C.byref(f1)) == reflib.gguf_get_f32(b, key.encode(), C.byref(f2))
        assert f1.value == f2.value
        s1, s2 = vl.vireo_gguf_get_str(a, key.encode(), C.byref(n1)), reflib.gguf_get_str(b, key.encode(), C.byref(n2))
        assert (s1 is None) == (s2 is None) and n1.value == n2.value
        if s1:
            assert s1 - a.contents.map == s2 - b.contents.map
    for name in ["blk.0.ffn_down_exps.weight", "token_embd.weight", "output.weight", "nope"]:
        t1, t2 = vl.vireo_gguf_tensor_by_name(a, name.encode()), reflib.gguf_tensor_by_name(b, name.encode())
        assert bool(t1) == bool(t2)
        if t1:
            assert t1.contents.data - a.contents.map == t2.contents.data - b.contents.map
    vl.vireo_gguf_close(a)
    reflib.gguf_close(b)


def test_reader_values(vl, tmp_path):
    """Values against what the writer put there (the reference's convention:
    integer scalars are their raw bits, zero-extended; F32/F64 as double)."""
    w = G.GGUFWriter(alignment=64)
    scalars = [("u8", G.U8, 200), ("i8", G.I8, -3), ("u16", G.U16, 65000), ("i16", G.I16, -300),
               ("u32", G.U32, 4000000000), ("i32", G.I32, -5), ("u64", G.U64, 2 ** 63 + 5), ("i64", G.I64, -7),
               ("bool", G.BOOL, True), ("f32", G.F32, 0.1), ("f64", G.F64, -2.5)]
    for k, t, v in scalars:
        w.add(k, t, v)
    w.add("s", G.STRING, "héllo")
    w.add("empty", G.STRING, "")
    w.add("arr_s", G.ARRAY, ["a", "", "ccc"], G.STRING)
    w.add("arr_f", G.ARRAY, [1.0, 2.0], G.F32)
    w.add("nested", G.ARRAY, [[1, 2], [3]], (G.ARRAY, G.U32))  # an array of arrays
    blobs = {"t0": np.arange(100, dtype=np.float32), "t1": np.arange(70, dtype=np.uint8)}
    w.add_tensor("t0", [100], W.F32, blobs["t0"])
    w.add_tensor("t1", [70], 99, blobs["t1"])  # a type without a block size: nbytes 0
    path = str(tmp_path / "v.gguf")
    w.write(path)
    p = vl.vireo_gguf_open(path.encode())
    assert p
    g = p.contents
    assert g.alignment == 64 and (g.data - g.map) % 64 == 0
    for k, t, v in scalars:
        kv = vl.vireo_gguf_find(p, k.encode()).contents
        assert kv.type == t
        if t in (G.F32, G.F64):
            assert struct.unpack("<d", struct.pack("<Q", kv.val))[0] == (np.float32(v) if t == G.F32 else v)
        else:
            raw = struct.unpack(G._FMT[t].replace("b", "B").replace("h", "H").replace("i", "I").replace("q", "Q")
                                .replace("?", "B"), struct.pack(G._FMT[t], v))[0]
            assert kv.val == raw
    n = C.c_uint64()
    s = vl.vireo_gguf_get_str(p, b"s", C.byref(n))
    assert C.string_at(s, n.value).decode() == "héllo"
    assert vl.vireo_gguf_get_str(p, b"empty", C.byref(n)) is not None and n.value == 0
    for key, at, ln in [("arr_s", G.STRING, 3), ("arr_f", G.F32, 2), ("nested", G.ARRAY, 2)]:
        kv = vl.vireo_gguf_find(p, key.encode()).contents
        assert kv.type == G.ARRAY and kv.arr_type == at and kv.arr_len == ln
    f = vl.vireo_gguf_find(p, b"arr_f").contents
    assert np.frombuffer(C.string_at(f.arr_data, 8), np.float32).tolist() == [1.0, 2.0]
    t0 = vl.vireo_gguf_tensor_by_name(p, b"t0").contents
    assert t0.nbytes == 400 and t0.n_elems == 100
    assert np.array_equal(np.frombuffer(C.string_at(t0.data, 400), np.float32), blobs["t0"])
    t1 = vl.vireo_gguf_tensor_by_name(p, b"t1").contents
    assert t1.nbytes == 0 and t1.offset % 64 == 0
    assert C.string_at(t1.data, 70) == blobs["t1"].tobytes()
    vl.vireo_gguf_close(p)


def small_file(tmp_path):
    w = G.GGUFWriter()
    w.add("general.architecture", G.STRING, "olmoe")
    w.add("arr", G.ARRAY, ["x", "yy"], G.STRING)
    w.add("n", G.U32, 3)
    w.add_tensor("a", [64], W.F32, np.ones(64, np.float32))
    w.add_tensor("b", [32, 2], W.Q8_0, np.zeros(68, np.uint8))
    path = str(tmp_path / "s.gguf")
    w.write(path)
    return path, open(path, "rb").read()


def test_reader_rejects_malformed(vl, tmp_path):
    path, data = small_file(tmp_path)
    ok = vl.vireo_gguf_open(path.encode())
    assert ok
    last = ok.contents.tensors[ok.contents.n_tensors - 1]
    end = last.data - ok.contents.map + last.nbytes  # the file may end anywhere after this
    vl.vireo_gguf_close(ok)
    bad = str(tmp_path / "bad.gguf")

    def opens(blob):
        with open(bad, "wb") as f:
            f.write(blob)
        p = vl.vireo_gguf_open(bad.encode())
        if p:
            vl.vireo_gguf_close(p)
        return bool(p)
    # every prefix that cuts into the header or the tensors' bytes fails
    for n in range(len(data) + 1):
        assert opens(data[:n]) == (n >= end), n
    assert not opens(b"GGUG" + data[4:])
    for v in (1, 4):
        assert not opens(data[:4] + struct.pack("<I", v) + data[8:])
    assert not opens(data[:8] + struct.pack("<Q", 1 << 40) + data[16:])  # tensor count beyond the file
    # a zero alignment
    w = G.GGUFWriter()
    w.add("general.alignment", G.U32, 0)
    w.write(bad)
    assert not vl.vireo_gguf_open(bad.encode())
    # random corruption: NULL or a context, never a fault
    rng = np.random.default_rng(3)
    for _ in range(300):
        blob = bytearray(data)
        for pos in rng.integers(0, len(blob), size=rng.integers(1, 6)):
            blob[pos] = int(rng.integers(0, 256))
        opens(bytes(blob))
    assert not vl.vireo_gguf_open(str(tmp_path / "missing.gguf").encode())


def test_loader_metadata_errors(vl, tmp_path):
    """vireo_gguf_moe_load stops at the metadata, with -EINVAL and a message,
    for a dense model and for a file without a block count."""
    for drop, why in [("expert_count", "expert_count"), ("block_count", "block_count")]:
        w = G.GGUFWriter()
        w.add("general.architecture", G.STRING, "qwen3moe")
        for key, val in [("block_count", 1), ("embedding_length", 256), ("expert_count", 8)]:
            if key != drop:
                w.add(f"qwen3moe.{key}", G.U32, val)
        path = str(tmp_path / f"no_{drop}.gguf")
        w.write(path)
        out = C.POINTER(_lib.GGUFMoE)()
        rc = vl.vireo_gguf_moe_load(path.encode(), 0, 0, C.byref(out))
        assert rc == -errno.EINVAL and not out
        assert why in vl.vireo_gguf_moe_error().decode()
    out = C.POINTER(_lib.GGUFMoE)()
    assert vl.vireo_gguf_moe_load(str(tmp_path / "absent.gguf").encode(), 0, 0, C.byref(out)) == -errno.ENOENT


def test_whole_model_file_binds_in_the_reference(tmp_path):
    """write_model_gguf writes what the reference's forward() runs on: the
    reference binds the file (shape as written) and two fresh instances give the
    same bits for the same token sequence (the KV store starts empty)."""
    from oracle.oracle import Reference, RefModel
    if not Reference.available():
        pytest.skip("oracle/_ref not built")
    ref = Reference()
    path = tmp_path / "m.gguf"
    moe = W.MoEShape("m", 256, 8, 2, 256, True, W.Q4_K, W.Q4_K, W.Q6_K)
    G.write_model_gguf(str(path), "qwen3moe", 2, 256, 8, 2, 64, 300, 3, moe=moe, untied=True)
    runs = []
    for _ in range(2):
        r = RefModel(ref, path, block_tokens=4)
        assert (r.dim, r.vocab, r.n_layers, r.n_heads, r.n_kv_heads, r.head_size, r.is_moe) == (256, 300, 2, 8, 2,
                                                                                             64, 1)
        out = [r.forward(t, p, p >= 2) for p, t in enumerate([5, 6, 7, 8, 9])]
        runs.append(out)
        r.close()
    for (xa, la), (xb, lb) in zip(*runs):
        np.testing.assert_array_equal(xa, xb)
        if la is not None:
            assert np.isfinite(la).all()
            np.testing.assert_array_equal(la, lb)


def test_reader_under_sanitizers(vl, tmp_path):
    """The library's GGUF reader built with AddressSanitizer and
    UndefinedBehaviorSanitizer (host code only) reads the malformed files of
    test_reader_rejects_malformed - every truncation, bad magic and version,
    impossible counts, a zero alignment, random corruption - without a
    report, and accepts exactly the files the product library accepts."""
    import shutil
    import subprocess
    if not shutil.which("gcc"):
        pytest.skip("no gcc")
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    exe = str(tmp_path / "gguf_open_check")
    r = subprocess.run(["gcc", "-std=c11", "-O1", "-g", "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
                        "-fno-omit-frame-pointer", "-I", os.path.join(root, "include"),
                        os.path.join(root, "tests", "c", "gguf_open_check.c"),
                        os.path.join(root, "vireo_amd", "csrc", "gguf.c"), "-o", exe],
                       capture_output=True, text=True)
    if r.returncode != 0 and "asan" in (r.stderr or "").lower():
        pytest.skip("sanitizer runtime not available: " + r.stderr[-200:])
    assert r.returncode == 0, r.stderr
    path, data = small_file(tmp_path)
    blobs = [data[:n] for n in range(len(data) + 1)]
    blobs += [b"GGUG" + data[4:], data[:4] + struct.pack("<I", 1) + data[8:], data[:4] + struct.pack("<I", 4) + data[8:],
              data[:8] + struct.pack("<Q", 1 << 40) + data[16:]]
    w = G.GGUFWriter()
    w.add("general.alignment", G.U32, 0)
    zero = str(tmp_path / "zero.gguf")
    w.write(zero)
    blobs.append(open(zero, "rb").read())
    rng = np.random.default_rng(3)
    for _ in range(300):
        blob = bytearray(data)
        for pos in rng.integers(0, len(blob), size=rng.integers(1, 6)):
            blob[pos] = int(rng.integers(0, 256))
        blobs.append(bytes(blob))
    files = []
    for i, b in enumerate(blobs):
        fn = str(tmp_path / f"m{i}.gguf")
        with open(fn, "wb") as f:
            f.write(b)
        files.append(fn)
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0", UBSAN_OPTIONS="print_stacktrace=1")
    r = subprocess.run([exe, *files], capture_output=True, text=True, env=env, timeout=600)
    assert r.returncode == 0, r.stderr[-2000:]
    got = [int(x) for x in r.stdout.split()]
    want = []
    for fn in files:
        p = vl.vireo_gguf_open(fn.encode())
        want.append(int(bool(p)))
        if p:
            vl.vireo_gguf_close(p)
    assert got == want
