"""Adapter checkpoints of the host mirror (sa3.cpp_amd/host/sa3/train_checkpoint.h: the reference's
write_train_lora_gguf / load_train_lora_gguf, src/train_checkpoint.h:38-173) against the GGUF v3
format and the adapter contract (docs/lora_checkpoint_contract.md).

The reference writes these files with ggml's gguf code, which is not in the reference tree, so no
reference-written file exists to compare with. Parity is pinned by the format itself: a GGUF parser
and a GGUF writer written here from the published layout (independent of gguf_io.h) check every
byte the mirror writes and produce files the mirror must read (f16 tensors, array metadata, a
non-default alignment, unrelated tensors, a missing adapter type), and tests/host/checkpoint_test.cpp
covers the round trip and every rejected input.

The trainer-state sidecar and the checkpoint pair (sa3.cpp_amd/host/sa3/train_resume.h; the
reference's src/train_resume.h:23-538) are checked the same way: the sidecar's keys, value types,
arrays and moment tensors against the published layout, and the pair's contract (immutable,
resolvable from either file, bound to its adapter by fingerprint, exact RNG continuation) with the
inputs of the reference's tests/train_checkpoint_test.cpp.
"""
import os
import struct
import subprocess

import numpy as np
import pytest

from conftest import PKG, ROOT

SRC = os.path.join(ROOT, "tests", "host", "checkpoint_test.cpp")
KV_SCALAR = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<?", 10: "<Q", 11: "<q", 12: "<d"}


@pytest.fixture(scope="module")
def tool(tmp_path_factory):
    out = str(tmp_path_factory.mktemp("ckpt") / "checkpoint_test")
    cmd = ["g++", "-std=c++17", "-O1", "-Wall", "-Wextra", "-Werror", "-I", os.path.join(ROOT, "include"),
           "-I", os.path.join(PKG, "host"), SRC, "-o", out]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-4000:]
    return out


def parse_gguf(data):
    """GGUF v3 from the published layout: header, metadata, tensor infos, aligned data section."""
    pos = 0

    def take(fmt):
        nonlocal pos
        v = struct.unpack_from(fmt, data, pos)
        pos += struct.calcsize(fmt)
        return v[0]

    def string():
        nonlocal pos
        n = take("<Q")
        s = data[pos:pos + n].decode()
        pos += n
        return s

    arr_types = {}

    def value(t, key=None):
        if t == 8:
            return string()
        if t == 9:
            et, n = take("<I"), take("<Q")
            if key is not None:
                arr_types[key] = et
            return [value(et) for _ in range(n)]
        return take(KV_SCALAR[t])

    assert data[:4] == b"GGUF"
    pos = 4
    version, n_t, n_kv = take("<I"), take("<Q"), take("<Q")
    kv, kv_types = {}, {}
    for _ in range(n_kv):
        k = string()
        t = take("<I")
        kv[k], kv_types[k] = value(t, k), t
    infos = []
    for _ in range(n_t):
        name = string()
        nd = take("<I")
        ne = [take("<Q") for _ in range(nd)]
        infos.append((name, ne, take("<I"), take("<Q")))
    align = kv.get("general.alignment", 32)
    meta_end = pos
    start = (pos + align - 1) // align * align
    return dict(version=version, kv=kv, kv_types=kv_types, arr_types=arr_types, infos=infos, start=start,
                meta_end=meta_end, align=align)


def write_gguf(path, kvs, tensors, align=32):
    """kvs: [(key, type, value)], tensors: [(name, ne, np array f32/f16)]"""
    out = bytearray(b"GGUF") + struct.pack("<IQQ", 3, len(tensors), len(kvs))

    def s(x):
        b = x.encode()
        return struct.pack("<Q", len(b)) + b

    for k, t, v in kvs:
        out += s(k) + struct.pack("<I", t)
        if t == 8:
            out += s(v)
        elif t == 9:
            et, items = v
            out += struct.pack("<IQ", et, len(items))
            for it in items:
                out += s(it) if et == 8 else struct.pack(KV_SCALAR[et], it)
        else:
            out += struct.pack(KV_SCALAR[t], v)
    off = 0
    blobs = []
    for name, ne, arr in tensors:
        ty = 0 if arr.dtype == np.float32 else 1
        out += s(name) + struct.pack("<I", len(ne)) + b"".join(struct.pack("<Q", e) for e in ne)
        out += struct.pack("<IQ", ty, off)
        b = arr.tobytes()
        blobs.append(b)
        off += (len(b) + align - 1) // align * align
    out += b"\0" * ((-len(out)) % align)
    for b in blobs:
        out += b + b"\0" * ((-len(b)) % align)
    open(path, "wb").write(bytes(out))


def val(t, kind, k):
    return np.float32(t * 1000 + kind * 100) + np.float32(k % 97) * np.float32(0.25) - np.float32(7.0)


def test_mirror_file_matches_gguf_layout_and_contract(tool, tmp_path):
    path = str(tmp_path / "adapter.gguf")
    assert subprocess.run([tool, "write", path], capture_output=True).returncode == 0
    data = open(path, "rb").read()
    g = parse_gguf(data)
    assert g["version"] == 3
    # the contract's metadata, with the reference's value types (string, u32, f32)
    assert g["kv"] == {"general.architecture": "sa3-lora", "general.name": "sa3 native trained adapter",
                       "lora.adapter_type": "dora-rows", "lora.rank": 4, "lora.alpha": 6.5, "lora.n_targets": 3}
    assert [g["kv_types"][k] for k in ("general.architecture", "lora.rank", "lora.alpha", "lora.n_targets")] == [8, 4, 6, 4]
    # tensors in state order, per target lora_A [in, rank], lora_B [rank, out], magnitude [out], f32
    stems = [("dit.1.self.qkv", 16, 40), ("dit.0.ff.out", 24, 16), ("dit.proj_in", 8, 12)]
    want = []
    for t, (s, i, o) in enumerate(stems):
        want += [(f"{s}.lora_A", [i, 4], 0), (f"{s}.lora_B", [4, o], 1), (f"{s}.magnitude", [o], 5)]
    assert [(n, ne) for n, ne, _, _ in g["infos"]] == [(n, ne) for n, ne, _ in want]
    assert all(ty == 0 for _, _, ty, _ in g["infos"])
    # offsets aligned, packed in order, zero padding, data = the written values, nothing after
    assert g["meta_end"] <= g["start"] and not any(data[g["meta_end"]:g["start"]])
    expect_off = 0
    for (name, ne, _, off), (_, _, kind) in zip(g["infos"], want):
        assert off == expect_off and off % 32 == 0, name
        n = int(np.prod(ne))
        arr = np.frombuffer(data, np.float32, n, g["start"] + off)
        t = [s for s, _, _ in stems].index(name.rsplit(".", 1)[0])
        assert np.array_equal(arr, [val(t, kind, k) for k in range(n)]), name
        pad = (-(4 * n)) % 32
        assert not any(data[g["start"] + off + 4 * n:g["start"] + off + 4 * n + pad])
        expect_off += 4 * n + pad
    assert len(data) == g["start"] + expect_off


def summary(tool, path):
    r = subprocess.run([tool, "read", path], capture_output=True, text=True)
    return r.returncode, r.stdout.strip().splitlines()


def checksum(v):
    v = np.asarray(v, np.float64).ravel()
    return float(np.sum(v * (np.arange(v.size) % 13 + 1)))


def test_mirror_reads_an_independently_written_file(tool, tmp_path):
    # f16 magnitudes, an array-valued key (skipped), alignment 64, a bias tensor that is not an
    # adapter tensor, no lora.adapter_type (defaults to "lora"), stems out of order
    rng = np.random.default_rng(3)
    A1, B1 = rng.normal(0, 1, (8, 48)).astype(np.float32), rng.normal(0, 1, (20, 8)).astype(np.float32)
    A0, B0 = rng.normal(0, 1, (8, 32)).astype(np.float32), rng.normal(0, 1, (24, 8)).astype(np.float32)
    m0 = rng.normal(1, 0.1, 24).astype(np.float16)
    path = str(tmp_path / "ext.gguf")
    write_gguf(path, [("general.alignment", 4, 64), ("general.architecture", 8, "sa3-lora"),
                      ("general.tags", 9, (8, ["a", "bc"])), ("lora.rank", 4, 8), ("lora.alpha", 6, 16.0),
                      ("other.ints", 9, (5, [1, -2, 3]))],
               [("dit.5.cross.q.lora_A", [48, 8], A1), ("dit.5.cross.q.lora_B", [8, 20], B1),
                ("dit.5.cross.q.bias", [20], np.ones(20, np.float32)),
                ("dit.0.self.out.lora_B", [8, 24], B0), ("dit.0.self.out.magnitude", [24], m0),
                ("dit.0.self.out.lora_A", [32, 8], A0)], align=64)
    rc, lines = summary(tool, path)
    assert rc == 0, lines
    assert lines[0] == "type=lora rank=8 alpha=16 targets=2"

    def line(stem, i, o, A, B, m):
        return (f"{stem} in={i} out={o} A={A.size}:{checksum(A):.17g} B={B.size}:{checksum(B):.17g} "
                f"m={m.size}:{checksum(m):.17g}")
    got = [l.split() for l in lines[1:]]
    for g_, w in zip(got, [line("dit.0.self.out", 32, 24, A0, B0, m0.astype(np.float32)),
                           line("dit.5.cross.q", 48, 20, A1, B1, np.zeros(0))]):
        assert g_[:4] == w.split()[:4]
        for a, b in zip(g_[4:], w.split()[4:]):   # size:checksum, summed in the same order
            (na, sa), (nb, sb) = a.split(":"), b.split(":")
            assert na == nb and abs(float(sa) - float(sb)) <= 1e-9 * max(1.0, abs(float(sb))), (a, b)


def test_round_trip_and_rejections(tool, tmp_path):
    r = subprocess.run([tool, "errors", str(tmp_path)], capture_output=True, text=True)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "checkpoint_test: ok" in r.stdout


def test_rejects_unsupported_tensor_type(tool, tmp_path):
    path = str(tmp_path / "q.gguf")
    write_gguf(path, [("lora.rank", 4, 2), ("lora.alpha", 6, 1.0)],
               [("x.lora_A", [4, 2], np.zeros(8, np.float32))])
    data = bytearray(open(path, "rb").read())
    i = data.find(b"x.lora_A") + 8 + 4 + 16     # name, n_dims, ne -> the type field
    data[i:i + 4] = struct.pack("<I", 8)         # a quantised type
    open(path, "wb").write(bytes(data))
    rc, lines = summary(tool, path)
    assert rc == 1 and "unsupported type" in lines[0]


def test_full_scope_adapter_write_read_time(tool, tmp_path):
    # host cost of an adapter checkpoint at the DiT's full scope (180 targets, rank 32, ~154 MB)
    r = subprocess.run([tool, "bench", str(tmp_path / "big.gguf")], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    print(r.stdout.strip())


@pytest.mark.parametrize("patch", ["zero_extent", "huge_extent", "product_overflow", "offset_wrap", "offset_past_end",
                                   "alignment"])
def test_rejects_malformed_extents_and_offsets(tool, tmp_path, patch):
    # tensor infos from an untrusted file: extents must be in [1, 2^62) with an int64 product, and
    # offset + bytes must stay inside the data section; the alignment must be a power of two
    path = str(tmp_path / "m.gguf")
    write_gguf(path, [("general.alignment", 4, 32), ("lora.rank", 4, 2), ("lora.alpha", 6, 1.0)],
               [("x.lora_A", [4, 2], np.zeros(8, np.float32)), ("x.lora_B", [2, 3], np.zeros(6, np.float32))])
    data = bytearray(open(path, "rb").read())
    i = data.find(b"x.lora_A") + 8 + 4          # the first extent of x.lora_A
    ty_off = i + 16                              # type, then the u64 offset
    if patch == "zero_extent":
        data[i:i + 8] = struct.pack("<Q", 0)
    elif patch == "huge_extent":
        data[i:i + 8] = struct.pack("<Q", 1 << 62)
    elif patch == "product_overflow":
        data[i:i + 16] = struct.pack("<QQ", (1 << 61) + 1, 1 << 4)
    elif patch == "offset_wrap":
        data[ty_off + 4:ty_off + 12] = struct.pack("<Q", (1 << 64) - 16)
    elif patch == "offset_past_end":
        data[ty_off + 4:ty_off + 12] = struct.pack("<Q", len(data))
    else:
        j = data.find(b"general.alignment") + len(b"general.alignment") + 4
        data[j:j + 4] = struct.pack("<I", 48)
    open(path, "wb").write(bytes(data))
    rc, lines = summary(tool, path)
    assert rc == 1, lines


def test_trainer_state_sidecar_layout(tool, tmp_path):
    path = str(tmp_path / "trainer-state-step-3.gguf")
    assert subprocess.run([tool, "state", path], capture_output=True).returncode == 0
    data = open(path, "rb").read()
    g = parse_gguf(data)
    kv, ty = g["kv"], g["kv_types"]
    # the reference's keys and value types (src/train_resume.h:346-366): u32 = 4, u64 = 10, string = 8
    assert kv["general.architecture"] == "sa3-trainer-state" and ty["general.architecture"] == 8
    assert kv["general.name"] == "sa3 native trainer continuation state"
    assert kv["trainer.state_version"] == 1 and ty["trainer.state_version"] == 4
    for k, v in (("trainer.step", 3), ("trainer.epoch", 2), ("trainer.next_sample", 1)):
        assert kv[k] == v and ty[k] == 10, k
    assert kv["trainer.n_targets"] == 1 and ty["trainer.n_targets"] == 4
    assert kv["trainer.adapter_file"] == "adapter-step-3.gguf"
    assert kv["trainer.adapter_fingerprint"] == "fnv1a64:0123456789abcdef"
    assert kv["trainer.compatibility"] == "test-compatibility"
    # an mt19937_64 in the standard stream format: 312 words and the position
    for k in ("shuffle", "crop", "cfg", "prompt", "inpaint"):
        assert len(kv[f"trainer.rng.{k}"].split()) == 313 and ty[f"trainer.rng.{k}"] == 8
    assert ty["trainer.rng.diffusion"] == 8 and kv["trainer.rng.diffusion"]
    assert kv["trainer.order"] == [1, 0] and ty["trainer.order"] == 9 and g["arr_types"]["trainer.order"] == 10
    assert kv["trainer.targets"] == ["dit.0.self.qkv"] and g["arr_types"]["trainer.targets"] == 8
    # moments: optimizer.<stem>.<kind>.m / .v, 1-D f32, in visit order
    names = [(n, ne, t) for n, ne, t, _ in g["infos"]]
    assert names == [("optimizer.dit.0.self.qkv.lora_A.m", [6], 0), ("optimizer.dit.0.self.qkv.lora_A.v", [6], 0),
                     ("optimizer.dit.0.self.qkv.lora_B.m", [10], 0), ("optimizer.dit.0.self.qkv.lora_B.v", [10], 0)]
    off = dict((n, o) for n, _, _, o in g["infos"])
    k = np.arange(6, dtype=np.float32)
    m = np.frombuffer(data, np.float32, 6, g["start"] + off["optimizer.dit.0.self.qkv.lora_A.m"])
    assert np.array_equal(m, np.float32(1.0) + np.float32(0.125) * k)


def test_checkpoint_pair_contract(tool, tmp_path):
    r = subprocess.run([tool, "resume", str(tmp_path)], capture_output=True, text=True)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "checkpoint_test resume: ok" in r.stdout
