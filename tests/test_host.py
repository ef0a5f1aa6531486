"""CPU-side tests of the C-ABI library: it loads, exports every symbol that
include/llmcp_q8.h declares, its host packer (llmcp-pack's
quantizeTensorQ8_0Packed) matches the oracle byte for byte, and its arena
loader applies the reference's validation rules (PackedWeightsTest.cpp:186-223,
WeightArena.cpp:27-131).  No device is touched.
"""
import ctypes
import json
import os
import re
import struct

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    text = open(os.path.join(ROOT, "include", "llmcp_q8.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b((?:llmcp_q8|_mlir_ciface_llmcp_q8)_\w+)\s*\(", text)))


def test_library_exports_every_declared_symbol(q8):
    names = declared_functions()
    assert len(names) >= 30
    L = q8.lib()
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing
    assert set(names) == set(q8.EXPORTS)


def test_abi_version(q8):
    assert q8.lib().llmcp_q8_abi_version() == 7


def test_host_packer_matches_oracle(q8, oracle):
    rng = np.random.default_rng(21)
    for n, k in [(8, 32), (40, 320), (64, 2560)]:
        w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
        w[3, 32:64] = 0.0  # zero block -> d = 0
        assert np.array_equal(q8.pack_p4_host(w), oracle.pack_q8_0_p4(w))


def test_host_packer_rejects_unpackable(q8):
    with pytest.raises(q8.Declined):
        q8.pack_p4_host(np.zeros((12, 64), np.float32))


def _arena(tmp_path, q8, tensors):
    path = str(tmp_path / "w.bin")
    q8.write_arena(path, tensors)
    return np.fromfile(path, dtype=np.uint8)


def test_arena_round_trip(q8, oracle, tmp_path):
    rng = np.random.default_rng(22)
    a = oracle.pack_q8_0_p4((rng.standard_normal((16, 64)) * 0.02).astype(np.float32))
    b = oracle.pack_q8_0_p4((rng.standard_normal((8, 96)) * 0.02).astype(np.float32))
    f = _arena(tmp_path, q8, [("model.a.weight", 16, 64, a), ("model.b.weight", 8, 96, b)])
    assert bytes(f[:8]) == b"LLMCPWGT"
    version, hdr = struct.unpack_from("<II", f, 8)
    arena, moff, mbytes = struct.unpack_from("<QQQ", f, 16)
    assert (version, hdr) == (1, 64) and moff == arena and mbytes == f.size - arena
    manifest = json.loads(bytes(f[moff:]).decode())
    assert manifest["quantization"] == "q8_0" and manifest["quant_layout"] == "q8_0_p4"
    for entry, data in zip(manifest["tensors"], [a, b]):
        assert entry["offset"] % 64 == 0
        assert np.array_equal(f[entry["offset"]:entry["offset"] + entry["size"]], data)
    assert q8.arena_inspect(f) == (2, 2)


def _rewrite_manifest(f, edit):
    arena = struct.unpack_from("<Q", f, 16)[0]
    m = json.loads(bytes(f[arena:]).decode())
    edit(m)
    body = json.dumps(m).encode()
    out = np.concatenate([f[:arena], np.frombuffer(body, np.uint8)])
    struct.pack_into("<Q", out, 32, len(body))
    return out


@pytest.mark.parametrize("corruption", [
    "magic", "version", "header_size", "manifest_bounds", "json", "total",
    "block_size", "layout", "offset_align", "outside", "size", "dtype",
    "duplicate", "shape_rank",
])
def test_arena_rejects_corruption(q8, oracle, tmp_path, corruption):
    a = oracle.pack_q8_0_p4(np.ones((8, 64), np.float32))
    f = _arena(tmp_path, q8, [("t", 8, 64, a)]).copy()
    if corruption == "magic":
        f[0] = ord("X")
    elif corruption == "version":
        struct.pack_into("<I", f, 8, 2)
    elif corruption == "header_size":
        struct.pack_into("<I", f, 12, 32)
    elif corruption == "manifest_bounds":
        struct.pack_into("<Q", f, 32, 5)
    elif corruption == "json":
        arena = struct.unpack_from("<Q", f, 16)[0]
        f[arena] = ord("[")
    elif corruption == "total":
        f = _rewrite_manifest(f, lambda m: m.update(total_bytes=m["total_bytes"] + 64))
    elif corruption == "block_size":
        f = _rewrite_manifest(f, lambda m: m.update(block_size=16))
    elif corruption == "layout":
        f = _rewrite_manifest(f, lambda m: m.update(quant_layout="q8_0"))
    elif corruption == "offset_align":
        f = _rewrite_manifest(f, lambda m: m["tensors"][0].update(offset=96))
    elif corruption == "outside":
        f = _rewrite_manifest(f, lambda m: m["tensors"][0].update(offset=m["total_bytes"]))
    elif corruption == "size":
        f = _rewrite_manifest(f, lambda m: m["tensors"][0].update(size=m["tensors"][0]["size"] - 34))
    elif corruption == "dtype":
        f = _rewrite_manifest(f, lambda m: m["tensors"][0].update(dtype="Q4_0"))
    elif corruption == "duplicate":
        f = _rewrite_manifest(f, lambda m: m["tensors"].append(dict(m["tensors"][0])))
    elif corruption == "shape_rank":
        f = _rewrite_manifest(f, lambda m: m["tensors"][0].update(shape=[8 * 64]))
    with pytest.raises(q8.Q8Error) as e:
        q8.arena_inspect(f)
    assert e.value.code == q8.EFORMAT


def test_arena_accepts_mixed_dtypes(q8, tmp_path, oracle):
    a = oracle.pack_q8_0_p4(np.ones((8, 64), np.float32))
    f = _arena(tmp_path, q8, [("t", 8, 64, a)])

    def add_f32(m):
        m["tensors"].append({"name": "norm", "offset": 64, "size": 16,
                             "dtype": "F32", "shape": [4]})
    f2 = _rewrite_manifest(f, add_f32)
    assert q8.arena_inspect(f2) == (2, 1)


def consumer_binary():
    from llmcp_amd import build as b
    if not os.path.exists(b.CONSUMER):
        b.build_consumer()
    return b.CONSUMER


def test_cpp_consumer_host_part(q8, tmp_path):
    """A C++17 program that includes only llmcp_q8.h and links -lllmcp_q8
    (tests/c_consumer/q8_consumer.cpp) packs the matmul benchmark's all-ones
    rows, writes, maps and inspects an arena, and finds its tensors through
    the manifest, with no device touched."""
    import subprocess
    r = subprocess.run([consumer_binary(), "--cpu", str(tmp_path)],
                       capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "host part ok" in r.stdout


# Property tests of the arena validator on corrupted files: whatever the
# bytes, llmcp_q8_arena_inspect returns OK or LLMCP_Q8_EFORMAT and never
# reads outside the buffer it was given (each case runs on a copy cut to its
# exact length, so an over-read past the end would touch unmapped memory or
# garbage, not the original file's tail).
from hypothesis import HealthCheck, given, settings  # noqa: E402
from hypothesis import strategies as st  # noqa: E402


def _inspect_outcome(q8, f):
    try:
        n, nq = q8.arena_inspect(f)
    except q8.Q8Error as e:
        assert e.code == q8.EFORMAT, e
        return None
    assert 0 <= nq <= n
    return n, nq


@pytest.fixture(scope="module")
def fuzz_arena(q8, oracle, tmp_path_factory):
    rng = np.random.default_rng(5)
    a = oracle.pack_q8_0_p4((rng.standard_normal((16, 64)) * 0.02).astype(np.float32))
    b = oracle.pack_q8_0_p4((rng.standard_normal((8, 96)) * 0.02).astype(np.float32))
    path = str(tmp_path_factory.mktemp("fuzz") / "w.bin")
    q8.write_arena(path, [("model.a.weight", 16, 64, a), ("model.b.weight", 8, 96, b)])
    return np.fromfile(path, dtype=np.uint8)


_SETTINGS = settings(max_examples=400, deadline=None, derandomize=True,
                     suppress_health_check=[HealthCheck.function_scoped_fixture])


@_SETTINGS
@given(data=st.data())
def test_arena_fuzz_byte_mutations(q8, fuzz_arena, data):
    f = fuzz_arena.copy()
    edits = data.draw(st.lists(st.tuples(st.integers(0, f.size - 1), st.integers(0, 255)),
                               min_size=1, max_size=8))
    for pos, val in edits:
        f[pos] = val
    cut = data.draw(st.integers(0, f.size))
    _inspect_outcome(q8, np.array(f[:cut]))


@_SETTINGS
@given(data=st.data())
def test_arena_fuzz_manifest_text(q8, fuzz_arena, data):
    arena = struct.unpack_from("<Q", fuzz_arena, 16)[0]
    text = bytearray(fuzz_arena[arena:].tobytes())
    for _ in range(data.draw(st.integers(1, 4))):
        op = data.draw(st.sampled_from(["replace", "insert", "delete"]))
        pos = data.draw(st.integers(0, len(text) - 1))
        ch = data.draw(st.sampled_from(list(b'{}[]":,0123456789-.eE \\tnulfas') + [0, 0xff]))
        if op == "replace":
            text[pos] = ch
        elif op == "insert":
            text.insert(pos, ch)
        elif len(text) > 1:
            del text[pos]
    out = np.concatenate([fuzz_arena[:arena], np.frombuffer(bytes(text), np.uint8)])
    struct.pack_into("<Q", out, 32, len(text))
    _inspect_outcome(q8, out)


@_SETTINGS
@given(field=st.sampled_from(["offset", "size", "shape0", "shape1", "total_bytes",
                              "arena_offset", "manifest_bytes"]),
       value=st.one_of(st.integers(-2 ** 63, 2 ** 64 - 1),
                       st.sampled_from([2 ** 63 - 1, 2 ** 63, 2 ** 64 - 1, -1, 2 ** 32,
                                        2 ** 62, 3 * 2 ** 61])))
def test_arena_fuzz_numeric_extremes(q8, fuzz_arena, field, value):
    f = fuzz_arena.copy()
    if field in ("arena_offset", "manifest_bytes"):
        struct.pack_into("<Q", f, 16 if field == "arena_offset" else 32, value % 2 ** 64)
        _inspect_outcome(q8, f)
        return

    def edit(m):
        t = m["tensors"][1]
        if field == "total_bytes":
            m["total_bytes"] = value
        elif field.startswith("shape"):
            t["shape"][int(field[-1])] = value
        else:
            t[field] = value
    _inspect_outcome(q8, _rewrite_manifest(f, edit))


def test_model_arena_layout_matches_the_reference_pack():
    # WeightLayout::build restated for the 4B-class config: the reference's
    # own packing of the real model reports 426 tensors and 4,469,519,936
    # arena bytes (docs/int8-quantization.md:718-724).
    from llmcp_amd import model_arena
    entries, stride, groups, total = model_arena.layout()
    assert len(entries) == 426
    assert total == 4469519936
    assert groups == 8 and stride % 64 == 0
    assert sum(e["dtype"] == "Q8_0" for e in entries) == 249
    offsets = [e["offset"] for e in entries]
    assert offsets == sorted(offsets) and all(o % 64 == 0 for o in offsets)
    assert entries[0]["name"] == "model.language_model.embed_tokens.weight"
    assert entries[0]["dtype"] == "Q8_0" and entries[0]["size"] == 248320 * 2560 // 32 * 34


def test_model_arena_image_validates(q8):
    # a reduced model (4 layers, small vocab) built by the same code passes
    # the host validator with every tensor and dtype counted
    from llmcp_amd import model_arena
    cfg = dict(model_arena.CONFIG_4B, layers=4, vocab=1024, intermediate=512)
    image, entries = model_arena.build_image(cfg, seed=1)
    q8n = sum(e["dtype"] == "Q8_0" for e in entries)
    assert q8.arena_inspect(image) == (len(entries), q8n)
    assert {e["dtype"] for e in entries} == {"Q8_0", "BF16", "F32"}
