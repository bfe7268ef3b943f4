"""GGUF v3 reader, writer and config derivation (CPU; the GPU load is in test_gpu_model.py).

* The reference's own fixtures of the real 27B Q4_K_M file (tests/golden/gguf/, from the reference's
  tests/fixtures/: every metadata entry, tokenizer included, and the tensor index): a header written from them in
  the file's order must read back with the real file's data offset (10,995,296 B), every tensor's offset, size and
  shape as indexed, and the derived model config equal to the 27B config (tests/config_vs_fixture.rs of the
  reference). The data section is a sparse file; no tensor byte is read.
* The writer's layout of the 27B plan in the real file's tensor order gives the indexed offsets (alignment 32).
* The synthetic tiny model written to a GGUF file reads back with the plan's names, types, shapes and bytes, and
  its config derives to the tiny config.
* Malformed files (bad magic, truncation, misaligned or out-of-file tensors) are refused with an error code.
"""
import ctypes as C
import json
import lzma
import os
import struct

import numpy as np
import pytest

import aqueduct as aq

HERE = os.path.dirname(os.path.abspath(__file__))
GG = os.path.join(HERE, "golden", "gguf")
TYPES = {"UINT8": (0, "<B"), "INT8": (1, "<b"), "UINT16": (2, "<H"), "INT16": (3, "<h"), "UINT32": (4, "<I"),
         "INT32": (5, "<i"), "FLOAT32": (6, "<f"), "BOOL": (7, "<?"), "STRING": (8, None), "ARRAY": (9, None),
         "UINT64": (10, "<Q"), "INT64": (11, "<q"), "FLOAT64": (12, "<d")}


def gstr(s):
    b = s.encode("utf-8")
    return struct.pack("<Q", len(b)) + b


def gval(types, v):
    t = types[0]
    if t == "STRING":
        return gstr(v)
    if t == "ARRAY":
        et = types[1]
        out = struct.pack("<IQ", TYPES[et][0], len(v))
        if et == "STRING":
            return out + b"".join(gstr(x) for x in v)
        return out + np.asarray(v, dtype=np.dtype(TYPES[et][1])).tobytes()
    return struct.pack(TYPES[t][1], v)


def index():
    return json.load(open(os.path.join(GG, "gguf_index.json")))


def metadata():
    with lzma.open(os.path.join(GG, "gguf_metadata.json.xz"), "rt", encoding="utf-8") as f:
        return json.load(f)


def write_header_from_fixtures(path):
    """The real file's header, rebuilt from the fixtures, then a sparse data section of the real size."""
    idx, meta = index(), metadata()
    kv = [(k, v) for k, v in meta.items() if not k.startswith("GGUF.")]
    assert len(kv) == meta["GGUF.kv_count"]["value"]
    with open(path, "wb") as f:
        f.write(struct.pack("<IIQQ", 0x46554747, 3, len(idx["tensors"]), len(kv)))
        for k, v in kv:
            f.write(gstr(k) + struct.pack("<I", TYPES[v["types"][0]][0]) + gval(v["types"], v["value"]))
        for t in idx["tensors"]:
            dims = t["shape_gguf_order"]
            f.write(gstr(t["name"]) + struct.pack("<I", len(dims)) + struct.pack(f"<{len(dims)}Q", *dims) +
                    struct.pack("<IQ", t["ggml_type_id"], t["rel_offset"]))
        f.truncate(idx["file_size"])
    return idx


def cfg_dict(c):
    return {n: round(getattr(c, n), 9) if isinstance(getattr(c, n), float) else getattr(c, n)
            for n, _ in aq.AqModelConfig._fields_}


def test_reader_and_config_on_the_real_files_header(tmp_path):
    p = tmp_path / "real27b_header.gguf"
    idx = write_header_from_fixtures(p)
    g = aq.Gguf(p)
    info = g.info()
    assert info["data_offset"] == idx["data_offset"] == 10995296
    assert info["alignment"] == idx["alignment"] == 32 and info["n_tensors"] == 866
    got = g.tensors()
    assert [e[0] for e in got] == [t["name"] for t in idx["tensors"]]
    for (name, ty, rows, cols, off, nb), t in zip(got, idx["tensors"]):
        shp = t["shape_numpy_order"]
        assert (ty, off, nb) == (t["ggml_type_id"], t["rel_offset"], t["byte_size"]), name
        assert (rows, cols) == ((shp[0], shp[1]) if len(shp) == 2 else (1, shp[0])), name
    assert g.get_str("general.architecture") == "qwen35" and g.get_u32("qwen35.block_count") == 65
    assert g.get_f32("qwen35.rope.freq_base") == 1e7
    assert cfg_dict(g.model_config()) == cfg_dict(aq.config_27b())
    g.close()


def test_writer_layout_of_the_27b_plan_gives_the_real_offsets():
    idx = index()
    plan = dict(aq.model_plan(aq.config_27b(), aq.MIX_Q4_K_M, 1))
    order = [(t["name"], plan[t["name"]]) for t in idx["tensors"]]
    off = aq.gguf_layout(order, 32)
    assert off.tolist() == [t["rel_offset"] for t in idx["tensors"]]


def test_synthetic_tiny_model_round_trip(tmp_path):
    cfg = aq.tiny_config()
    p = tmp_path / "tiny.gguf"
    aq.gguf_write_synth(p, cfg, aq.MIX_TINY, 1234, threads=4)
    g = aq.Gguf(p)
    plan = aq.model_plan(cfg, aq.MIX_TINY, 1234)
    got = g.tensors(with_data=True)
    assert [e[0] for e in got] == [n for n, _ in plan]
    for (name, ty, rows, cols, off, nb, data), (_, sp) in zip(got, plan):
        assert (ty, rows, cols) == (sp.ggml_type, sp.rows, sp.cols), name
        assert off % 32 == 0
        assert np.array_equal(data, aq.synth_host(sp).view(np.uint8)), name
    assert cfg_dict(g.model_config()) == cfg_dict(cfg)
    assert g.get_u32("general.alignment") == 32
    g.close()


def test_malformed_files_are_refused(tmp_path):
    L = aq.lib()
    h = C.c_void_p()
    bad = tmp_path / "bad.gguf"
    bad.write_bytes(b"NOPE" + b"\0" * 40)
    assert L.aq_gguf_open(os.fsencode(bad), C.byref(h)) == -1
    assert b"magic" in L.aq_last_error()
    good = tmp_path / "tiny.gguf"
    aq.gguf_write_synth(good, aq.tiny_config(), aq.MIX_TINY, 5, threads=2)
    raw = good.read_bytes()
    trunc = tmp_path / "trunc.gguf"
    trunc.write_bytes(raw[:4000])  # inside the metadata
    assert L.aq_gguf_open(os.fsencode(trunc), C.byref(h)) < 0
    short = tmp_path / "short.gguf"
    short.write_bytes(raw[:-100])  # the last tensor runs past the end
    assert L.aq_gguf_open(os.fsencode(short), C.byref(h)) < 0
    assert b"past the end" in L.aq_last_error()
    assert L.aq_gguf_open(os.fsencode(tmp_path / "missing.gguf"), C.byref(h)) < 0


def one_tensor_file(path, dims, ggml_type, rel_offset, kv=b"", n_kv=0, data=b"\0" * 256):
    """A GGUF v3 file with the given metadata bytes and one tensor info `w` (alignment 32), then `data`."""
    head = b"GGUF" + struct.pack("<IQQ", 3, 1, n_kv) + kv
    head += gstr("w") + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
    head += struct.pack("<IQ", ggml_type, rel_offset)
    head += b"\0" * (-len(head) % 32)
    path.write_bytes(head + data)


def test_crafted_offsets_counts_and_arrays_are_refused(tmp_path):
    """Header fields a crafted file can make wrap in 64 bits are refused with AQ_EINVAL before anything is read or
    reserved: a tensor offset near 2^64 (a multiple of the alignment, so offset + size wraps below the file size), an
    element count whose dimension product overflows, and a metadata array whose count exceeds what the bytes left
    could hold (no allocation is attempted for it). The same file with sane fields opens."""
    L = aq.lib()
    h = C.c_void_p()
    p = tmp_path / "ok.gguf"
    one_tensor_file(p, [32], 0, 0)  # 32 F32 values at offset 0: inside the 256 data bytes
    g = aq.Gguf(p)
    assert g.tensors()[0][4:] == (0, 128)
    g.close()
    for name, dims, off in [("wrap_offset", [32], (1 << 64) - 32), ("wrap_count", [1 << 33, 1 << 33], 0),
                            ("count_times_size", [1 << 62], 0)]:
        p = tmp_path / f"{name}.gguf"
        one_tensor_file(p, dims, 0, off)
        rc = L.aq_gguf_open(os.fsencode(p), C.byref(h))
        assert rc == aq.AQ_EINVAL or rc == aq.AQ_EUNSUP, (name, rc)
        assert rc != aq.AQ_EUNSUP or b"not supported" in L.aq_last_error()
    # an array of 2^40 UINT64 values in a file of a few hundred bytes
    kv = gstr("general.bad") + struct.pack("<IIQ", 9, 10, 1 << 40)
    p = tmp_path / "big_array.gguf"
    one_tensor_file(p, [32], 0, 0, kv=kv, n_kv=1)
    assert L.aq_gguf_open(os.fsencode(p), C.byref(h)) == aq.AQ_EINVAL
