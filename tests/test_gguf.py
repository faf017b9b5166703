"""GGUF loader (include/qwen35_gguf.h, include/loader_gguf.hpp).

CPU: files written by tests/gguf_writer.py are parsed through the C ABI --
metadata text as the reference stores it (src/loader_gguf.cpp:155-175:
std::to_string, "true"/"false", strings verbatim, arrays element-wise),
tensor infos and sizes (GGML block tables), the aligned payload start, and
every rejection the reference makes with its message (:17-26, :61-101,
:189-306). GPU: the upload (device bytes equal the file bytes, 256-byte aligned
slots in one arena, blk.N filtering as :331-343) and the loaded Q4_K / Q6_K
tables through the dequant-gather and the GEMV against the oracle.
"""

from __future__ import annotations

import struct

import numpy as np
import pytest

import gguf_writer as gw
from qwen35_hip import _lib
from qwen35_hip.gguf import GgufFile
from qwen35_hip._lib import QwenError

Q4_K, Q6_K, Q8_0, Q4_0, F32, F16, BF16 = 12, 14, 8, 2, 0, 1, 30

META = [
    ("general.architecture", gw.STR, "qwen35moe"),
    ("general.name", gw.STR, "unit-test model é中"),
    ("qwen35moe.block_count", gw.U32, 3),
    ("qwen35moe.rope.freq_base", gw.F32, 10000000.0),
    ("qwen35moe.attention.layer_norm_rms_epsilon", gw.F32, 1e-6),
    ("u8", gw.U8, 255), ("i8", gw.I8, -128), ("u16", gw.U16, 65535), ("i16", gw.I16, -32768),
    ("i32", gw.I32, -2147483648), ("u64", gw.U64, 2 ** 64 - 1), ("i64", gw.I64, -2 ** 63),
    ("f64", gw.F64, 3.14159265358979), ("f32.small", gw.F32, 1.5e-7), ("b.true", gw.BOOL, 1), ("b.false", gw.BOOL, 0),
    ("empty", gw.STR, ""),
    ("qwen35moe.rope.dimension_sections", gw.ARR, (gw.I32, [11, 11, 10, 0])),
    ("tokenizer.ggml.tokens", gw.ARR, (gw.STR, ["<|a|>", "b", "", "Ġthe"])),
    ("floats", gw.ARR, (gw.F32, [0.5, -2.25, 1e-3])),
    ("bools", gw.ARR, (gw.BOOL, [1, 0])),
    ("none", gw.ARR, (gw.U8, [])),
]


def _tensors(rng, layers=3):
    ts = [("token_embd.weight", (2048, 64), Q4_K), ("output_norm.weight", (2048,), F32),
          ("output.weight", (2048, 48), Q6_K)]
    for i in range(layers):
        ts += [(f"blk.{i}.attn_norm.weight", (2048,), F32), (f"blk.{i}.attn_qkv.weight", (2048, 96), Q8_0),
               (f"blk.{i}.ffn_down.weight", (512, 64), Q4_0), (f"blk.{i}.ssm_a", (32,), F16),
               (f"blk.{i}.x.weight", (256, 3), BF16)]
    out = []
    for name, shape, t in ts:
        n = int(np.prod(shape))
        out.append((name, shape, t, gw.random_tensor_bytes(rng, t, n)))
    return out


def _write(tmp_path, name, data: bytes):
    p = tmp_path / name
    p.write_bytes(data)
    return p


def _expect_text(vtype, v):
    if vtype in (gw.F32, gw.F64):
        return gw.to_string_float(np.float32(v) if vtype == gw.F32 else v)
    if vtype == gw.BOOL:
        return "true" if v else "false"
    return str(v)


def _size(t, n):
    import ggml_blocks

    if t in ggml_blocks.BLOCK:
        e, b = ggml_blocks.BLOCK[t]
        return n // e * b
    return n * {F32: 4, F16: 2, BF16: 2}[t]


def test_parse_metadata_and_tensor_infos(tmp_path):
    rng = np.random.default_rng(0)
    ts = _tensors(rng)
    p = _write(tmp_path, "m.gguf", gw.build(META, ts))
    with GgufFile(p) as f:
        info = f.info()
        assert info["version"] == 3 and info["tensor_count"] == len(ts) and info["metadata_count"] == len(META)
        assert info["device_bytes"] == 0 and info["payload_offset"] % 32 == 0
        assert f.keys() == [(k, t == gw.ARR) for k, t, _ in META]
        for k, t, v in META:
            if t == gw.ARR:
                et, items = v
                assert f.meta(k) is None
                assert f.meta_array(k) == [_expect_text(et, x) if et != gw.STR else x for x in items]
            else:
                assert f.meta_array(k) is None
                assert f.meta(k) == (v if t == gw.STR else _expect_text(t, v)), k
        assert f.meta("absent") is None and f.meta_array("absent") is None
        assert f.meta("qwen35moe.rope.freq_base") == "10000000.000000"
        assert f.meta("qwen35moe.attention.layer_norm_rms_epsilon") == "0.000001"
        got = f.tensors()
        pos = 0
        for g, (name, shape, t, data) in zip(got, ts):
            assert (g.name, g.type, g.shape) == (name, t, shape)
            assert g.num_elements == int(np.prod(shape)) and g.size_bytes == len(data) == _size(t, g.num_elements)
            pos = (pos + 31) // 32 * 32
            assert g.offset == pos and g.device_ptr is None
            pos += len(data)
            assert f.find(name) == got.index(g)
        assert f.find("nope") == -1


def test_alignment_and_version2(tmp_path):
    rng = np.random.default_rng(1)
    ts = _tensors(rng, layers=1)
    meta = [("general.alignment", gw.U32, 256)]
    data = gw.build(meta, ts, alignment=256, version=2)
    with GgufFile(_write(tmp_path, "a.gguf", data)) as f:
        assert f.info()["version"] == 2 and f.info()["payload_offset"] % 256 == 0
        for g in f.tensors():
            assert g.offset % 256 == 0
        payload = f.info()["payload_offset"]
        for g, (_, _, _, d) in zip(f.tensors(), ts):
            assert data[payload + g.offset:payload + g.offset + g.size_bytes] == d


def _status(path):
    lib = _lib.load()
    import ctypes

    h = ctypes.c_void_p()
    st = lib.qwen_gguf_open(str(path).encode(), ctypes.byref(h))
    msg = lib.qwen_last_error().decode()
    if st == 0:
        lib.qwen_gguf_close(h)
    return st, msg


T1 = [("t.weight", (256, 2), Q4_K, bytes(288))]
HDR01 = b"GGUF" + struct.pack("<IQQ", 3, 0, 1)   # v3, no tensors, one metadata pair


@pytest.mark.parametrize("case,status,message", [
    ("missing", _lib.STATUS_IO_ERROR, "cannot open"),
    ("magic", _lib.STATUS_IO_ERROR, "cannot open"),
    ("version1", _lib.STATUS_MALFORMED, "unsupported GGUF version 1"),
    ("version4", _lib.STATUS_MALFORMED, "unsupported GGUF version 4"),
    ("counts", _lib.STATUS_MALFORMED, "unreasonable GGUF header counts"),
    ("trunc_header", _lib.STATUS_MALFORMED, "truncated GGUF while reading tensor count"),
    ("trunc_string", _lib.STATUS_MALFORMED, "truncated GGUF string"),
    ("long_string", _lib.STATUS_MALFORMED, "unreasonable GGUF string length"),
    ("dup_key", _lib.STATUS_MALFORMED, "duplicate GGUF metadata key: k"),
    ("bad_vtype", _lib.STATUS_MALFORMED, "Unknown GGUF metadata value type"),
    ("nested", _lib.STATUS_MALFORMED, "nested GGUF arrays are unsupported"),
    ("big_array", _lib.STATUS_MALFORMED, "invalid GGUF metadata array"),
    ("dup_tensor", _lib.STATUS_MALFORMED, "duplicate GGUF tensor name: t.weight"),
    ("dims0", _lib.STATUS_MALFORMED, "invalid dimensions for tensor t.weight"),
    ("dims5", _lib.STATUS_MALFORMED, "invalid dimensions for tensor t.weight"),
    ("dim_neg", _lib.STATUS_MALFORMED, "invalid or overflowing shape for tensor t.weight"),
    ("dim_overflow", _lib.STATUS_MALFORMED, "invalid or overflowing shape for tensor t.weight"),
    ("type99", _lib.STATUS_MALFORMED, "unsupported or malformed tensor 't.weight' (GGML type 99)"),
    ("row_width", _lib.STATUS_MALFORMED, "quantized row width is not block-aligned for tensor t.weight"),
    ("alignment3", _lib.STATUS_MALFORMED, "invalid GGUF alignment"),
    ("misaligned", _lib.STATUS_MALFORMED, "invalid data range for tensor t.weight"),
    ("past_eof", _lib.STATUS_MALFORMED, "invalid data range for tensor t.weight"),
    ("overlap", _lib.STATUS_MALFORMED, "overlapping GGUF tensors: a.weight and b.weight"),
    ("trunc_tensor_info", _lib.STATUS_MALFORMED, "truncated GGUF while reading tensor type"),
])
def test_rejections(tmp_path, case, status, message):
    """Each malformed file is rejected with the reference's status class (open()
    returning false vs throwing) and message."""
    meta = [("k", gw.U32, 1)]
    if case == "missing":
        p = tmp_path / "absent.gguf"
    else:
        if case == "magic":
            data = gw.build(meta, T1, magic=b"GGUX")
        elif case == "version1":
            data = gw.build(meta, T1, version=1)
        elif case == "version4":
            data = gw.build(meta, T1, version=4)
        elif case == "counts":
            data = gw.build(meta, T1, counts=(1, (1 << 24) + 1))
        elif case == "trunc_header":
            data = b"GGUF" + struct.pack("<I", 3) + b"\x01\x00"
        elif case == "trunc_string":
            data = b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + struct.pack("<Q", 100) + b"abc"
        elif case == "long_string":
            data = b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + struct.pack("<Q", (1 << 32) + 1) + b"abc"
        elif case == "dup_key":
            data = gw.build(meta + meta, T1)
        elif case == "bad_vtype":
            data = HDR01 + gw.gguf_string("x") + struct.pack("<I", 13)
        elif case == "nested":
            data = HDR01 + gw.gguf_string("x") + struct.pack("<IIQ", gw.ARR, gw.ARR, 1)
        elif case == "big_array":
            data = HDR01 + gw.gguf_string("x") + struct.pack("<IIQ", gw.ARR, gw.U8, (1 << 32) + 1)
        elif case == "dup_tensor":
            data = gw.build(meta, T1 + T1)
        elif case == "dims0":
            data = gw.build(meta, [("t.weight", (), Q4_K, b"")])
        elif case == "dims5":
            data = gw.build(meta, [("t.weight", (256, 1, 1, 1, 1), Q4_K, bytes(144))])
        elif case == "dim_neg":
            data = gw.build(meta, [("t.weight", (256, -1), Q4_K, bytes(144))])
        elif case == "dim_overflow":
            data = gw.build(meta, [("t.weight", (2 ** 40, 2 ** 40), F32, bytes(4))])
        elif case == "type99":
            data = gw.build(meta, [("t.weight", (256, 2), 99, bytes(288))])
        elif case == "row_width":
            data = gw.build(meta, [("t.weight", (128, 2), Q4_K, bytes(144))])
        elif case == "alignment3":
            data = gw.build([("general.alignment", gw.U32, 3)], T1)
        elif case == "misaligned":
            data = gw.build(meta, T1, offsets=[16])
        elif case == "past_eof":
            data = gw.build(meta, T1)[:-1]
        elif case == "overlap":
            data = gw.build(meta, [("a.weight", (256, 2), Q4_K, bytes(288)), ("b.weight", (256,), Q4_K, bytes(144))],
                            offsets=[0, 256])
        elif case == "trunc_tensor_info":
            full = gw.build(meta, T1)
            data = full[:full.index(b"t.weight") + len("t.weight") + 4 + 16 + 2]
        p = _write(tmp_path, case + ".gguf", data)
    st, msg = _status(p)
    assert st == status and message in msg, (st, msg)


def test_alignment_text_rules(tmp_path):
    """general.alignment goes through std::stoi of its text like the reference:
    a string "64" counts, an unparsable one falls back to 32."""
    for value, vtype, align in (("64", gw.STR, 64), ("x", gw.STR, 32), (64, gw.U64, 64)):
        data = gw.build([("general.alignment", vtype, value)], T1, alignment=align)
        with GgufFile(_write(tmp_path, "al.gguf", data)) as f:
            assert f.info()["payload_offset"] % align == 0


def test_load_after_truncation_is_an_io_error(tmp_path):
    """A file cut short between open and load: the upload re-maps it and finds a
    tensor past the new end before any device call, so this runs on the CPU.
    The reference's read reports the failure instead of faulting
    (src/loader_gguf.cpp:355-360)."""
    rng = np.random.default_rng(6)
    ts = _tensors(rng, layers=1)
    data = gw.build(META, ts)
    p = _write(tmp_path, "cut.gguf", data)
    with GgufFile(p) as f:
        last = max(f.tensors(), key=lambda g: g.offset)
        with open(p, "r+b") as fh:
            fh.truncate(len(data) - 7)
        with pytest.raises(QwenError) as e:
            f.load()
        assert e.value.status == _lib.STATUS_IO_ERROR, e.value
        assert "cannot re-read GGUF file" in str(e.value) and last.name in str(e.value)
        assert f.info()["device_bytes"] == 0 and all(g.device_ptr is None for g in f.tensors())


# ------------------------------------------------------------------ device upload
@pytest.mark.gpu
def test_load_bytes_and_layer_filter(tmp_path):
    import torch

    rng = np.random.default_rng(5)
    ts = _tensors(rng, layers=3)
    # one tensor larger than a staging buffer (64 MB): 100000 x 1024 Q6_K = 82 MB
    big = gw.random_tensor_bytes(rng, Q6_K, 100000 * 1024)
    ts.insert(1, ("big.weight", (1024, 100000), Q6_K, big))
    data = gw.build(META, ts)
    p = _write(tmp_path, "load.gguf", data)
    with GgufFile(p) as f:
        payload = f.info()["payload_offset"]
        f.load()
        assert f.info()["device_bytes"] == sum(len(d) for *_, d in ts)
        for g in f.tensors():
            assert g.device_ptr and g.device_ptr % 256 == 0
            got = f.tensor(g.name).cpu().numpy().tobytes()
            assert got == data[payload + g.offset:payload + g.offset + g.size_bytes], g.name
        f.unload()
        assert all(g.device_ptr is None for g in f.tensors()) and f.info()["device_bytes"] == 0
        f.load(base_layer_count=2)
        for g in f.tensors():
            blk = int(g.name.split(".")[1]) if g.name.startswith("blk.") else -1
            assert (g.device_ptr is None) == (blk >= 2), g.name
        torch.cuda.synchronize()


@pytest.mark.gpu
def test_loaded_tables_through_gather_and_gemv(tmp_path):
    """A GGUF's Q4_K embedding and Q6_K output tables, loaded by the library,
    through the dequant-gather (bit-exact) and the GEMV (fp32 tolerance)."""
    import torch

    import pyoracle as oracle
    from conftest import assert_bits_equal, assert_f32_close
    from qwen35_hip import ops, synth

    rows, cols = 5000, 2048
    q4 = synth.q4k_table(rows, cols, seed_tensor=9)
    q6 = synth.q6k_table(rows, cols, seed_tensor=10)
    data = gw.build([("general.architecture", gw.STR, "qwen35moe")],
                    [("token_embd.weight", (cols, rows), Q4_K, q4.tobytes()),
                     ("output.weight", (cols, rows), Q6_K, q6.tobytes())])
    with GgufFile(_write(tmp_path, "tables.gguf", data)) as f:
        f.load()
        ids = synth.token_ids(300, rows)
        emb = f.tensor("token_embd.weight")
        got = ops.dequant_gather_rows(emb, "Q4_K", rows * cols, torch.from_numpy(ids).cuda(), cols)
        assert_bits_equal(got.cpu().numpy(), oracle.dequant_gather(q4, Q4_K, ids, cols), "gguf Q4_K gather")
        x = np.random.default_rng(3).standard_normal(cols).astype(np.float32)
        y = ops.matmul_dispatch(f.tensor("output.weight"), "Q6_K", rows * cols, torch.from_numpy(x).cuda(), rows, cols)
        assert_f32_close(y.cpu().numpy(), oracle.gemv(q6, Q6_K, x, rows, cols, threads=16), group=rows,
                         what="gguf Q6_K gemv")
