"""GGUF pack ingestion, host side (no GPU): the oracle pinned against the
reference's own converter and pack-reader test, and the library's parser,
drop-in reader and loader plans against the oracle.

* tests/golden/pack_*.gguf were written by the reference's converter
  (scripts/convert_pixal3d_to_gguf.py, driven by tests/golden/
  make_gguf_golden.py): the oracle writer reproduces them byte for byte, the
  oracle reader recovers every key and tensor, and the payloads decode to the
  converter's float32 sources under its precision policy (F16 by numpy's
  IEEE half conversion, BF16 equal to torch's rounding, flex_gemm conv
  weights in the [27, out, in] compact-v1 layout).
* The reference's tests/test_pack_reader.cpp case (offset 0, byte round
  trip, missing tensor and closed reader rejected) through the oracle, the C
  ABI and the C++ drop-in.
* Malformed packs: the library's verdict and message equal the oracle's,
  which are the reference's (src/pack.cpp:127-288).
* pxs_slat_flow_pack_plan / pxs_slat_decoder_pack_plan (host functions):
  hyperparameters and messages of SLatFlowModel::load /
  SLatDecoderModel::load."""

import ctypes as C
import json
import struct
from pathlib import Path

import numpy as np
import pytest
import torch

import oracle as O
import pack_oracle as G
import pxs

GOLD = Path(__file__).resolve().parent / "golden"
META = json.loads((GOLD / "pack_golden.json").read_text())
SOURCES = dict(np.load(GOLD / "pack_golden.npz"))


@pytest.fixture(scope="module")
def px():
    return pxs.Pxs()


def golden(stem):
    return GOLD / META[stem]["file"]


def expected_values(stem, entry):
    """The converter's source of one table entry, through the storage
    transform and rounding its ggml type implies."""
    src = SOURCES[f"{META[stem]['sources']}/{entry['source']}"]
    if src.ndim == 5:  # flex_gemm [out, 3, 3, 3, in] -> [27, out, in]
        src = np.ascontiguousarray(src.transpose(1, 2, 3, 0, 4)).reshape(27, src.shape[0],
                                                                         src.shape[4])
    if entry["ggml_type"] == G.GGML_F16:
        return src.astype(np.float16).astype(np.float32)
    if entry["ggml_type"] == G.GGML_BF16:
        return torch.from_numpy(src).to(torch.bfloat16).float().numpy()
    return src


# --- the oracle against the reference's converter -----------------------------------

@pytest.mark.parametrize("stem", list(META))
def test_oracle_writer_reproduces_converter_bytes(stem):
    path = golden(stem)
    info = G.load_pack_info(path)
    kvs = [(k, vt, v) for k, (vt, v) in info.kv.items()]
    tensors = [G.Tensor(t.name, t.ggml_type, tuple(e["dims"]), G.read_tensor(info, t.name))
               for t, e in zip(info.tensors, META[stem]["tensors"])]
    assert G.pack_bytes(kvs, tensors, alignment=info.alignment) == path.read_bytes()


@pytest.mark.parametrize("stem", list(META))
def test_oracle_reader_recovers_converter_table_and_values(stem):
    info = G.load_pack_info(golden(stem))
    meta = META[stem]
    assert (info.gguf_version, info.alignment, info.architecture, info.name) == \
        (3, 32, "pixal3d", meta["stem"])
    assert info.components == [(meta["component"], meta["component"], meta["model_class"],
                                meta["variant"])]
    assert info.file_type == {0: 0, 1: 1, 2: 24}[meta["ftype"]]
    assert [t.name for t in info.tensors] == [e["name"] for e in meta["tensors"]]
    for t, e in zip(info.tensors, meta["tensors"]):
        dims = e["dims"] + [1] * (4 - len(e["dims"]))
        assert t.ne == tuple(dims) and t.ggml_type == e["ggml_type"] and t.n_bytes == e["nbytes"]
        got = G.decode_f32(G.read_tensor(info, t.name), t.ggml_type)
        np.testing.assert_array_equal(got, expected_values(stem, e).reshape(-1), err_msg=t.name)


def test_converter_precision_policy_is_visible_in_the_packs():
    """ftype 1: F16 matrices, F32 vectors and every norm / gamma / modulation
    (choose_flow_type, scripts/convert_pixal3d_to_gguf.py:347-353); ftype 2:
    all BF16; decoder ftype 1: F16 for every tensor of two or more dims."""
    for e in META["pack_flow_f16"]["tensors"]:
        sensitive = any(s in e["source"] for s in ("gamma", "modulation", "norm"))
        want = G.GGML_F16 if len(e["dims"]) >= 2 and not sensitive else G.GGML_F32
        assert e["ggml_type"] == want, e["name"]
    assert {e["ggml_type"] for e in META["pack_flow_bf16"]["tensors"]} == {G.GGML_BF16}
    for e in META["pack_decoder_f16"]["tensors"]:
        assert e["ggml_type"] == (G.GGML_F16 if len(e["dims"]) >= 2 else G.GGML_F32)
    assert all(e["name"].startswith("sh1024.") for e in META["pack_flow_f16"]["tensors"])


def test_bf16_rounding_matches_torch():
    rng = np.random.default_rng(5)
    x = np.concatenate([rng.standard_normal(4096).astype(np.float32) * 3,
                        np.array([0.0, -0.0, 1.0, 1.00390625, 1.01171875, 3.4e38, -3.4e38,
                                  1e-40, -1e-40, 65504.0], np.float32)])
    # exact ties in both directions
    ties = (np.arange(64, dtype=np.uint32) << 16 | 0x8000).view(np.float32) + np.float32(0)
    x = np.concatenate([x, ties.astype(np.float32)])
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(G.bf16_bits(x), want)


# --- the library parser against the oracle -----------------------------------------

@pytest.mark.parametrize("stem", list(META))
def test_library_reader_matches_oracle(px, stem):
    path = golden(stem)
    info = G.load_pack_info(path)
    with px.pack_open(path) as pack:
        d = pack.describe()
        assert (d["gguf_version"], d["alignment"], d["data_offset"], d["architecture"],
                d["name"], d["tensor_name_scheme"], d["file_type"], d["bundle_format"]) == \
            (info.gguf_version, info.alignment, info.data_offset, info.architecture, info.name,
             info.tensor_name_scheme, info.file_type, info.bundle_format)
        assert [(c["key"], c["stage"], c["model_class"], c["variant"]) for c in d["components"]] \
            == info.components
        assert len(d["tensors"]) == len(info.tensors)
        for t, o in zip(d["tensors"], info.tensors):
            assert (t["name"], t["n_dims"], tuple(t["ne"]), t["ggml_type"], t["type_name"],
                    t["n_bytes"], t["offset"]) == \
                (o.name, o.n_dims, o.ne, o.ggml_type, o.type_name, o.n_bytes, o.offset)
            assert pack.read_tensor(t["name"]) == G.read_tensor(info, t["name"])
        prefix = "pixal3d." + META[stem]["component"] + "."
        for key, (vt, value) in info.kv.items():
            kind = {G.VT_STRING: "string", G.VT_F32: "f32", G.VT_BOOL: "bool",
                    G.VT_U32: "u32"}.get(vt)
            if kind is None:
                continue
            got = pack.metadata(key, kind)
            assert got == (np.float32(value) if kind == "f32" else value), key
        assert pack.metadata(prefix + "absent", "f32", required=False) == 0.0
        assert pack.metadata(prefix + "absent", "bool", required=False) is False
        assert pack.metadata(prefix + "absent", "string", required=False) == ""


def test_upload_rejects_misaligned_workspace(px):
    """Workspaces must be 256-byte aligned (the staging chunks are read with
    16-byte loads): a misaligned one is an argument error, raised before any
    device work (so the call runs here without a device; the pointers are
    never dereferenced)."""
    path = golden("pack_flow_f16")
    info = G.load_pack_info(path)
    t = next(t for t in info.tensors if t.ggml_type == G.GGML_F32)
    count = t.n_bytes // 4
    with px.pack_open(path) as pack:
        rc = px.lib.pxs_pack_upload(pack.handle, t.name.encode(), pxs.PXS_F32, 1 << 20, count,
                                    (1 << 20) + 8, None)
        assert rc == pxs.PXS_ERR_ARG
        assert px.lib.pxs_last_error().decode() == \
            "pxs_pack_upload: workspace must be 256-byte aligned"
        # a null argument is reported before the alignment
        rc = px.lib.pxs_pack_upload(None, t.name.encode(), pxs.PXS_F32, 1 << 20, count,
                                    (1 << 20) + 8, None)
        assert rc == pxs.PXS_ERR_ARG
        assert px.lib.pxs_last_error().decode() == "pxs_pack_upload: null argument"


def reference_case_pack(path):
    """The pack tests/test_pack_reader.cpp:29-49 writes: one F32 [2, 3]
    tensor ss.input_layer.bias in an otherwise empty compact-v1 pack."""
    values = np.array([1.25, -2.5, 3.75, 4.5, -5.25, 6.0], np.float32).reshape(2, 3)
    kvs = [("general.architecture", G.VT_STRING, "pixal3d"),
           ("general.name", G.VT_STRING, "pack-reader-test"),
           ("general.file_type", G.VT_U32, 0), ("general.alignment", G.VT_U32, 32),
           ("pixal3d.bundle_format", G.VT_U32, 1),
           ("pixal3d.tensor_name_scheme", G.VT_STRING, "compact-v1")]
    G.write_pack(path, kvs, [G.f32_tensor("ss.input_layer.bias", values)])
    return values


def test_reference_pack_reader_case(px, tmp_path):
    path = tmp_path / "pixal3d-pack-reader-test.gguf"
    values = reference_case_pack(path)
    info = G.load_pack_info(path)
    assert len(info.tensors) == 1 and info.tensors[0].offset == 0
    assert G.read_tensor(info, "ss.input_layer.bias") == values.tobytes()
    with pytest.raises(G.PackError, match="tensor not found: missing"):
        G.read_tensor(info, "missing")
    with px.pack_open(path) as pack:
        d = pack.describe()
        assert len(d["tensors"]) == 1 and d["tensors"][0]["offset"] == 0
        assert d["tensors"][0]["ne"] == [3, 2, 1, 1] and d["tensors"][0]["n_dims"] == 2
        assert pack.read_tensor("ss.input_layer.bias") == values.tobytes()
        n = C.c_size_t()
        rc = pack.lib.pxs_pack_read_tensor(pack.handle, b"missing", None, 0, C.byref(n))
        assert rc != 0 and pack.lib.pxs_last_error().decode() == "tensor not found: missing"


def test_reference_pack_reader_case_dropin(tmp_path):
    """The C++ drop-in Pixal3DPackReader (host code of libpxs.so, no GPU)."""
    path = tmp_path / "pixal3d-pack-reader-test.gguf"
    values = reference_case_pack(path)
    d = O.DropIn()
    r, raw = d.pack_reader_case(path, "ss.input_layer.bias", "general.alignment")
    assert r["load_pack_info"] == (1, "") and r["open"] == (1, "") and r["is_open"] == 1
    assert r["tensors"] == 1 and r["offset"] == 0 and r["has_tensor"] == 1
    assert r["tensor_bytes"] == 24 and r["read"] == (1, "") and raw == values.tobytes()
    assert r["missing"] == (0, "tensor not found: missing")
    assert r["meta"] == (1, "32")
    assert r["closed_is_open"] == 0
    assert r["closed_read"] == (0, "pack reader is not open")
    assert r["closed_meta"] == (0, "pack reader is not open")
    bad = tmp_path / "bad.gguf"
    bad.write_bytes(b"GGUF" + struct.pack("<I", 2) + bytes(16))
    r, _ = d.pack_reader_case(bad, "x", "general.alignment")
    assert r["open"] == (0, "unsupported GGUF version: 2")
    assert r["load_pack_info"] == (0, "unsupported GGUF version: 2")


# --- malformed packs ---------------------------------------------------------------

def base_kvs(**changes):
    kvs = G.pixal3d_kvs(name="t", components=("shape_flow_1024",))
    out = []
    for k, vt, v in kvs:
        if k in changes:
            if changes[k] is None:
                continue
            vt, v = changes[k]
        out.append((k, vt, v))
    return out


def small_tensors(n=2):
    return [G.f32_tensor(f"sh1024.t{i}", np.arange(5 + i, dtype=np.float32)) for i in range(n)]


def write_raw(tmp_path, data, name="case.gguf"):
    p = tmp_path / name
    p.write_bytes(data)
    return p


PARSE = "gguf_init_from_file failed: "


def malformed(tmp_path, case):
    """-> (path, expected message or None for a valid pack)."""
    t = small_tensors()
    if case == "version2":
        return write_raw(tmp_path, G.pack_bytes(base_kvs(), t, version=2)), \
            "unsupported GGUF version: 2"
    if case == "version4":
        p = write_raw(tmp_path, G.pack_bytes(base_kvs(), t, version=4))
        return p, PARSE + str(p)
    if case == "version1":
        p = write_raw(tmp_path, G.pack_bytes(base_kvs(), t, version=1))
        return p, PARSE + str(p)
    if case == "magic":
        p = write_raw(tmp_path, G.pack_bytes(base_kvs(), t, magic=b"GGUG"))
        return p, PARSE + str(p)
    if case == "architecture":
        return write_raw(tmp_path, G.pack_bytes(base_kvs(**{
            "general.architecture": (G.VT_STRING, "llama")}), t)), \
            "unexpected GGUF architecture: llama"
    if case == "architecture_type":
        return write_raw(tmp_path, G.pack_bytes(base_kvs(**{
            "general.architecture": (G.VT_U32, 3)}), t)), \
            "GGUF metadata is not a string: general.architecture"
    if case == "no_name":
        return write_raw(tmp_path, G.pack_bytes(base_kvs(**{"general.name": None}), t)), \
            "missing GGUF metadata: general.name"
    if case == "scheme":
        return write_raw(tmp_path, G.pack_bytes(base_kvs(**{
            "pixal3d.tensor_name_scheme": (G.VT_STRING, "compact-v0")}), t)), \
            "unsupported Pixal3D tensor name scheme: compact-v0"
    if case == "no_scheme":
        return write_raw(tmp_path, G.pack_bytes(base_kvs(**{
            "pixal3d.tensor_name_scheme": None}), t)), \
            "missing GGUF metadata: pixal3d.tensor_name_scheme"
    if case == "file_type_negative":
        return write_raw(tmp_path, G.pack_bytes(base_kvs(**{
            "general.file_type": (G.VT_I32, -1)}), t)), \
            "GGUF metadata is not a non-negative integer: general.file_type"
    if case == "file_type_f32":
        return write_raw(tmp_path, G.pack_bytes(base_kvs(**{
            "general.file_type": (G.VT_F32, 1.0)}), t)), \
            "GGUF metadata is not a non-negative integer: general.file_type"
    if case == "file_type_i8":
        return write_raw(tmp_path, G.pack_bytes(base_kvs(**{
            "general.file_type": (G.VT_I8, 5)}), t)), None
    if case == "file_type_u64":
        return write_raw(tmp_path, G.pack_bytes(base_kvs(**{
            "general.file_type": (G.VT_U64, 1)}), t)), \
            "GGUF metadata is not a non-negative integer: general.file_type"
    if case == "no_bundle_format":
        return write_raw(tmp_path, G.pack_bytes(base_kvs(**{"pixal3d.bundle_format": None}), t)), \
            "missing GGUF metadata: pixal3d.bundle_format"
    if case == "component_type":
        return write_raw(tmp_path, G.pack_bytes(base_kvs(**{
            "pixal3d.component.0": (G.VT_U32, 7)}), t)), \
            "component metadata is not a string: pixal3d.component.0"
    if case == "duplicate_key":
        kvs = base_kvs() + [("general.name", G.VT_STRING, "again")]
        p = write_raw(tmp_path, G.pack_bytes(kvs, t))
        return p, PARSE + str(p)
    if case == "alignment_not_pow2":
        p = write_raw(tmp_path, G.pack_bytes(base_kvs(**{
            "general.alignment": (G.VT_U32, 48)}), t, alignment=48))
        return p, PARSE + str(p)
    if case == "alignment_64":
        return write_raw(tmp_path, G.pack_bytes(base_kvs(**{
            "general.alignment": (G.VT_U32, 64)}), t, alignment=64)), None
    if case == "alignment_u16":
        p = write_raw(tmp_path, G.pack_bytes(base_kvs(**{
            "general.alignment": (G.VT_U16, 32)}), t))
        return p, PARSE + str(p)
    if case == "bool_2":
        kvs = base_kvs() + [("pixal3d.flag", G.VT_U8, 0)]
        data = bytearray(G.pack_bytes(kvs, t))
        key = G.gguf_string("pixal3d.flag") + struct.pack("<I", G.VT_U8)
        at = data.index(key) + len(key)
        data[at - 4:at] = struct.pack("<I", G.VT_BOOL)
        data[at] = 2
        p = write_raw(tmp_path, bytes(data))
        return p, PARSE + str(p)
    if case == "array_kv":
        kvs = base_kvs() + [("pixal3d.list", G.VT_ARRAY, (G.VT_STRING, ["a", "bc"])),
                            ("pixal3d.nums", G.VT_ARRAY, (G.VT_I64, [1, -2, 3]))]
        return write_raw(tmp_path, G.pack_bytes(kvs, t)), None
    if case == "nested_array":
        kvs = base_kvs() + [("pixal3d.list", G.VT_ARRAY, (G.VT_U8, [1]))]
        data = bytearray(G.pack_bytes(kvs, t))
        key = G.gguf_string("pixal3d.list") + struct.pack("<I", G.VT_ARRAY)
        at = data.index(key) + len(key)
        data[at:at + 4] = struct.pack("<I", G.VT_ARRAY)
        p = write_raw(tmp_path, bytes(data))
        return p, PARSE + str(p)
    if case == "name_64":
        p = write_raw(tmp_path, G.pack_bytes(base_kvs(), [G.f32_tensor("n" * 64, np.ones(3))]))
        return p, PARSE + str(p)
    if case == "name_63":
        return write_raw(tmp_path, G.pack_bytes(base_kvs(), [G.f32_tensor("n" * 63,
                                                                           np.ones(3))])), None
    if case == "name_empty":
        return write_raw(tmp_path, G.pack_bytes(base_kvs(), [G.f32_tensor("", np.ones(3))])), \
            "GGUF tensor names must be non-empty, unique, and <64 bytes"
    if case == "name_duplicate":
        p = write_raw(tmp_path, G.pack_bytes(base_kvs(), [G.f32_tensor("a", np.ones(3)),
                                                          G.f32_tensor("a", np.ones(2))]))
        return p, PARSE + str(p)
    if case == "offset_gap":
        t[1].offset = 64
        p = write_raw(tmp_path, G.pack_bytes(base_kvs(), t))
        return p, PARSE + str(p)
    if case == "dims_5":
        bad = G.Tensor("a", G.GGML_F32, (1, 1, 1, 1, 1), np.ones(1, np.float32).tobytes())
        p = write_raw(tmp_path, G.pack_bytes(base_kvs(), [bad]))
        return p, PARSE + str(p)
    if case == "type_unknown":
        bad = G.Tensor("a", 99, (4,), bytes(16))
        p = write_raw(tmp_path, G.pack_bytes(base_kvs(), [bad]))
        return p, PARSE + str(p)
    if case == "q4_0_partial_block":
        bad = G.Tensor("a", 2, (33,), bytes(18))
        p = write_raw(tmp_path, G.pack_bytes(base_kvs(), [bad]))
        return p, PARSE + str(p)
    if case == "q4_0":
        return write_raw(tmp_path, G.pack_bytes(base_kvs(), [G.Tensor("a", 2, (64, 3),
                                                                      bytes(108))])), None
    if case == "trailing_unit_dims":
        return write_raw(tmp_path, G.pack_bytes(base_kvs(), [G.Tensor(
            "a", G.GGML_F32, (4, 1, 1), np.ones(4, np.float32).tobytes())])), None
    if case == "zero_dim":
        return write_raw(tmp_path, G.pack_bytes(base_kvs(), [G.Tensor(
            "a", G.GGML_F32, (4, 0), b"")])), None
    if case == "truncated_payload":
        data = G.pack_bytes(base_kvs(), t)
        p = write_raw(tmp_path, data[:-40])
        return p, "GGUF tensor payload is outside the file: sh1024.t1"
    if case == "truncated_header":
        data = G.pack_bytes(base_kvs(), t)
        p = write_raw(tmp_path, data[:200])
        return p, PARSE + str(p)
    if case == "data_offset_beyond_end":
        data = G.pack_bytes(base_kvs(**{"general.name": (G.VT_STRING, "tt")}), [])
        header_end = len(data.rstrip(b"\0"))
        assert header_end % 32 != 0
        return write_raw(tmp_path, data[:header_end]), \
            "GGUF tensor data offset is beyond end of file"
    if case == "components_mixed":
        kvs = base_kvs(**{"pixal3d.component.0": (G.VT_STRING, "stage|Cls|var|x")})
        kvs += [("pixal3d.component.1", G.VT_STRING, "texture_decoder"),
                ("pixal3d.texture_decoder.model_class", G.VT_STRING, "SparseUnetVaeDecoder"),
                ("pixal3d.component.3", G.VT_STRING, "not reached")]
        return write_raw(tmp_path, G.pack_bytes(kvs, t)), None
    if case == "component_class_type":
        kvs = base_kvs() + [("pixal3d.shape_flow_1024.variant", G.VT_U32, 1)]
        return write_raw(tmp_path, G.pack_bytes(kvs, t)), \
            "GGUF metadata is not a string: pixal3d.shape_flow_1024.variant"
    raise KeyError(case)


CASES = ["version2", "version4", "version1", "magic", "architecture", "architecture_type",
         "no_name", "scheme", "no_scheme", "file_type_negative", "file_type_f32", "file_type_i8",
         "file_type_u64", "no_bundle_format", "component_type", "duplicate_key",
         "alignment_not_pow2", "alignment_64", "alignment_u16", "bool_2", "array_kv",
         "nested_array", "name_64", "name_63", "name_empty", "name_duplicate", "offset_gap",
         "dims_5", "type_unknown", "q4_0_partial_block", "q4_0", "trailing_unit_dims",
         "zero_dim", "truncated_payload", "truncated_header", "data_offset_beyond_end",
         "components_mixed", "component_class_type"]


def library_open(px, path):
    h = C.c_void_p()
    rc = px.lib.pxs_pack_open(str(path).encode(), C.byref(h))
    if rc != 0:
        return None, px.lib.pxs_last_error().decode("utf-8", errors="surrogateescape")
    return h, None


@pytest.mark.parametrize("case", CASES)
def test_malformed_pack(px, tmp_path, case):
    path, want = malformed(tmp_path, case)
    try:
        info, omsg = G.load_pack_info(path), None
    except G.PackError as e:
        info, omsg = None, str(e)
    assert omsg == want, f"oracle: {omsg!r} != {want!r}"
    h, lmsg = library_open(px, path)
    assert lmsg == want, f"library: {lmsg!r} != {want!r}"
    if h is not None:
        n = px.lib.pxs_pack_describe(h, None, 0)
        buf = C.create_string_buffer(n)
        px.lib.pxs_pack_describe(h, buf, n)
        d = json.loads(buf.value.decode())
        px.lib.pxs_pack_close(h)
        assert [(c["key"], c["stage"], c["model_class"], c["variant"])
                for c in d["components"]] == info.components
        assert [(t["name"], t["n_dims"], tuple(t["ne"]), t["type_name"], t["n_bytes"],
                 t["offset"]) for t in d["tensors"]] == \
            [(t.name, t.n_dims, t.ne, t.type_name, t.n_bytes, t.offset) for t in info.tensors]
        assert d["alignment"] == info.alignment and d["data_offset"] == info.data_offset


def test_malformed_pack_details(tmp_path):
    """What the valid odd cases must read as."""
    info = G.load_pack_info(malformed(tmp_path, "components_mixed")[0])
    assert info.components == [("stage|Cls|var|x", "stage", "Cls", "var|x"),
                               ("texture_decoder", "texture_decoder", "SparseUnetVaeDecoder", "")]
    info = G.load_pack_info(malformed(tmp_path, "q4_0")[0])
    assert (info.tensors[0].type_name, info.tensors[0].n_bytes, info.tensors[0].n_dims) == \
        ("q4_0", 108, 2)
    info = G.load_pack_info(malformed(tmp_path, "trailing_unit_dims")[0])
    assert info.tensors[0].n_dims == 1 and info.tensors[0].ne == (4, 1, 1, 1)
    info = G.load_pack_info(malformed(tmp_path, "alignment_64")[0])
    assert info.alignment == 64 and info.tensors[1].offset == 64 and info.data_offset % 64 == 0


def test_metadata_type_rules(px, tmp_path):
    kvs = base_kvs() + [("k.u8", G.VT_U8, 200), ("k.u16", G.VT_U16, 60000),
                        ("k.i16", G.VT_I16, 7), ("k.i16neg", G.VT_I16, -7),
                        ("k.f32", G.VT_F32, 0.25), ("k.f64", G.VT_F64, 0.25),
                        ("k.bool", G.VT_BOOL, True), ("k.str", G.VT_STRING, "x y")]
    path = write_raw(tmp_path, G.pack_bytes(kvs, small_tensors()))
    info = G.load_pack_info(path)
    err = lambda m: ("error", m)  # noqa: E731
    cases = [("k.u8", "u32", 200), ("k.u16", "u32", 60000), ("k.i16", "u32", 7),
             ("k.i16neg", "u32", err("GGUF metadata is not a non-negative integer: k.i16neg")),
             ("k.f32", "f32", 0.25), ("k.f64", "f32", err("GGUF metadata is not float32: k.f64")),
             ("k.u8", "f32", err("GGUF metadata is not float32: k.u8")), ("k.bool", "bool", True),
             ("k.u8", "bool", err("GGUF metadata is not bool: k.u8")), ("k.str", "string", "x y"),
             ("k.bool", "string", err("GGUF metadata is not a string: k.bool")),
             ("k.none", "u32", err("missing GGUF metadata: k.none"))]
    with px.pack_open(path) as pack:
        for key, kind, want in cases:
            for read in (lambda: G.metadata(info, key, kind), lambda: pack.metadata(key, kind)):
                if isinstance(want, tuple):
                    with pytest.raises((G.PackError, pxs.PxsError), match=want[1]):
                        read()
                else:
                    assert read() == want, (key, kind)
        for kind, default in (("u32", 0), ("f32", 0.0), ("bool", False), ("string", "")):
            assert G.metadata(info, "k.none", kind, False) == default
            assert pack.metadata("k.none", kind, required=False) == default


# --- loader plans (host) -----------------------------------------------------------

def rewrite(src, dst, kv=None, drop=(), extra_kv=()):
    """A golden pack with metadata changed (key -> (vtype, value) or None to
    drop) and tensors dropped."""
    info = G.load_pack_info(src)
    kvs = []
    for k, (vt, v) in info.kv.items():
        if kv and k in kv:
            if kv[k] is None:
                continue
            vt, v = kv[k]
        kvs.append((k, vt, v))
    kvs += list(extra_kv)
    tensors = [G.Tensor(t.name, t.ggml_type, t.ne[:max(t.n_dims, 1)], G.read_tensor(info, t.name))
               for t in info.tensors if t.name not in drop]
    G.write_pack(dst, kvs, tensors)
    return dst


def flow_plan(px, path, component="shape_flow_1024", dtype=pxs.PXS_F32):
    cfg, need = pxs.FlowConfig(), C.c_size_t()
    with px.pack_open(path) as pack:
        rc = px.lib.pxs_slat_flow_pack_plan(pack.handle, component.encode(), dtype,
                                            C.byref(cfg), C.byref(need))
        if rc != 0:
            raise pxs.PxsError(px.lib.pxs_last_error().decode())
    return cfg, need.value


def test_flow_plan_reads_hyperparameters(px):
    args = META["pack_flow_f16"]["args"]
    cfg, f32_bytes = flow_plan(px, golden("pack_flow_f16"))
    assert (cfg.in_channels, cfg.out_channels, cfg.model_channels, cfg.cond_channels,
            cfg.num_blocks, cfg.num_heads, cfg.proj_in_channels, cfg.mlp_hidden) == \
        (args["in_channels"], args["out_channels"], args["model_channels"],
         args["cond_channels"], args["num_blocks"], args["num_heads"], args["cond_channels"],
         int(args["model_channels"] * args["mlp_ratio"]))
    assert (cfg.norm_eps, cfg.rope_freq_min, cfg.rope_freq_base) == \
        (np.float32(1e-6), 1.0, 10000.0)
    assert (cfg.qk_rms_norm, cfg.qk_rms_norm_cross, cfg.use_projection) == (1, 1, 0)
    info = G.load_pack_info(golden("pack_flow_f16"))
    elements = [t.ne[0] * t.ne[1] * t.ne[2] * t.ne[3] for t in info.tensors]
    assert f32_bytes == sum((4 * e + 255) // 256 * 256 for e in elements)
    _, bf16_bytes = flow_plan(px, golden("pack_flow_bf16"), dtype=pxs.PXS_BF16)
    assert bf16_bytes < f32_bytes


FLOW_ERRORS = [
    ("component", {}, (), "texture_flow_2048", "unsupported SLat flow component: texture_flow_2048"),
    ("not_in_pack", {}, (), "shape_flow_512",
     "GGUF pack does not contain SLat flow component: shape_flow_512"),
    ("no_input", {}, ("sh1024.input_layer.weight",), None,
     "GGUF pack does not contain SLat flow component: shape_flow_1024"),
    ("no_class", {"pixal3d.shape_flow_1024.model_class": None}, (), None,
     "missing GGUF metadata: pixal3d.shape_flow_1024.model_class"),
    ("no_heads", {"pixal3d.shape_flow_1024.num_heads": None}, (), None,
     "missing GGUF metadata: pixal3d.shape_flow_1024.num_heads"),
    ("ratio_type", {"pixal3d.shape_flow_1024.mlp_ratio": (G.VT_U32, 4)}, (), None,
     "GGUF metadata is not float32: pixal3d.shape_flow_1024.mlp_ratio"),
    ("odd_head_dim", {"pixal3d.shape_flow_1024.num_heads": (G.VT_U32, 16)}, (), None,
     "invalid SLat flow hyperparameters"),
    ("no_rope_min", {"pixal3d.shape_flow_1024.rope_freq_min": None}, (), None,
     "invalid SLat flow hyperparameters"),
    ("share_mod", {"pixal3d.shape_flow_1024.share_mod": (G.VT_BOOL, False)}, (), None,
     "SLat flow currently requires pe_mode=rope and share_mod=true"),
    ("pe_mode", {"pixal3d.shape_flow_1024.pe_mode": (G.VT_STRING, "ape")}, (), None,
     "SLat flow currently requires pe_mode=rope and share_mod=true"),
    ("attn_mode", {"pixal3d.shape_flow_1024.image_attn_mode": (G.VT_STRING, "self")}, (), None,
     "SLat flow supports image_attn_mode cross or proj"),
]


@pytest.mark.parametrize("case", FLOW_ERRORS, ids=[c[0] for c in FLOW_ERRORS])
def test_flow_plan_errors(px, tmp_path, case):
    _, kv, drop, component, want = case
    path = rewrite(golden("pack_flow_f16"), tmp_path / "f.gguf", kv, drop)
    with pytest.raises(pxs.PxsError) as e:
        flow_plan(px, path, component or "shape_flow_1024")
    assert str(e.value) == want


def test_flow_plan_defaults(px, tmp_path):
    """pe_mode / image_attn_mode default to rope / cross; proj mode takes
    proj_in_channels, or cond_channels when it is absent
    (src/slat_flow.cpp:425-427)."""
    p = rewrite(golden("pack_flow_f16"), tmp_path / "a.gguf",
                {"pixal3d.shape_flow_1024.pe_mode": None,
                 "pixal3d.shape_flow_1024.image_attn_mode": None})
    cfg, _ = flow_plan(px, p)
    assert cfg.use_projection == 0
    p = rewrite(golden("pack_flow_f16"), tmp_path / "b.gguf",
                {"pixal3d.shape_flow_1024.image_attn_mode": (G.VT_STRING, "proj")},
                extra_kv=[("pixal3d.shape_flow_1024.proj_in_channels", G.VT_U32, 24)])
    cfg, _ = flow_plan(px, p)
    assert (cfg.use_projection, cfg.proj_in_channels) == (1, 24)
    p = rewrite(golden("pack_flow_f16"), tmp_path / "c.gguf",
                {"pixal3d.shape_flow_1024.image_attn_mode": (G.VT_STRING, "proj")})
    cfg, _ = flow_plan(px, p)
    assert (cfg.use_projection, cfg.proj_in_channels) == (1, cfg.cond_channels)


def decoder_plan(px, path, component="texture_decoder", dtype=pxs.PXS_F32):
    hp, need = pxs.DecoderHParams(), C.c_size_t()
    with px.pack_open(path) as pack:
        rc = px.lib.pxs_slat_decoder_pack_plan(pack.handle, component.encode(), dtype,
                                               C.byref(hp), C.byref(need))
        if rc != 0:
            raise pxs.PxsError(px.lib.pxs_last_error().decode())
    return hp, need.value


def test_decoder_plan_reads_metadata(px, tmp_path):
    args = META["pack_decoder_f16"]["args"]
    hp, f32_bytes = decoder_plan(px, golden("pack_decoder_f16"))
    assert (hp.resolution, hp.latent_channels, hp.out_channels, hp.levels, hp.pred_subdiv,
            hp.n_blocks) == (16, args["latent_channels"], args["out_channels"], 2, 1, 3)
    assert list(hp.model_channels[:2]) == args["model_channels"]
    assert list(hp.num_blocks[:2]) == args["num_blocks"]
    assert hp.norm_eps == np.float32(1e-6)
    _, bf16_bytes = decoder_plan(px, golden("pack_decoder_f16"), dtype=pxs.PXS_BF16)
    assert bf16_bytes < f32_bytes
    for eps, want in ((0.0, 1e-6), (-1.0, 1e-6), (1e-5, 1e-5)):
        p = rewrite(golden("pack_decoder_f16"), tmp_path / "e.gguf",
                    {"pixal3d.texture_decoder.norm_eps": (G.VT_F32, eps)})
        assert decoder_plan(px, p)[0].norm_eps == np.float32(want)


DECODER_ERRORS = [
    ("name_dot", {}, (), "texture.decoder", "invalid SLat decoder component name"),
    ("name_empty", {}, (), "", "invalid SLat decoder component name"),
    ("not_in_pack", {}, (), "shape_decoder",
     "GGUF pack does not contain SLat decoder component: shape_decoder"),
    ("no_levels", {"pixal3d.texture_decoder.n_levels": None}, (), None,
     "missing GGUF metadata: pixal3d.texture_decoder.n_levels"),
    ("levels_17", {"pixal3d.texture_decoder.n_levels": (G.VT_U32, 17)}, (), None,
     "invalid SLat decoder metadata"),
    ("latent_0", {"pixal3d.texture_decoder.latent_channels": (G.VT_U32, 0)}, (), None,
     "invalid SLat decoder metadata"),
    ("channels_0", {"pixal3d.texture_decoder.model_channels.1": (G.VT_U32, 0)}, (), None,
     "invalid SLat decoder level metadata"),
    ("no_blocks_1", {"pixal3d.texture_decoder.num_blocks.1": None}, (), None,
     "missing GGUF metadata: pixal3d.texture_decoder.num_blocks.1"),
    ("pred_type", {"pixal3d.texture_decoder.pred_subdiv": (G.VT_U32, 1)}, (), None,
     "GGUF metadata is not bool: pixal3d.texture_decoder.pred_subdiv"),
]


@pytest.mark.parametrize("case", DECODER_ERRORS, ids=[c[0] for c in DECODER_ERRORS])
def test_decoder_plan_errors(px, tmp_path, case):
    _, kv, drop, component, want = case
    path = rewrite(golden("pack_decoder_f16"), tmp_path / "d.gguf", kv, drop)
    with pytest.raises(pxs.PxsError) as e:
        decoder_plan(px, path, "texture_decoder" if component is None else component)
    assert str(e.value) == want


# --- fuzzing the parser ------------------------------------------------------------

from hypothesis import HealthCheck, given, settings  # noqa: E402
from hypothesis import strategies as st  # noqa: E402

_FUZZ_BASE = {stem: golden(stem).read_bytes() for stem in ("pack_flow_f16", "pack_decoder_f16")}


@st.composite
def mutated_pack(draw):
    """A golden pack with a few random edits: byte overwrites (biased to the
    header and tensor table, where the parser decides), a truncation, or a
    spliced run of bytes."""
    stem = draw(st.sampled_from(sorted(_FUZZ_BASE)))
    data = bytearray(_FUZZ_BASE[stem])
    head = G.load_pack_info(golden(stem)).data_offset
    for _ in range(draw(st.integers(1, 4))):
        kind = draw(st.sampled_from(["byte", "byte", "byte", "truncate", "splice", "u64"]))
        lim = min(head, len(data))
        if kind == "byte":
            at = draw(st.integers(0, lim - 1))
            data[at] = draw(st.integers(0, 255))
        elif kind == "u64":
            if lim < 8:
                continue
            at = draw(st.integers(0, lim - 8))
            data[at:at + 8] = draw(st.sampled_from([
                (2 ** 63 - 1).to_bytes(8, "little"), (2 ** 64 - 1).to_bytes(8, "little"),
                (1 << 40).to_bytes(8, "little"), (0).to_bytes(8, "little")]))
        elif kind == "truncate":
            del data[draw(st.integers(0, len(data) - 1)):]
        else:
            at = draw(st.integers(0, lim))
            data[at:at] = draw(st.binary(min_size=1, max_size=24))
        if not data:
            break
    return bytes(data)


@settings(max_examples=400, derandomize=True, deadline=None,
          suppress_health_check=[HealthCheck.function_scoped_fixture, HealthCheck.too_slow])
@given(data=mutated_pack())
def test_parser_fuzz_matches_oracle(px, tmp_path, data):
    """Random damage to a real pack: the library neither crashes nor reads
    past the file, and its verdict (and message) equals the oracle's."""
    path = tmp_path / "fuzz.gguf"
    path.write_bytes(data)
    try:
        info, want = G.load_pack_info(path), None
    except G.PackError as e:
        info, want = None, str(e)
    h, got = library_open(px, path)
    assert got == want
    if h is not None:
        n = px.lib.pxs_pack_describe(h, None, 0)
        buf = C.create_string_buffer(n)
        px.lib.pxs_pack_describe(h, buf, n)
        d = json.loads(buf.value.decode("utf-8", errors="surrogateescape"))
        px.lib.pxs_pack_close(h)
        assert [t["name"] for t in d["tensors"]] == [t.name for t in info.tensors]
        assert [t["offset"] for t in d["tensors"]] == [t.offset for t in info.tensors]
