"""CPU checks of the weight-image manifest reader (qwen_weights_scan): the
real model's manifest (tests/golden/manifest_64k.json, the exporter's output)
validates against its image size, and each rule of the exporter / packer
format rejects the entry that breaks it.  No GPU is touched."""
import ctypes
import json
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
MANIFEST = ROOT / "tests" / "golden" / "manifest_64k.json"


@pytest.fixture(scope="module")
def lib():
    """The library; QWEN_KERNELS_LIB_UNDER_TEST names another build of it (the
    sanitizer run, tests/test_sanitizers.py)."""
    import os

    import qwen_kernels_gpu as qk
    return qk.load(os.environ.get("QWEN_KERNELS_LIB_UNDER_TEST") or None)


def scan(lib, path, image_bytes):
    n = [ctypes.c_int(), ctypes.c_int(), ctypes.c_int()]
    wb = ctypes.c_uint64()
    rc = lib.qwen_weights_scan(str(path).encode(), image_bytes, *(ctypes.byref(x) for x in n), ctypes.byref(wb))
    return rc, [x.value for x in n], wb.value


def test_real_manifest_validates(lib):
    m = json.loads(MANIFEST.read_text())
    total = m["total_binary_bytes"]
    rc, counts, wb = scan(lib, MANIFEST, total)
    assert rc == 320 and counts == [150, 169, 1]
    # BFP8 bytes from the shapes alone: M*K mantissas + ceil8(M*K/64) exponents
    want = sum(M * K + (M * K // 64 + 7) // 8 * 8 for M, K in
               (t["shape"] for t in m["tensors"].values() if t["type"] == "block64_bfp8"))
    assert wb == want
    # the last tensor ends at the image's end; one byte less rejects it
    assert scan(lib, MANIFEST, total - 1)[0] < 0
    assert b"outside" in lib.bfp8_last_error()


def write(tmp_path, tensors, name="m.json"):
    p = tmp_path / name
    p.write_text(json.dumps({"model_name": "t", "tensors": tensors}))
    return p


def bfp8(M, K, off, **kw):
    e = {"dtype": "bfp8_soa", "shape": [M, K], "type": "block64_bfp8", "mantissa_bytes": M * K,
         "exponent_bytes": (M * K // 64 + 7) // 8 * 8, "file_offset": off}
    e["byte_size"] = e["mantissa_bytes"] + e["exponent_bytes"]
    e.update(kw)
    return e


@pytest.mark.parametrize("bad,why", [
    ({"exponent_bytes": 6}, "exponent plane not padded to 8"),
    ({"shape": [3, 96], "mantissa_bytes": 288}, "K not a multiple of 64"),
    ({"file_offset": 32}, "unaligned offset"),
    ({"type": "block32_bfp4"}, "unknown type"),
    ({"byte_size": 10}, "byte_size != planes"),
    ({"mantissa_bytes": 100}, "mantissa plane size"),
])
def test_rejects_broken_entries(lib, tmp_path, bad, why):
    good = bfp8(3, 128, 64)
    assert scan(lib, write(tmp_path, {"w": good}), 4096)[0] == 1
    broken = dict(good)
    broken.update(bad)
    assert scan(lib, write(tmp_path, {"w": good, "x.weight": broken}, "b.json"), 4096)[0] < 0, why
    assert b"x.weight" in lib.bfp8_last_error()


def test_json_reader_edge_cases(lib, tmp_path):
    """Escapes, nested arrays, numbers with exponents, whitespace; malformed
    documents are rejected."""
    t = {"aé\\\"b": {"type": "raw_fp32", "shape": [2, 3], "file_offset": 0, "byte_size": 24,
                          "extra": [[1, 2.5e3, -1e-2], {"k": None, "t": True}]},
         "emb": {"type": "raw_bf16", "shape": [4, 8], "file_offset": 64, "byte_size": 64}}
    p = tmp_path / "e.json"
    p.write_text(json.dumps({"tensors": t}, indent=3))
    rc, counts, wb = scan(lib, p, 128)
    assert rc == 2 and counts == [0, 1, 1] and wb == 0
    for text in ('{"tensors": {', '{"tensors": [1, 2]}', '{"tensors": {"a": {"type": "raw_fp32"}}}', "nope",
                 '{"tensors": {"a": {"type": "raw_fp32", "shape": [1], "file_offset": 0, "byte_size": 4}}} x'):
        p.write_text(text)
        assert scan(lib, p, 4096)[0] < 0, text
    assert scan(lib, tmp_path / "missing.json", 0)[0] < 0
