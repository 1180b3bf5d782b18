"""Regenerate tests/golden/manifest_64k.json, the weight manifest the
reference's exporter wrote for the real model (06/qwen35_weights_64k_manifest.json:
320 tensors -- 150 block64_bfp8, 169 raw_fp32, 1 raw_bf16 -- with their
shapes, 64-byte aligned file offsets and byte sizes).  It is data (the
exporter's output), copied as compact JSON; the weight image itself is not in
the reference.

    python tests/golden/make_manifest_fixture.py
"""
import json
from pathlib import Path

SRC = Path("/root/reference/06-模型与权重/qwen35_weights_64k_manifest.json")
DST = Path(__file__).resolve().parent / "manifest_64k.json"

if __name__ == "__main__":
    m = json.loads(SRC.read_text())
    DST.write_text(json.dumps(m, separators=(",", ":"), sort_keys=False) + "\n")
    print(f"wrote {DST} ({DST.stat().st_size} bytes, {len(m['tensors'])} tensors)")
