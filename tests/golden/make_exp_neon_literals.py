"""Writes exp_neon_literals.json: the numeric literals of the reference's
exp_neon (04-板载脚本与工具/qwen_kernels_opt.c:332-352), in source order, as
the text they are written in.  Run from the repository root in a checkout
that has the reference at /root/reference:

    python tests/golden/make_exp_neon_literals.py
"""
from __future__ import annotations

import json
import re
from pathlib import Path

REF = Path("/root/reference/04-板载脚本与工具/qwen_kernels_opt.c")
LINES = (332, 352)
OUT = Path(__file__).resolve().parent / "exp_neon_literals.json"
# float literals (with an f suffix) and the two integer operands (127, 23)
FLOAT = re.compile(r"(?<![\w.])-?\d+\.\d*(?:[eE][-+]?\d+)?f")
INT = re.compile(r"vdupq_n_s32\((\d+)\)|vshlq_n_s32\(\w+, (\d+)\)")


def parse(text: str) -> dict:
    lines = text.splitlines()[LINES[0] - 1:LINES[1]]
    body = "\n".join(lines)
    assert "exp_neon" in lines[0], lines[0]
    floats = FLOAT.findall(body)
    ints = [a or b for a, b in INT.findall(body)]
    return {"source": f"04-板载脚本与工具/qwen_kernels_opt.c:{LINES[0]}-{LINES[1]}", "floats": floats,
            "ints": ints}


def main() -> None:
    d = parse(REF.read_text(encoding="utf-8"))
    OUT.write_text(json.dumps(d, ensure_ascii=False, indent=1) + "\n", encoding="utf-8")
    print(f"wrote {OUT}: {len(d['floats'])} float literals, ints {d['ints']}")


if __name__ == "__main__":
    main()
