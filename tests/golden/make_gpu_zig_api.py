"""Writes gpu_zig_api.json: the public op wrappers of the reference's
src/gpu.zig (lines 483-830) -- each name, its line and its parameter names in
order -- read from the source as text. This is the interface the C ABI and
both host mirrors keep; tests/test_host_mirror.py checks them against it.

Usage: python tests/golden/make_gpu_zig_api.py [path/to/gpu.zig]
"""

from __future__ import annotations

import json
import re
import sys
from pathlib import Path

OUT = Path(__file__).resolve().parent / "gpu_zig_api.json"


def extract(text: str) -> dict:
    lines = text.split("\n")
    api = {}
    i = 0
    while i < len(lines):
        m = re.match(r"pub fn (\w+)\(", lines[i])
        if m and 483 <= i + 1 <= 830:
            j, sig = i, ""
            while True:
                sig += lines[j].strip() + " "
                if re.search(r"\)\s*void\s*\{", lines[j]):
                    break
                j += 1
            inner = sig[sig.index("(") + 1: sig.rindex(")")]
            params = [p.strip().split(":")[0].strip() for p in inner.split(",") if p.strip()]
            api[m.group(1)] = {"line": i + 1, "params": params}
            i = j
        i += 1
    return api


def main() -> None:
    src = Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference/src/gpu.zig")
    ops = extract(src.read_text())
    OUT.write_text(json.dumps({"source": "src/gpu.zig:483-830", "ops": ops}, indent=1) + "\n")
    print(OUT, len(ops))


if __name__ == "__main__":
    main()
