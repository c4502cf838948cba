"""Writes gpu_zig_callers.json: every identifier of the reference's
src/gpu.zig that the rest of the reference uses -- each `gpu.<name>` in a
src/**/*.zig file that imports gpu.zig as `gpu` (gpu.zig itself excluded) --
with the callers' file:line and the declaration gpu.zig gives it (kind, line,
parameter names and types, return type), read from the source as text. This
is the public surface a drop-in replacement of gpu.zig must keep so that the
layers, network, parser, main, benchmark and gputest compile unchanged;
tests/test_zig_binding.py checks darknet_zig_amd/zig/gpu.zig against it.

Usage: python tests/golden/make_gpu_zig_callers.py [path/to/reference/src]
"""

from __future__ import annotations

import json
import re
import sys
from pathlib import Path

OUT = Path(__file__).resolve().parent / "gpu_zig_callers.json"

# `gpu.name` not preceded by a word character or a '.' (a field such as
# l.gpu.output), matched in code with comments and string literals (the
# "../gpu.zig" of an @import) removed
USE = re.compile(r'(?<![\w.])gpu\.([A-Za-z_]\w*)')
STRING = re.compile(r'"(?:[^"\\]|\\.)*"')
IMPORT = re.compile(r'^const gpu = @import\("(?:\.\./)*gpu\.zig"\);', re.M)


def split_params(inner: str) -> list[tuple[str, str]]:
    """'a: T, b: []const U' -> [('a', 'T'), ('b', '[]const U')] (top-level commas)."""
    out, depth, cur = [], 0, ""
    for c in inner:
        if c in "([{":
            depth += 1
        elif c in ")]}":
            depth -= 1
        if c == "," and depth == 0:
            out.append(cur)
            cur = ""
        else:
            cur += c
    if cur.strip():
        out.append(cur)
    params = []
    for p in out:
        name, _, typ = p.strip().partition(":")
        params.append((name.strip(), " ".join(typ.split())))
    return params


def declarations(gpu_zig: str) -> dict:
    """name -> declaration of every `pub` fn / const / var of gpu.zig."""
    lines = gpu_zig.split("\n")
    decls = {}
    i = 0
    while i < len(lines):
        m = re.match(r"pub (fn|const|var) (\w+)", lines[i])
        if not m:
            i += 1
            continue
        kind, name = m.groups()
        d = {"kind": kind, "line": i + 1}
        if kind == "fn":
            j, sig = i, ""
            while True:
                sig += lines[j].strip() + " "
                if re.search(r"\)\s*[^)]*\{\s*$", lines[j]):
                    break
                j += 1
            open_at = sig.index("(")
            depth, k = 0, open_at
            while True:
                depth += {"(": 1, ")": -1}.get(sig[k], 0)
                if depth == 0:
                    break
                k += 1
            d["params"] = split_params(sig[open_at + 1:k])
            d["returns"] = " ".join(sig[k + 1:sig.rindex("{")].split())
            i = j
        else:
            rest = lines[i][m.end():]
            tm = re.match(r"\s*:\s*([^=]+?)\s*=", rest)
            d["type"] = " ".join(tm.group(1).split()) if tm else None
            if re.match(r"\s*=\s*struct\b", rest):
                d["struct"] = True
            else:
                vm = re.search(r"=\s*(.+?);\s*$", rest)
                d["value"] = vm.group(1) if vm else None
        decls[name] = d
        i += 1
    return decls


def struct_members(gpu_zig: str, name: str) -> dict:
    """Fields and pub fns of `pub const <name> = struct { ... }`."""
    start = gpu_zig.index(f"pub const {name} = struct")
    body_at = gpu_zig.index("{", start)
    depth, k = 0, body_at
    while True:
        depth += {"{": 1, "}": -1}.get(gpu_zig[k], 0)
        if depth == 0:
            break
        k += 1
    body = gpu_zig[body_at + 1:k]
    fields = re.findall(r"^    (\w+): ([^=,]+?)\s*(?:=[^,]*)?,", body, flags=re.M)
    fns = {}
    for m in re.finditer(r"^    pub fn (\w+)\(([^)]*)\)\s*([^{]+)\{", body, flags=re.M):
        fns[m.group(1)] = {"params": split_params(m.group(2)), "returns": " ".join(m.group(3).split())}
    return {"fields": [(f, " ".join(t.split())) for f, t in fields], "fns": fns}


def main() -> None:
    src = Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference/src")
    gpu_text = (src / "gpu.zig").read_text()
    decls = declarations(gpu_text)
    uses: dict[str, list[str]] = {}
    for f in sorted(src.rglob("*.zig")):
        rel = f.relative_to(src).as_posix()
        if rel == "gpu.zig":
            continue
        text = f.read_text()
        if not IMPORT.search(text):
            continue
        for ln, line in enumerate(text.split("\n"), 1):
            code = STRING.sub('""', line.split("//", 1)[0])
            for m in USE.finditer(code):
                uses.setdefault(m.group(1), []).append(f"src/{rel}:{ln}")
    ids = {}
    for name in sorted(uses):
        if name not in decls:
            raise SystemExit(f"gpu.{name} is used ({uses[name][0]}) but not declared pub in gpu.zig")
        d = dict(decls[name])
        if d.get("struct"):
            d["members"] = struct_members(gpu_text, name)
        d["callers"] = uses[name]
        ids[name] = d
    OUT.write_text(json.dumps({"source": "src/gpu.zig (declarations); src/**/*.zig (callers)",
                               "identifiers": ids}, indent=1) + "\n")
    print(OUT, len(ids), "identifiers")


if __name__ == "__main__":
    main()
