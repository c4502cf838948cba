"""The Zig side of the drop-in, checked as text (no Zig toolchain here):

* darknet_zig_amd/zig/dkz.zig declares every entry point of
  include/dkz_ops.h, in the header's order, with the header's parameter
  names and types mapped the way Zig's C ABI requires (int -> c_int,
  unsigned -> c_uint, float -> f32, size_t -> usize, pointers -> Zig
  pointers of the same element type, device buffers -> ?*anyopaque);
* darknet_zig_amd/zig/gpu.zig keeps every public op of the reference's
  src/gpu.zig:483-830 (tests/golden/gpu_zig_api.json) under the same name
  with the same parameter names, and each op's body is one call of a
  dkz_* function declared in dkz.zig with that function's number of
  arguments.
"""

from __future__ import annotations

import json
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "dkz_ops.h"
ZIG_DKZ = ROOT / "darknet_zig_amd" / "zig" / "dkz.zig"
ZIG_GPU = ROOT / "darknet_zig_amd" / "zig" / "gpu.zig"
API = json.loads((ROOT / "tests" / "golden" / "gpu_zig_api.json").read_text())["ops"]


def header_decls():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    out = []
    for ret, name, params in re.findall(r"^\s*((?:const\s+)?[\w ]+?\s*\**)\s*(dkz_\w+)\s*\(([^)]*)\)\s*;", text,
                                        flags=re.M):
        ps = []
        params = params.strip()
        if params and params != "void":
            for p in params.split(","):
                m = re.match(r"(.*?)(\w+)$", " ".join(p.split()))
                ps.append((" ".join(m.group(1).split()), m.group(2)))
        out.append((name, " ".join(ret.split()), ps))
    return out


def zig_externs():
    out = []
    for name, params, ret in re.findall(r"^pub extern fn (dkz_\w+)\((.*)\) (.+);$", ZIG_DKZ.read_text(), flags=re.M):
        ps = []
        if params.strip():
            for p in params.split(", "):
                pn, pt = p.split(": ", 1)
                ps.append((pn, pt))
        out.append((name, ps, ret))
    return out


def c_to_zig_ok(ctype: str, ztype: str) -> bool:
    """Whether Zig type `ztype` is the C ABI type of parameter type `ctype`."""
    base = ctype.replace("const ", "").replace(" ", "")
    const = ctype.startswith("const")
    scalars = {"int": "c_int", "unsigned": "c_uint", "unsignedint": "c_uint", "float": "f32", "size_t": "usize"}
    if base in scalars:
        return ztype == scalars[base]
    if base in ("float*", "int*") and ztype == "?*anyopaque":  # a device buffer (gpu.zig's Buf.ptr)
        return True
    host = {"int*": "*c_int", "size_t*": "*usize", "char*": "[*]u8", "void**": "*?*anyopaque"}
    if base in host:
        return ztype == host[base]
    if base == "void*":
        return ztype in (("*const anyopaque", "?*const anyopaque") if const else ("*anyopaque", "?*anyopaque"))
    return False


def ret_ok(ctype: str, ztype: str) -> bool:
    return {"int": ("Status", "c_int"), "void": ("void",), "const char *": ("[*:0]const u8",),
            "void *": ("?*anyopaque",)}.get(ctype, ()) .__contains__(ztype)


def test_every_header_entry_point_is_declared_in_order():
    hdr, zig = header_decls(), zig_externs()
    assert len(hdr) == 58
    assert [h[0] for h in hdr] == [z[0] for z in zig]


@pytest.mark.parametrize("decl", header_decls(), ids=lambda d: d[0])
def test_extern_matches_header(decl):
    name, ret, params = decl
    zig = {z[0]: z for z in zig_externs()}[name]
    _, zparams, zret = zig
    assert ret_ok(ret, zret), (name, ret, zret)
    assert [p[1] for p in params] == [z[0] for z in zparams], (name, "parameter names")
    for (ctype, pname), (_, ztype) in zip(params, zparams):
        assert c_to_zig_ok(ctype, ztype), (name, pname, ctype, ztype)


def zig_pub_fns():
    """name -> (parameter names, body) of gpu.zig's pub fns."""
    text = ZIG_GPU.read_text()
    out = {}
    for m in re.finditer(r"^pub fn (\w+)\((.*?)\)\s*(?:!?\w+)\s*\{", text, flags=re.M | re.S):
        params = [p.strip().split(":")[0].strip() for p in m.group(2).split(",") if p.strip()]
        depth, i = 1, m.end()
        while depth:
            depth += {"{": 1, "}": -1}.get(text[i], 0)
            i += 1
        out[m.group(1)] = (params, text[m.end():i - 1])
    return out


def call_args(body: str, start: int) -> int:
    """Top-level arguments of the call whose '(' is at body[start]."""
    depth, n, i = 0, 1, start
    while True:
        c = body[i]
        if c == "(":
            depth += 1
        elif c == ")":
            depth -= 1
            if depth == 0:
                return n if body[start + 1:i].strip() else 0
        elif c == "," and depth == 1:
            n += 1
        i += 1


@pytest.mark.parametrize("op", sorted(API))
def test_gpu_zig_keeps_the_reference_op(op):
    fns = zig_pub_fns()
    assert op in fns, op
    params, body = fns[op]
    assert params == API[op]["params"], (op, params, API[op]["params"])
    calls = [(m.group(1), m.end() - 1) for m in re.finditer(r"dkz\.(dkz_\w+)\(", body)]
    assert len(calls) == 1, (op, calls)
    arity = {z[0]: len(z[1]) for z in zig_externs()}
    name, at = calls[0]
    assert call_args(body, at) == arity[name], (op, name)


def test_gpu_zig_keeps_the_host_api():
    fns = zig_pub_fns()
    for name in ("init", "alloc", "allocInts", "make", "free", "push", "pull", "pullInts", "sync",
                 "setSyncAfterLaunch"):
        assert name in fns, name
    assert "pub const Buf = struct" in ZIG_GPU.read_text()
