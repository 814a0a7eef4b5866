"""Pins INTEGRATION.md's reference-side binding to the library it binds (CPU only).

The Rust crate a maintainer adds (`crates/backend-hip`, standing where the reference's
`crates/backend-cuda/build.rs:7-57` and its FFI stand) is written out in INTEGRATION.md but cannot
be compiled here (no Rust toolchain). These tests keep it from drifting:

* the `extern "C"` block declares exactly the functions of `include/helix_hip.h`, in order, with the
  same argument count and the header's C types spelled in Rust;
* `check()` maps every status code to the `TensorError` variant the header names for it
  (`crates/tensor-core/src/error.rs:7-37`);
* `build.rs` takes every `csrc/*.hip` file (read from the directory) with `helixml_amd/build.py`'s
  hipcc flags, and a library linked from exactly those sources with `--no-undefined` resolves
  every name the extern block declares.
"""
from __future__ import annotations

import re
import shutil
import subprocess
from pathlib import Path

import pytest

from helixml_amd import build as hb

ROOT = Path(__file__).resolve().parents[1]
DOC = ROOT / "INTEGRATION.md"
HEADER = ROOT / "include" / "helix_hip.h"

# C type of the header -> its Rust spelling in the extern block
C_TO_RUST = {
    "int64_t": "i64", "int": "c_int", "size_t": "usize", "float": "f32", "double": "f64",
    "const float*": "*const f32", "float*": "*mut f32", "const void*": "*const c_void",
    "void*": "*mut c_void", "void**": "*mut *mut c_void", "const int32_t*": "*const i32",
    "const int64_t*": "*const i64", "int*": "*mut c_int", "size_t*": "*mut usize",
    "double*": "*mut f64", "const char*": "*const c_char",
}


def _strip_c_comments(s: str) -> str:
    return re.sub(r"/\*.*?\*/", "", s, flags=re.S)


def header_functions() -> list[tuple[str, str, list[str]]]:
    """(name, return type, [argument types]) of every function the header declares, in order."""
    h = _strip_c_comments(HEADER.read_text())
    out = []
    for m in re.finditer(r"^([A-Za-z_][\w \*]*?)\s*\b(hx_\w+)\s*\((.*?)\)\s*;", h, flags=re.S | re.M):
        ret = " ".join(m.group(1).split()).replace(" *", "*")
        args = " ".join(m.group(3).split())
        types = []
        if args != "void":
            for a in args.split(","):
                a = a.strip()
                mm = re.match(r"(.*?)\b(\w+)$", a)
                assert mm, a
                types.append(" ".join(mm.group(1).split()).replace(" *", "*"))
        out.append((m.group(2), ret, types))
    return out


def _rust_blocks() -> list[str]:
    return re.findall(r"```rust\n(.*?)```", DOC.read_text(), flags=re.S)


def rust_extern_functions() -> list[tuple[str, str, list[str]]]:
    """(name, return type, [argument types]) of every `pub fn` in INTEGRATION.md's extern block."""
    blocks = [b for b in _rust_blocks() if 'extern "C"' in b]
    assert len(blocks) == 1, "INTEGRATION.md must hold exactly one extern \"C\" block"
    body = blocks[0].split('extern "C" {', 1)[1]
    body = body[: body.index("\n}")]
    body = re.sub(r"//[^\n]*", "", body)
    out = []
    for m in re.finditer(r"pub fn (hx_\w+)\s*\((.*?)\)\s*->\s*([^;]+);", body, flags=re.S):
        args = " ".join(m.group(2).split())
        types = [a.split(":", 1)[1].strip() for a in args.split(",") if a.strip()] if args else []
        out.append((m.group(1), " ".join(m.group(3).split()), types))
    return out


def test_extern_block_matches_header():
    hdr = header_functions()
    rs = rust_extern_functions()
    assert len(hdr) >= 40, "header parse found too few functions"
    assert [n for n, _, _ in rs] == [n for n, _, _ in hdr], (
        "extern block and header differ in names/order:\n"
        f"missing in doc: {sorted(set(n for n, _, _ in hdr) - set(n for n, _, _ in rs))}\n"
        f"not in header: {sorted(set(n for n, _, _ in rs) - set(n for n, _, _ in hdr))}")
    for (name, cret, cargs), (_, rret, rargs) in zip(hdr, rs):
        assert len(rargs) == len(cargs), f"{name}: {len(rargs)} args in the doc, {len(cargs)} in the header"
        assert rret == C_TO_RUST[cret], f"{name}: returns {rret}, header {cret}"
        for i, (ct, rt) in enumerate(zip(cargs, rargs)):
            assert rt == C_TO_RUST[ct], f"{name} arg {i}: {rt} in the doc, {ct} in the header"


def test_parsers_catch_a_drift():
    """A dropped argument or a renamed function in the doc text must fail the comparison."""
    rs = rust_extern_functions()
    hdr = header_functions()
    name, ret, args = rs[12]
    assert len(args) == len(hdr[12][2])
    assert len(args[:-1]) != len(hdr[12][2])
    assert {n for n, _, _ in hdr} - {n for n, _, _ in rs[1:]} == {rs[0][0]}


def test_check_maps_every_status_to_its_variant():
    h = HEADER.read_text()
    enum = re.search(r"typedef enum \{(.*?)\} hx_status;", h, flags=re.S).group(1)
    want = {}
    for m in re.finditer(r"HX_(\w+)\s*=\s*(\d+),?\s*(?:/\*\s*TensorError::(\w+))?", enum):
        if m.group(3):
            want[int(m.group(2))] = m.group(3)
    assert len(want) == 10 and sorted(want) == list(range(1, 11))
    blocks = [b for b in _rust_blocks() if "pub fn check(" in b]
    assert len(blocks) == 1
    got = {int(m.group(1)): m.group(2)
           for m in re.finditer(r"^\s*(\d+)\s*=>\s*E::(\w+)", blocks[0], flags=re.M)}
    assert got == want


def _build_rs() -> str:
    blocks = [b for b in _rust_blocks() if "fn main()" in b and "hipcc" in b]
    assert len(blocks) == 1, "INTEGRATION.md must hold exactly one build.rs"
    return blocks[0]


def build_rs_flags() -> list[str]:
    m = re.search(r"const HIPCC_FLAGS: &\[&str\] = &\[(.*?)\];", _build_rs(), flags=re.S)
    assert m, "build.rs must list its hipcc flags in HIPCC_FLAGS"
    return re.findall(r'"([^"]*)"', m.group(1))


def test_build_rs_takes_every_hip_source_with_the_library_flags():
    src = _build_rs()
    # the source list is the directory's *.hip files, not a hand-kept list
    assert re.search(r"fs::read_dir\(&csrc\)", src)
    assert re.search(r'x == "hip"', src)
    assert not re.search(r'"hx_\w+"', src), "build.rs must not name sources by hand"
    assert "--no-undefined" in src
    # flags: build.py's, without the arch (build.rs passes HELIX_HIP_ARCH), warnings and -I
    ours = [f for f in hb.HIPCC_FLAGS
            if not f.startswith(("--offload-arch", "-W", "-I"))]
    assert build_rs_flags() == ours


def _objects_for(srcs: list[Path], tmp: Path) -> list[Path]:
    """The build's objects where they are newer than every source and header they depend on,
    else fresh ones compiled with build.rs's flags."""
    deps = list(hb.CSRC.glob("*.h")) + list(hb.INCLUDE.rglob("*.h"))
    newest_dep = max(p.stat().st_mtime for p in deps)
    objs, todo = [], []
    for s in srcs:
        o = hb.OBJDIR / (s.stem + ".o")
        if o.exists() and o.stat().st_mtime > max(s.stat().st_mtime, newest_dep):
            objs.append(o)
        else:
            todo.append(s)
    flags = build_rs_flags()
    procs = []
    for s in todo:
        o = tmp / (s.stem + ".o")
        cmd = [hb.hipcc(), f"--offload-arch={hb.ARCH}", *flags, f"-I{hb.INCLUDE}", f"-I{hb.CSRC}",
               "-c", str(s), "-o", str(o)]
        procs.append((s, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT)))
        objs.append(o)
    for s, p in procs:
        out = p.communicate()[0]
        assert p.returncode == 0, f"hipcc failed on {s.name}:\n{out.decode()[-2000:]}"
    return objs


@pytest.mark.skipif(shutil.which("gcc") is None, reason="gcc needed")
def test_library_from_build_rs_sources_resolves_every_extern(tmp_path):
    srcs = sorted(hb.CSRC.glob("*.hip"))
    assert srcs
    objs = _objects_for(srcs, tmp_path)
    lib = tmp_path / "libhelix_hip.so"
    r = subprocess.run([hb.hipcc(), f"--offload-arch={hb.ARCH}", "-shared", "-fPIC",
                        "-Wl,--no-undefined", *map(str, objs), "-o", str(lib)],
                       capture_output=True, text=True)
    assert r.returncode == 0, f"link with --no-undefined failed:\n{r.stdout}\n{r.stderr}"
    names = [n for n, _, _ in rust_extern_functions()]
    prog = tmp_path / "uses_every_extern.c"
    prog.write_text("".join(f"extern char {n};\n" for n in names)
                    + "void* table[] = {" + ", ".join(f"&{n}" for n in names) + "};\n"
                    + "int main(void) { return table[0] == 0; }\n")
    r = subprocess.run(["gcc", str(prog), f"-L{tmp_path}", "-lhelix_hip", "-Wl,--no-undefined",
                        "-Wl,-rpath-link,/opt/rocm/lib", "-o", str(tmp_path / "uses_every_extern")],
                       capture_output=True, text=True)
    assert r.returncode == 0, f"an extern of the doc is not defined by the library:\n{r.stderr}"
    # the same link without one source must fail: the check has teeth
    prim = [o for o in objs if o.stem == "hx_prim"]
    assert prim
    r = subprocess.run([hb.hipcc(), f"--offload-arch={hb.ARCH}", "-shared", "-fPIC",
                        "-Wl,--no-undefined", *[str(o) for o in objs if o.stem != "hx_prim"],
                        "-o", str(tmp_path / "libpartial.so")], capture_output=True, text=True)
    assert r.returncode != 0 and "hx_fill_f32" in (r.stdout + r.stderr)
