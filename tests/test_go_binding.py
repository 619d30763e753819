"""The Go drop-in (go/mixtureofexperts/gpu_unix.go) against the C ABI it
binds, without a Go toolchain:

* its mirror structs gtmoeLayerDesc and gtmoeRows, laid out by Go's rules
  for 64-bit targets (each field at the next multiple of its alignment,
  int32 4, float64 / pointers / uintptr 8, the size rounded to the largest
  alignment), field by field against gcc's offsetof and sizeof of
  gtmoe_layer_desc and gtmoe_rows (tests/go_layout/layout.c);
* every entry point it registers with purego is declared in include/gtmoe.h,
  exported by libgtmoe.so, and takes as many arguments as the Go function
  type it is registered into."""
import os
import re
import shutil
import subprocess

import pytest

import gotransformers_amd as gt

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GO_FILE = os.path.join(ROOT, "go", "mixtureofexperts", "gpu_unix.go")

GO_SIZES = {"int32": 4, "uint32": 4, "int64": 8, "float64": 8, "uintptr": 8, "unsafe.Pointer": 8}


def go_struct_layout(source, name):
    """[(field, offset, size)] and the size of Go struct `name` in `source`."""
    body = re.search(r"type\s+" + name + r"\s+struct\s*\{(.*?)\n\}", source, re.S).group(1)
    fields = []
    for line in body.strip().splitlines():
        line = line.split("//")[0].strip()
        if not line:
            continue
        *names, typ = line.replace(",", " ").split()
        fields += [(n, typ) for n in names]
    out, off, biggest = [], 0, 1
    for field, typ in fields:
        size = GO_SIZES[typ] if not typ.startswith("*") else 8
        off = (off + size - 1) // size * size
        out.append((field, off, size))
        off += size
        biggest = max(biggest, size)
    return out, (off + biggest - 1) // biggest * biggest


def c_layouts(tmp_path):
    exe = tmp_path / "layout"
    r = subprocess.run(["gcc", "-std=c11", "-Wall", "-I", os.path.join(ROOT, "include"),
                        os.path.join(ROOT, "tests", "go_layout", "layout.c"), "-o", str(exe)],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    lines = subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.splitlines()
    fields, sizes = {}, {}
    for ln in lines:
        parts = ln.split()
        if parts[1] == "sizeof":
            sizes[parts[0]] = int(parts[2])
        else:
            fields.setdefault(parts[0], []).append((parts[1], int(parts[2]), int(parts[3])))
    return fields, sizes


def camel(snake):
    return "".join(p.capitalize() for p in snake.split("_"))


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
@pytest.mark.parametrize("go_name,c_name", [("gtmoeLayerDesc", "gtmoe_layer_desc"), ("gtmoeRows", "gtmoe_rows")])
def test_go_structs_match_the_c_abi(tmp_path, go_name, c_name):
    source = open(GO_FILE).read()
    go_fields, go_size = go_struct_layout(source, go_name)
    fields, sizes = c_layouts(tmp_path)
    assert go_size == sizes[c_name]
    assert len(go_fields) == len(fields[c_name])
    for (gf, goff, gsize), (cf, coff, csize) in zip(go_fields, fields[c_name]):
        assert gf == camel(cf), (gf, cf)
        assert (goff, gsize) == (coff, csize), (gf, goff, gsize, cf, coff, csize)


def c_prototypes():
    text = open(os.path.join(ROOT, "include", "gtmoe.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    protos = {}
    for m in re.finditer(r"\b(gtmoe_[a-z0-9_]+)\s*\(([^)]*)\)\s*;", text):
        args = m.group(2).strip()
        protos[m.group(1)] = 0 if args in ("", "void") else args.count(",") + 1
    return protos


def test_registered_entry_points_exist_with_matching_arity():
    source = open(GO_FILE).read()
    registered = dict(re.findall(r'"(gtmoe_[a-z0-9_]+)":\s*&(\w+)', source))
    assert len(registered) >= 9
    protos = c_prototypes()
    lib = gt.library()
    for c_name, go_var in registered.items():
        assert c_name in protos, c_name
        assert hasattr(lib, c_name), c_name
        sig = re.search(r"\b" + go_var + r"\s+func\((.*?)\)", source).group(1)
        # every parameter is written as "name type", so commas count them
        go_arity = 0 if not sig.strip() else sig.count(",") + 1
        assert go_arity == protos[c_name], (c_name, sig, protos[c_name])
