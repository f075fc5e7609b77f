"""CPU check of the Rust binding (rust/willamette-hip-sys/src/sys.rs) against
the C header: the same functions, parameter types and return types, and the
same field order and types in the two plain structs.  There is no Rust
toolchain here, so this is the binding's only check."""
import re
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "willamette_hip.h"
SYS_RS = ROOT / "rust" / "willamette-hip-sys" / "src" / "sys.rs"

SCALAR = {"uint32_t": "u32", "uint64_t": "u64", "int64_t": "i64", "int": "c_int", "size_t": "usize",
          "float": "f32", "double": "f64", "int8_t": "i8", "uint8_t": "u8", "int32_t": "i32",
          "char": "c_char", "void": "c_void", "wm_status": "wm_status"}


def c_to_rust(ty: str) -> str:
    """A C parameter/return type as the Rust FFI type it must be bound to."""
    ty = " ".join(ty.split()).replace(" *", "*").replace("* ", "*")
    if "*" not in ty:
        return SCALAR.get(ty, ty)
    parts = ty.split("*")
    base = parts[0].strip()
    const = base.startswith("const ")
    base = SCALAR.get(base.replace("const ", "").strip(), base.replace("const ", "").strip())
    r = ("*const " if const else "*mut ") + base
    for q in parts[1:-1]:
        r = ("*const " if q.strip() == "const" else "*mut ") + r
    return r


def header_functions():
    t = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    out = {}
    for ret, name, args in re.findall(r"\n((?:const\s+)?[a-z_0-9]+\s*\**)\s*(wm_[a-z0-9_]+)\s*\(([^;]*?)\)\s*;",
                                      t, flags=re.S):
        params = []
        args = " ".join(args.split())
        for a in ([] if args in ("", "void") else args.split(",")):
            a = a.strip()
            m = re.match(r"(.*?)\s*([a-z_0-9]+)\[\d+\]$", a)
            if m:  # uint64_t shape[2] decays to a pointer
                params.append("*mut " + SCALAR.get(m.group(1), m.group(1)))
                continue
            m = re.match(r"(.*?)([a-z_0-9]+)$", a)
            params.append(c_to_rust(m.group(1)))
        r = ret.strip()
        out[name] = (params, None if r == "void" else c_to_rust(r))
    return out


def rust_functions():
    t = SYS_RS.read_text()
    block = t[t.index('extern "C" {'):]
    out = {}
    for name, args, ret in re.findall(r"pub fn (wm_[a-z0-9_]+)\((.*?)\)\s*(?:->\s*([^;]+))?;", block, flags=re.S):
        params = [p.split(":", 1)[1].strip() for p in args.split(",") if p.strip()]
        out[name] = (params, ret.strip() if ret else None)
    return out


def test_rust_extern_block_matches_header():
    h, r = header_functions(), rust_functions()
    assert len(h) > 80
    assert set(h) == set(r), set(h) ^ set(r)
    for name in h:
        assert h[name] == r[name], (name, h[name], r[name])


def struct_fields_c(name):
    t = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    body = re.search(r"typedef struct %s \{(.*?)\}" % name, t, flags=re.S).group(1)
    return [(f.split()[-1], SCALAR[f.split()[0]]) for f in (x.strip() for x in body.split(";")) if f]


def struct_fields_rust(name):
    t = SYS_RS.read_text()
    body = re.search(r"pub struct %s \{(.*?)\}" % name, t, flags=re.S).group(1)
    return [(n.strip().removeprefix("pub ").strip(), ty.strip())
            for n, ty in (x.split(":") for x in body.split(",") if x.strip())]


def test_rust_structs_match_header():
    for s in ("wm_model_config", "wm_sampling_params"):
        assert struct_fields_c(s) == struct_fields_rust(s), s


def test_status_codes_match_header():
    t = HEADER.read_text()
    c = dict(re.findall(r"(WM_[A-Z_0-9]+) = (\d+)", t))
    rs = dict(re.findall(r"pub const (WM_[A-Z_0-9]+): \w+ = (\d+);", SYS_RS.read_text()))
    for k, v in c.items():
        assert rs.get(k) == v, k
