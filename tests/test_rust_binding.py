"""The Rust binding (index-tts-rs_amd/rust/itts-hip-sys) against the C ABI (include/itts_hip.h),
checked mechanically since this image has no Rust toolchain: every C function is declared in
the extern block with the same parameter and return types (C declarators canonicalised to
Rust pointer forms: `const T *` -> `*const T`, `T *const *` -> `*const *mut T`, arrays as
pointers, enums as i32), every #[repr(C)] struct has the C struct's fields in the same order
and types, and every `sys::` item the safe wrapper crate (rust/core-hip) uses exists."""
import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "itts_hip.h")
SYS = os.path.join(ROOT, "index-tts-rs_amd", "rust", "itts-hip-sys", "src", "lib.rs")
WRAP = os.path.join(ROOT, "index-tts-rs_amd", "rust", "core-hip", "src", "lib.rs")

BASE = {"int32_t": "i32", "uint32_t": "u32", "int64_t": "i64", "uint64_t": "u64", "float": "f32",
        "void": "c_void", "char": "c_char", "itts_status": "i32", "itts_dtype": "i32",
        "itts_decode_path": "i32"}
ALIAS = {"itts_status": "i32", "itts_dtype": "i32", "itts_decode_path": "i32"}


def c_to_rust(decl):
    """(type, name) of one C declarator, the type in canonical Rust spelling."""
    decl = decl.strip()
    arr = re.search(r"\[\s*\d*\s*\]$", decl)
    if arr:
        decl = decl[:arr.start()].strip()
    m = re.match(r"^(.*?)([A-Za-z_]\w*)$", decl)
    head, name = m.group(1), m.group(2)
    toks = re.findall(r"\*|const|[A-Za-z_]\w*", head)
    base_const, base, stars = False, None, []
    for t in toks:
        if t == "const":
            if stars:
                stars[-1] = True
            else:
                base_const = True
        elif t == "*":
            stars.append(False)
        elif t not in ("struct", "enum"):
            base = t
    if arr:
        stars.append(False)
    s = BASE.get(base, base)
    prev_const = base_const
    for star_const in stars:
        s = ("*const " if prev_const else "*mut ") + s
        prev_const = star_const
    return s, name


def strip_c(src):
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    src = re.sub(r"//[^\n]*", "", src)
    return re.sub(r"^\s*#[^\n]*", "", src, flags=re.M)


def c_structs(src):
    out = {}
    for m in re.finditer(r"typedef\s+struct\s+(\w+)\s*\{(.*?)\}\s*(\w+)\s*;", src, re.S):
        fields = []
        for stmt in m.group(2).split(";"):
            stmt = " ".join(stmt.split())
            if not stmt:
                continue
            first, *rest = stmt.split(",")
            t, n = c_to_rust(first)
            fields.append((n, t))
            # further declarators share the base type: `const float *a, *b` / `int32_t a, b`
            base = re.match(r"^((?:const\s+)?[A-Za-z_]\w*)", first.strip()).group(1)
            for r in rest:
                t2, n2 = c_to_rust(base + " " + r.strip())
                fields.append((n2, t2))
        out[m.group(3)] = fields
    return out


def c_functions(src):
    body = re.sub(r"typedef\s+(struct|enum)\s+\w*\s*\{.*?\}\s*\w+\s*;", "", src, flags=re.S)
    body = re.sub(r"typedef\s+struct\s+\w+\s+\w+\s*;", "", body)
    out = {}
    for m in re.finditer(r"([A-Za-z_][\w\s\*]*?)\b(itts_\w+)\s*\(([^;]*?)\)\s*;", body, re.S):
        ret = " ".join(m.group(1).split())
        rt, _ = c_to_rust(ret + " x")
        params = [] if m.group(3).strip() in ("", "void") else [c_to_rust(" ".join(p.split()))[0]
                                                                for p in m.group(3).split(",")]
        out[m.group(2)] = ("" if rt == "c_void" else rt, params)
    return out


def rust_norm(t):
    t = " ".join(t.replace("*const", " *const ").replace("*mut", " *mut ").split())
    return " ".join(ALIAS.get(w, w) for w in t.split())


def rust_items(src):
    fns = {}
    ext = src[src.index('extern "C"'):]
    for m in re.finditer(r"pub fn (itts_\w+)\s*\((.*?)\)\s*(?:->\s*([^;]+))?;", ext, re.S):
        args = [a for a in (x.strip() for x in m.group(2).split(",")) if a]
        fns[m.group(1)] = (rust_norm(m.group(3) or ""), [rust_norm(a.split(":", 1)[1]) for a in args])
    structs = {}
    for m in re.finditer(r"pub struct (\w+)\s*\{(.*?)\}", src, re.S):
        fields = re.findall(r"pub (\w+):\s*([^,\n]+),", m.group(2))
        structs[m.group(1)] = [(n, rust_norm(t)) for n, t in fields]
    return fns, structs


def test_sys_crate_declares_the_c_abi():
    c_src = strip_c(open(HEADER).read())
    cf, cs = c_functions(c_src), c_structs(c_src)
    rf, rs = rust_items(open(SYS).read())
    assert len(cf) >= 45
    assert set(cf) == set(rf), (sorted(set(cf) - set(rf)), sorted(set(rf) - set(cf)))
    for name, (ret, params) in cf.items():
        rret, rparams = rf[name]
        assert rust_norm(ret) == rret, (name, ret, rret)
        assert [rust_norm(p) for p in params] == rparams, (name, params, rparams)
    for name, fields in cs.items():
        assert name in rs, name
        assert [(n, rust_norm(t)) for n, t in fields] == rs[name], (name, fields, rs[name])


def test_declarator_canonicalisation():
    assert c_to_rust("const int32_t *x")[0] == "*const i32"
    assert c_to_rust("itts_kv *const *caches")[0] == "*const *mut itts_kv"
    assert c_to_rust("const char *const *names")[0] == "*const *const c_char"
    assert c_to_rust("itts_gpt **out")[0] == "*mut *mut itts_gpt"
    assert c_to_rust("const uint64_t seen[129]")[0] == "*const u64"
    assert c_to_rust("uint64_t words[129]")[0] == "*mut u64"


def test_wrapper_uses_only_declared_items():
    rf, rs = rust_items(open(SYS).read())
    sys_src = open(SYS).read()
    consts = set(re.findall(r"pub const (\w+)", sys_src)) | set(re.findall(r"pub type (\w+)", sys_src))
    used = set(re.findall(r"sys::(\w+)", open(WRAP).read()))
    missing = [u for u in used if u not in rf and u not in rs and u not in consts]
    assert not missing, missing
