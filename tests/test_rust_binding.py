"""The Rust binding (ai-engine_amd/rust/ffi.rs) declares exactly the C ABI
of include/pagedkv.h: every function with the same argument names, order and
types (const-ness of every pointee included) and return type, every integer
constant with its value, and every struct with the same fields in the same
order.  Both files are parsed here; a header change that the binding does
not follow fails this test."""
import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "pagedkv.h")
FFI = os.path.join(ROOT, "ai-engine_amd", "rust", "ffi.rs")
BUILD = os.path.join(ROOT, "ai-engine_amd", "rust", "build.rs")

C_BASE = {"int": "c_int", "float": "f32", "double": "f64", "size_t": "usize",
          "long long": "c_longlong", "uint64_t": "u64", "int64_t": "i64", "int32_t": "i32",
          "uint32_t": "u32", "int8_t": "i8", "char": "c_char", "void": "c_void"}


def _rust_name(c):  # pkv_sched_plan -> PkvSchedPlan
    return "".join(w.capitalize() for w in c.split("_"))


def c_to_rust(ctype):
    """C type spelling -> the Rust type the binding must use."""
    toks = ctype.replace("*", " * ").split()
    stars = toks.count("*")
    const = "const" in toks[:toks.index("*")] if stars else False
    base = " ".join(t for t in toks if t not in ("*", "const"))
    r = C_BASE.get(base) or (_rust_name(base) if base.startswith("pkv_") else None)
    assert r, f"unmapped C type {ctype!r}"
    if stars == 0:
        return r
    r = ("*const " if const else "*mut ") + r
    return "*mut " * (stars - 1) + r


def _strip_c_comments(s):
    return re.sub(r"//[^\n]*", "", re.sub(r"/\*.*?\*/", "", s, flags=re.S))


def header():
    src = _strip_c_comments(open(HEADER).read())
    fns = {}
    for ret, name, args in re.findall(r"([A-Za-z_][\w \*]*?)\b(pkv_\w+)\s*\(([^;{)]*)\)\s*;", src):
        params = []
        a = " ".join(args.split())
        if a not in ("", "void"):
            for p in a.split(","):
                m = re.match(r"(.*?)(\w+)$", p.strip())
                params.append((m.group(2), c_to_rust(m.group(1))))
        rt = " ".join(ret.split())
        fns[name] = (params, None if rt == "void" else c_to_rust(rt))
    consts = {k: int(v) for k, v in re.findall(r"#define\s+(PKV_\w+)\s+\(?(-?\d+)\)?\s*$", src, re.M)}
    structs = {}
    for body, name in re.findall(r"typedef struct(?: \w+)?\s*\{(.*?)\}\s*(\w+)\s*;", src, re.S):
        fields = []
        for decl in body.split(";"):
            decl = " ".join(decl.split())
            if not decl:
                continue
            m = re.match(r"(.*?)(\w+(?:\s*\[\d+\])?(?:\s*,\s*\w+)*)$", decl)
            ctype, names = m.group(1).strip(), m.group(2)
            for n in names.split(","):
                n = n.strip()
                arr = re.match(r"(\w+)\s*\[(\d+)\]", n)
                if arr:
                    fields.append((arr.group(1), f"[{c_to_rust(ctype)}; {arr.group(2)}]"))
                else:
                    fields.append((n, c_to_rust(ctype)))
        structs[_rust_name(name)] = fields
    opaque = {_rust_name(n) for n in re.findall(r"typedef struct (\w+) \1;", src)}
    return fns, consts, structs, opaque


def binding():
    src = re.sub(r"//[^\n]*", "", open(FFI).read())
    block = src[src.index('extern "C" {'):]
    block = block[:block.index("\n}")]
    fns = {}
    for name, args, ret in re.findall(r"pub fn (\w+)\s*\((.*?)\)\s*(?:->\s*([^;]+?))?\s*;", block, re.S):
        params = []
        a = " ".join(args.split()).rstrip(",")
        if a:
            for p in a.split(","):
                n, t = p.split(":", 1)
                params.append((n.strip(), " ".join(t.split())))
        fns[name] = (params, " ".join(ret.split()) if ret else None)
    consts = {k: int(v) for k, v in re.findall(r"pub const (PKV_\w+): c_int = (-?\d+);", src)}
    structs = {}
    for name, body in re.findall(r"#\[repr\(C\)\]\s*pub struct (\w+)\s*\{(.*?)\}", src, re.S):
        fields = [(n, " ".join(t.split())) for n, t in
                  re.findall(r"pub (\w+):\s*([^,]+?),\s*(?=pub|$)", " ".join(body.split()) + " ")]
        structs[name] = fields
    return fns, consts, structs


def test_every_function_is_declared_alike():
    hf, _, _, _ = header()
    rf, _, _ = binding()
    assert len(hf) >= 60
    assert sorted(hf) == sorted(rf), (set(hf) ^ set(rf))
    for name, (params, ret) in hf.items():
        assert rf[name] == (params, ret), f"{name}: header {params} -> {ret}, ffi.rs {rf[name]}"


def test_constants_and_structs_match():
    _, hc, hs, opaque = header()
    _, rc, rs = binding()
    for k, v in hc.items():
        assert rc.get(k) == v, f"{k}: header {v}, ffi.rs {rc.get(k)}"
    for name, fields in hs.items():
        assert rs.get(name) == fields, f"{name}: header {fields}, ffi.rs {rs.get(name)}"
    for name in opaque:
        assert name in rs and rs[name] == [], name  # opaque handle: no public fields
    noalloc = re.search(r"PKV_NOALLOC_SCRATCH_BYTES\s+\(\(size_t\)(\d+) << (\d+)\)",
                        open(HEADER).read())
    rs_noalloc = re.search(r"PKV_NOALLOC_SCRATCH_BYTES: usize = (\d+) << (\d+);", open(FFI).read())
    assert noalloc and rs_noalloc and noalloc.groups() == rs_noalloc.groups()


def test_the_parsers_see_a_planted_difference():
    # not vacuous: a dropped const, a swapped argument and a missing function
    # are all told apart by the comparison above
    hf, _, _, _ = header()
    params, ret = hf["pkv_decode_workspace_bytes"]
    assert params[0] == ("pool", "*const PkvPool") and ret == "usize"
    assert c_to_rust("const float**") == "*mut *const f32"
    assert c_to_rust("pkv_pool**") == "*mut *mut PkvPool"
    assert c_to_rust("const int32_t*") != c_to_rust("int32_t*")
    p2 = list(params)
    p2[1], p2[2] = p2[2], p2[1]
    assert (p2, ret) != hf["pkv_decode_workspace_bytes"]


def test_build_script_uses_the_library_build():
    b = open(BUILD).read()
    assert "build.py" in b and "rustc-link-lib=dylib=pagedkv" in b
    assert os.path.exists(os.path.join(ROOT, "ai-engine_amd", "build.py"))
