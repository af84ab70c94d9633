"""CPU checks of the Rust binding crate (crates/coheryn-hip), which cannot be
compiled in this image (no cargo): every `extern "C"` declaration of
src/ffi.rs matches include/cohx.h in name, argument count and argument
types; every #[repr(C)] struct matches its C typedef field by field; and the
crate's build inputs exist (the manifest build.rs and build.py share)."""
import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CRATE = os.path.join(ROOT, "crates", "coheryn-hip")
HEADER = os.path.join(ROOT, "include", "cohx.h")
FFI = os.path.join(CRATE, "src", "ffi.rs")

# C spelling -> canonical spelling, and Rust spelling -> the same canonical one
C_SCALARS = {"int": "i32", "uint32_t": "u32", "uint64_t": "u64", "int32_t": "i32", "int64_t": "i64",
             "size_t": "usize", "float": "f32", "double": "f64", "char": "c_char", "uint8_t": "u8",
             "void": "void"}
RUST_SCALARS = {"c_int": "i32", "u32": "u32", "u64": "u64", "i32": "i32", "i64": "i64", "usize": "usize",
                "f32": "f32", "f64": "f64", "c_char": "c_char", "u8": "u8", "c_void": "void"}


def c_type(decl):
    """'const cohx_ctx *ctx' -> 'const cohx_ctx*'; function pointers -> 'fnptr'."""
    decl = " ".join(decl.split())
    if "(*" in decl:
        return "fnptr"
    decl = decl.replace("volatile ", "")
    m = re.match(r"^(.*?)([A-Za-z_]\w*)?(\[\d+\])?$", decl)
    body, array = m.group(1), m.group(3)
    if m.group(2) and not body.strip():
        body = m.group(2)  # a type with no parameter name
    body = body.replace("*", " * ").split()
    out, base = [], None
    for tok in body:
        if tok == "*":
            out.append("*")
        elif tok == "const":
            out.append("const")
        else:
            base = C_SCALARS.get(tok, tok)
    # pointer levels from right to left: `T *const *` = pointer to const pointer to T
    levels = []
    quals = []
    for tok in out:
        if tok == "const":
            quals.append("const")
        else:
            levels.append(quals)
            quals = []
    base_const = bool(levels) and "const" in levels[0]
    # in C, a leading `const T *` qualifies T; `T *const *` qualifies the first pointer
    s = base
    if not levels:
        return s + (array or "")
    mut = "const" if base_const else "mut"
    s = f"*{mut} {s}"
    for q in levels[1:]:
        mut = "const" if "const" in q else "mut"
        s = f"*{mut} {s}"
    return s + (array or "")


def rust_type(t):
    t = " ".join(t.split())
    if t.startswith("Option<unsafe extern") or t == "cohx_yield_fn":
        return "fnptr"
    m = re.match(r"^\[(\w+); (\d+)\]$", t)
    if m:
        return RUST_SCALARS.get(m.group(1), m.group(1)) + f"[{m.group(2)}]"
    ptrs = []
    while t.startswith("*"):
        m = re.match(r"^\*(const|mut) (.*)$", t)
        ptrs.append(m.group(1))
        t = m.group(2)
    s = RUST_SCALARS.get(t, t)
    for p in reversed(ptrs):
        s = f"*{p} {s}"
    return s


def header_functions():
    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    out = {}
    for m in re.finditer(r"^([A-Za-z_][\w\s\*]*?)\b(cohx_[a-z0-9_]+)\s*\(((?:[^;()]|\([^()]*\))*)\)\s*;", text,
                         flags=re.M | re.S):
        ret = c_type(m.group(1).strip())
        args = [a for a in re.split(r",(?![^()]*\))", " ".join(m.group(3).split())) if a.strip()]
        out[m.group(2)] = (ret if ret != "void" else "()", [c_type(a.strip()) for a in args])
    return out


def rust_functions():
    text = open(FFI).read()
    block = text[text.index('unsafe extern "C" {'):]
    out = {}
    for m in re.finditer(r"pub fn (cohx_\w+)\s*\(([^;]*?)\)\s*(?:->\s*([^;]+?))?\s*;", block, flags=re.S):
        args = [a.strip() for a in re.split(r",(?![^<>]*>)", " ".join(m.group(2).split())) if a.strip()]
        types = [rust_type(a.split(":", 1)[1]) for a in args]
        ret = rust_type(m.group(3)) if m.group(3) else "()"
        out[m.group(1)] = (ret, types)
    return out


def test_every_header_function_is_bound_with_the_same_signature():
    c, rust = header_functions(), rust_functions()
    assert len(c) >= 37
    assert sorted(c) == sorted(rust), (set(c) ^ set(rust))
    for name, (ret, args) in c.items():
        assert rust[name][0] == ret, (name, rust[name][0], ret)
        assert rust[name][1] == args, (name, rust[name][1], args)


def header_structs():
    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    out = {}
    for m in re.finditer(r"typedef struct\s*\{(.*?)\}\s*(cohx_\w+)\s*;", text, flags=re.S):
        fields = []
        for decl in m.group(1).split(";"):
            decl = " ".join(decl.split())
            if not decl:
                continue
            if "(*" in decl:
                fields.append(("fnptr", re.search(r"\(\*(\w+)\)", decl).group(1)))
                continue
            # `uint32_t a, b, c` declares several fields of one type
            bm = re.match(r"^((?:(?:const|volatile)\s+)*\w+)\s*(.*)$", decl)
            base, declarators = bm.group(1), bm.group(2)
            for d in declarators.split(","):
                nm = re.match(r"^\s*(\**)\s*(?:const\s+)?(\w+)(\[\d+\])?\s*$", d)
                fields.append((c_type(f"{base} {nm.group(1)}{nm.group(2)}{nm.group(3) or ''}"), nm.group(2)))
        out[m.group(2)] = fields
    return out


def rust_structs():
    text = open(FFI).read()
    out = {}
    for m in re.finditer(r"#\[repr\(C\)\]\s*(?:#\[derive[^\]]*\]\s*)?pub struct (cohx_\w+)\s*\{(.*?)\n\}", text,
                         flags=re.S):
        fields = []
        for line in m.group(2).split("\n"):
            line = line.strip().rstrip(",")
            fm = re.match(r"^pub (\w+): (.+)$", line)
            if fm:
                fields.append((rust_type(fm.group(2)), fm.group(1).rstrip("_")))
        out[m.group(1)] = fields
    return out


def test_every_header_struct_has_the_same_fields():
    c, rust = header_structs(), rust_structs()
    assert {"cohx_model_desc", "cohx_lane", "cohx_batch", "cohx_step_out", "cohx_qwen35_desc",
            "cohx_gen_options", "cohx_batch_step"} <= set(c)
    for name, fields in c.items():
        assert name in rust, name
        assert rust[name] == fields, (name, rust[name], fields)


def test_crate_allows_unsafe_and_builds_from_the_shared_manifest():
    cargo = open(os.path.join(CRATE, "Cargo.toml")).read()
    # the workspace forbids unsafe code (reference Cargo.toml [workspace.lints.rust]);
    # the crate keeps its own lint table instead of inheriting it
    assert re.search(r"^\[lints\.rust\]\s*\nunsafe_code = \"allow\"", cargo, flags=re.M)
    assert not re.search(r"^\[lints\]\s*\nworkspace = true", cargo, flags=re.M)
    build_rs = open(os.path.join(CRATE, "build.rs")).read()
    assert "build.manifest" in build_rs and "--offload-arch={arch}" in build_rs
    import sys
    sys.path.insert(0, os.path.join(ROOT, "coheryn-ai-studio_amd"))
    import build
    m = build.manifest()
    for src in m["sources"]:
        assert os.path.exists(os.path.join(ROOT, "coheryn-ai-studio_amd", src)), src
    assert "-ffp-contract=off" in m["flags"]


def test_type_mapping_catches_a_wrong_binding():
    """The comparison itself distinguishes const from mut, widths and levels."""
    assert c_type("const cohx_ctx *ctx") == "*const cohx_ctx"
    assert c_type("cohx_gen *const *states") == "*const *mut cohx_gen"
    assert c_type("cohx_ctx **out") == "*mut *mut cohx_ctx"
    assert c_type("size_t bytes") == "usize"
    assert rust_type("*const *mut cohx_gen") == "*const *mut cohx_gen"
    assert rust_type("*mut u32") != c_type("int32_t *out")
    assert rust_type("c_int") == c_type("int device")
