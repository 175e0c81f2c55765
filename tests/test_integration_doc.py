"""The Rust binding that INTEGRATION.md documents agrees with include/pkv.h, field by
field and parameter by parameter (CPU only; no library call).

A maintainer builds paramecia's `pkv_sys.rs` from INTEGRATION.md's Rust block, so a
struct or prototype that drifts from the C header is an ABI break at the FFI boundary
(restore_prefix_cache, qwen3_next.rs:5726-5740, passes an array of `PkvLayerTarget`
whose stride must equal sizeof(pkv_layer_target)). The header is parsed with a small
C-declaration reader, each C type is mapped to the Rust type with the same size,
alignment and indirection, and the two sides are compared:
  - every `#[repr(C)]` struct: field names, order and types;
  - every `extern "C"` function: present on both sides, same parameter types in order,
    same return type;
  - every `pub const` of the Rust block: the header's enum value.
"""
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

# C scalar / opaque names -> Rust spellings (std::os::raw and the binding's own types)
SCALARS = {
    "int": "c_int", "int64_t": "i64", "uint64_t": "u64", "uint32_t": "u32", "size_t": "usize",
    "float": "f32", "double": "f64", "char": "c_char", "void": "c_void",
    "pkv_cache": "PkvCache", "pkv_prefix": "PkvPrefix", "pkv_pool": "PkvPool",
    "pkv_seq": "PkvSeq", "pkv_rope": "PkvRope", "pkv_qk_prep": "PkvQkPrep",
    "pkv_layer_target": "PkvLayerTarget",
}
TYPEDEF_PTRS = {"pkv_stream": "*mut c_void"}  # typedef void *pkv_stream


def _strip_c(text):
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    text = re.sub(r"//[^\n]*", "", text)
    text = re.sub(r"^\s*#[^\n]*", "", text, flags=re.M)
    return text


def c_to_rust(decl):
    """Rust type of one C parameter / field declaration (name included), and the name.
    Pointer levels read right to left: `const float *const *x` is `*const *const f32`;
    an array parameter `int64_t s[4]` decays to a pointer."""
    decl = " ".join(decl.replace("*", " * ").split())
    m = re.match(r"^(.*?)([A-Za-z_]\w*)\s*(\[\s*\d*\s*\])?$", decl)
    assert m, decl
    tpart, name, arr = m.group(1).strip(), m.group(2), m.group(3)
    toks = tpart.split()
    # base type: the tokens before the first '*', minus qualifiers
    base_toks, rest = [], []
    for i, t in enumerate(toks):
        if t == "*":
            rest = toks[i:]
            break
        base_toks.append(t)
    base_const = "const" in base_toks
    base = [t for t in base_toks if t not in ("const", "struct", "unsigned", "signed")]
    assert len(base) == 1, decl
    b = base[0]
    if b in TYPEDEF_PTRS:
        rust = TYPEDEF_PTRS[b]
        levels = []
    else:
        rust = SCALARS[b]
        levels = []
    # each '*' makes a pointer whose pointee constness is the qualifier before it
    pointee_const = base_const
    for t in rest:
        if t == "*":
            levels.append(pointee_const)
            pointee_const = False
        elif t == "const":
            pointee_const = True  # the pointer itself is const: pointee of the NEXT level
    if arr is not None:
        levels.append(base_const if not levels else pointee_const)
    for c in levels:
        rust = ("*const " if c else "*mut ") + rust
    return rust, name


def header_decls():
    text = _strip_c(open(os.path.join(ROOT, "include", "pkv.h")).read())
    structs = {}
    for body, name in re.findall(r"typedef\s+struct\s*\{(.*?)\}\s*(\w+)\s*;", text, flags=re.S):
        fields = []
        for stmt in body.split(";"):
            stmt = " ".join(stmt.split())
            if not stmt:
                continue
            # `size_t a, b, c` declares several fields of one type
            head, *more = [s.strip() for s in stmt.split(",")]
            rt, fname = c_to_rust(head)
            fields.append((fname, rt))
            base = head[: head.rfind(fname)].strip()
            for extra in more:
                rt2, fname2 = c_to_rust(base + " " + extra)
                fields.append((fname2, rt2))
        structs[SCALARS[name]] = fields
    funcs = {}
    rest = re.sub(r"typedef\s+struct\s*\{.*?\}\s*\w+\s*;", ";", text, flags=re.S)
    rest = re.sub(r"enum\s*\{.*?\}\s*;", ";", rest, flags=re.S)
    rest = rest.replace('extern "C" {', ";").replace("}", ";")
    for stmt in rest.split(";"):
        m = re.match(r"^\s*([A-Za-z_][\w\s\*]*?)\b(pkv_\w+)\s*\((.*)\)\s*$", stmt, flags=re.S)
        if not m:
            continue
        ret, name, params = m.groups()
        ret = " ".join(ret.split())
        rret = None if ret == "void" else c_to_rust(ret + " r")[0]
        ps = []
        params = " ".join(params.split())
        if params and params != "void":
            for p in params.split(","):
                ps.append(c_to_rust(p.strip())[0])
        funcs[name] = (ps, rret)
    enums = {}
    for body in re.findall(r"enum\s*\{(.*?)\}", text, flags=re.S):
        for k, v in re.findall(r"(PKV_\w+)\s*=\s*(\d+)", body):
            enums[k] = int(v)
    return structs, funcs, enums


def rust_block():
    md = open(os.path.join(ROOT, "INTEGRATION.md")).read()
    blocks = re.findall(r"```rust\n(.*?)```", md, flags=re.S)
    decl = [b for b in blocks if 'extern "C"' in b]
    assert len(decl) == 1, "INTEGRATION.md holds one Rust block with the extern declarations"
    return decl[0]


def _norm_rust_type(t):
    return " ".join(t.replace("*", " *").replace("* ", "*").split()).replace("* ", "*")


def rust_decls(src=None):
    src = rust_block() if src is None else src
    code = re.sub(r"//[^\n]*", "", src)
    structs = {}
    for name, body in re.findall(r"#\[repr\(C\)\]\s*pub struct (\w+)\s*\{(.*?)\}", code, flags=re.S):
        fields = []
        for f in body.split(","):
            f = " ".join(f.split())
            if not f:
                continue
            m = re.match(r"^(?:pub\s+)?(\w+)\s*:\s*(.+)$", f)
            assert m, f
            fields.append((m.group(1), _norm_rust_type(m.group(2))))
        structs[name] = fields
    funcs = {}
    for name, params, ret in re.findall(r"pub fn (pkv_\w+)\s*\((.*?)\)\s*(?:->\s*([^;]+))?;", code,
                                        flags=re.S):
        ps = []
        params = " ".join(params.split())
        for p in [x.strip() for x in params.split(",") if x.strip()]:
            m = re.match(r"^(\w+)\s*:\s*(.+)$", p)
            assert m, p
            ps.append(_norm_rust_type(m.group(2)))
        funcs[name] = (ps, None if ret is None else _norm_rust_type(ret))
    consts = {k: int(v) for k, v in re.findall(r"pub const (PKV_\w+)\s*:\s*c_int\s*=\s*(\d+)", code)}
    return structs, funcs, consts


def _compare(rust, header):
    """Differences between the Rust declarations and the header, as strings."""
    rs, rf, rc = rust
    hs, hf, he = header
    bad = []
    for name, fields in rs.items():
        if fields and name not in hs:
            # opaque handles are `{ _p: [u8; 0] }` and have no C definition
            if fields != [("_p", "[u8; 0]")]:
                bad.append(f"struct {name} has no C counterpart")
            continue
        if name in hs and [(f, _norm_rust_type(t)) for f, t in hs[name]] != fields:
            bad.append(f"struct {name}: rust {fields} != C {hs[name]}")
    for name in hs:
        if name not in rs:
            bad.append(f"struct {name} missing from the Rust block")
    for name, (ps, ret) in hf.items():
        if name not in rf:
            bad.append(f"fn {name} missing from the Rust block")
            continue
        rps, rret = rf[name]
        cps = [_norm_rust_type(p) for p in ps]
        cret = None if ret is None else _norm_rust_type(ret)
        if rps != cps:
            bad.append(f"fn {name}: rust params {rps} != C {cps}")
        if rret != cret:
            bad.append(f"fn {name}: rust returns {rret} != C {cret}")
    for name in rf:
        if name not in hf:
            bad.append(f"fn {name} not in the header")
    for k, v in rc.items():
        if he.get(k) != v:
            bad.append(f"const {k} = {v}, header has {he.get(k)}")
    return bad


def test_header_parser_reads_every_function():
    _, funcs, enums = header_decls()
    text = _strip_c(open(os.path.join(ROOT, "include", "pkv.h")).read())
    assert set(funcs) == set(re.findall(r"\b(pkv_[a-z0-9_]+)\s*\(", text))
    assert enums["PKV_ERR_LAYERS"] == 6 and enums["PKV_QUANT_Q4K"] == 4


@pytest.mark.parametrize("decl,rust", [
    ("const float *q", "*const f32"),
    ("float *out", "*mut f32"),
    ("pkv_cache *const *caches", "*const *mut PkvCache"),
    ("const void *const *src", "*const *const c_void"),
    ("void *const *dst", "*const *mut c_void"),
    ("pkv_cache **out", "*mut *mut PkvCache"),
    ("const void **k_bytes", "*mut *const c_void"),
    ("const int64_t kv_strides[3]", "*const i64"),
    ("int64_t strides[4]", "*mut i64"),
    ("pkv_stream stream", "*mut c_void"),
    ("size_t ssm_cap", "usize"),
    ("const pkv_layer_target *targets", "*const PkvLayerTarget"),
])
def test_c_type_mapping(decl, rust):
    assert c_to_rust(decl)[0] == rust


def test_rust_binding_matches_header():
    bad = _compare(rust_decls(), header_decls())
    assert not bad, "\n".join(bad)


def test_drift_is_detected():
    """The comparison fails on a binding that lost the restore targets' capacity fields
    (the 40-byte PkvLayerTarget against the C struct's 64 bytes), that swaps two
    parameters, or that drops a function."""
    src = rust_block()
    cut = re.sub(r"\n\s*pub ssm_cap: usize,[^\n]*\n\s*pub conv_cap: usize,[^\n]*\n\s*pub gate_cap: usize,[^\n]*",
                 "", src)
    assert cut != src
    assert any("PkvLayerTarget" in b for b in _compare(rust_decls(cut), header_decls()))
    swapped = src.replace("k: *const f32, v: *const f32, n: i64, offset: i64",
                          "k: *const f32, v: *const f32, n: c_int, offset: i64", 1)
    assert swapped != src
    assert any("pkv_append" in b for b in _compare(rust_decls(swapped), header_decls()))
    dropped = re.sub(r"\n\s*pub fn pkv_clear\([^;]*;", "", src)
    assert any("pkv_clear" in b for b in _compare(rust_decls(dropped), header_decls()))
