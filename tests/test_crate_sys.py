"""The Rust binding (crates/kiln-hip) matches include/kiln_hip.h: every
declared function is bound in src/sys.rs with the same parameter list (each
C type mapped to its Rust FFI type, in order) and return type, the structs
have the header's fields in order with the same types, and the constants
carry the header's values. No cargo is needed: the sources are parsed.

The reference binds mlx-c the same way, as raw `extern "C"` declarations
under safe wrappers (crates/kiln-mlx/src/sys.rs, ops.rs)."""
import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = open(os.path.join(ROOT, "include", "kiln_hip.h")).read()
SYS = open(os.path.join(ROOT, "crates", "kiln-hip", "src", "sys.rs")).read()
OPS = open(os.path.join(ROOT, "crates", "kiln-hip", "src", "ops.rs")).read()

# C parameter type -> Rust FFI type
C2RUST = {
    "kh_array*": "*mut kh_array",
    "const kh_array*": "*const kh_array",
    "kh_array* const*": "*const *mut kh_array",
    "const kh_array* const*": "*const *const kh_array",
    "bool": "bool",
    "kh_optional_int": "kh_optional_int",
    "const char*": "*const c_char",
    "char*": "*mut c_char",
    "kh_stream": "kh_stream",
    "int": "c_int",
    "int64_t": "i64",
    "size_t": "usize",
}
RET = {"int": "c_int", "const char*": "*const c_char", "size_t": "usize"}


def _strip_comments(s):
    return re.sub(r"/\*.*?\*/", " ", s, flags=re.S)


def header_functions():
    text = _strip_comments(HEADER)
    out = {}
    for m in re.finditer(r"^(int|const char\*|size_t)\s+(kh_\w+)\s*\(([^)]*)\)\s*;", text, re.M):
        ret, name, params = m.group(1), m.group(2), m.group(3)
        types = []
        for p in params.split(","):
            p = " ".join(p.split())
            if p in ("void", ""):
                continue
            t = re.sub(r"\s*\b\w+$", "", p)          # drop the parameter name
            t = t.replace(" *", "*").replace("* ", "*").replace("*const", "* const")
            types.append(t)
        out[name] = (ret, types)
    return out


def rust_functions():
    block = re.search(r'unsafe extern "C" \{(.*?)\n\}', SYS, re.S).group(1)
    out = {}
    for m in re.finditer(r"pub fn (kh_\w+)\((.*?)\)(?:\s*->\s*([^;]+))?;", block, re.S):
        name, params, ret = m.group(1), m.group(2), (m.group(3) or "").strip()
        types = [" ".join(p.split(":", 1)[1].split()) for p in params.split(",") if p.strip()]
        out[name] = (ret, types)
    return out


def test_every_header_function_is_bound_with_its_signature():
    hdr, rs = header_functions(), rust_functions()
    assert len(hdr) >= 17, sorted(hdr)
    assert set(hdr) == set(rs), (set(hdr) ^ set(rs))
    for name, (ret, types) in hdr.items():
        rret, rtypes = rs[name]
        assert RET[ret] == rret, (name, ret, rret)
        assert [C2RUST[t] for t in types] == rtypes, (name, types, rtypes)


def test_structs_match_field_for_field():
    text = _strip_comments(HEADER)
    arr = re.search(r"typedef struct kh_array \{(.*?)\} kh_array;", text, re.S).group(1)
    fields = [" ".join(f.split()) for f in arr.split(";") if f.strip()]
    assert fields == ["void* data", "int32_t dtype", "int32_t ndim", "int64_t shape[KH_MAX_NDIM]"]
    rs = re.search(r"pub struct kh_array \{(.*?)\}", SYS, re.S).group(1)
    rfields = [" ".join(f.split()) for f in rs.split(",") if f.strip()]
    assert rfields == ["pub data: *mut c_void", "pub dtype: i32", "pub ndim: i32", "pub shape: [i64; KH_MAX_NDIM]"]
    opt = re.search(r"typedef struct kh_optional_int \{(.*?)\} kh_optional_int;", text, re.S).group(1)
    assert [" ".join(f.split()) for f in opt.split(";") if f.strip()] == ["int32_t value", "bool has_value"]
    ro = re.search(r"pub struct kh_optional_int \{(.*?)\}", SYS, re.S).group(1)
    assert [" ".join(f.split()) for f in ro.split(",") if f.strip()] == ["pub value: i32", "pub has_value: bool"]
    assert "#[repr(C)]\n#[derive(Clone, Copy, Debug)]\npub struct kh_array" in SYS
    assert re.search(r"#define KH_MAX_NDIM (\d+)", HEADER).group(1) == \
        re.search(r"pub const KH_MAX_NDIM: usize = (\d+);", SYS).group(1)


def test_constants_match():
    text = _strip_comments(HEADER)
    consts = dict((k, int(v)) for k, v in re.findall(r"\b(KH_[A-Z0-9_]+)\s*=\s*(\d+)", text))
    assert len(consts) >= 14 + 5 + 2
    for k, v in consts.items():
        m = re.search(rf"pub const {k}: \w+ = (\d+);", SYS)
        assert m and int(m.group(1)) == v, k


def test_safe_layer_wraps_the_path():
    """ops.rs wraps every entry point of the path (the diagnostics and the
    allocation-free variant are reached through sys directly)."""
    for name in header_functions():
        if name in ("kh_last_error", "kh_version", "kh_quantized_matmul_plan", "kh_noalloc_scratch_bytes",
                    "kh_quantized_matmul_noalloc", "kh_quantized_matmul_multi", "kh_quantized_gate_up"):
            continue
        assert f"sys::{name}(" in OPS, name
    for f in ("quantized_matmul", "gather_qmm", "dequantize", "take"):  # kiln_mlx::ops names
        assert re.search(rf"pub fn {f}\(", OPS), f
