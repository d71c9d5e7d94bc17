"""The Rust FFI crate (crates/rtensor-hip) declares exactly the C ABI of
include/rtensor_hip.h: the same entry points with the same parameter and
return types, the same enum values and the same config struct.  No Rust
toolchain is needed: both files are parsed as text, and each C type is
translated to the Rust type that has its ABI."""
import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "rtensor_hip.h")
CRATE = os.path.join(ROOT, "crates", "rtensor-hip")
FFI = os.path.join(CRATE, "src", "ffi.rs")

# C scalar -> Rust scalar.  Enums are int-sized (they are passed as c_int).
SCALAR = {
    "int": "c_int", "size_t": "usize", "float": "f32", "double": "f64", "char": "c_char", "void": "c_void",
    "uint64_t": "u64", "rt_dtype": "c_int", "rt_layout": "c_int", "rt_epilogue": "c_int",
    "rt_unary_op": "c_int", "rt_binary_op": "c_int", "rt_loss_kind": "c_int", "rt_status": "c_int",
    "rt_ctx": "RtCtx", "rt_buf": "RtBuf", "rt_mlp": "RtMlp", "rt_mlp_config": "RtMlpConfig",
}


def c_to_rust(ctype: str) -> str:
    """`const float* const*` -> `*const *const f32`: each `*` makes a pointer
    whose Rust mutability is the const-ness of what it points to, and a
    `const` after a `*` qualifies the pointer that `*` made."""
    parts = ctype.replace("*", " * ").split()
    words = [p for p in parts if p not in ("const", "*")]
    assert len(words) == 1, ctype
    rust = SCALAR[words[0]]
    if "*" not in parts:
        return rust
    i = parts.index("*")
    pointee_const = "const" in parts[:i]  # `const T*` / `T const*`
    while i < len(parts):
        assert parts[i] == "*", ctype
        rust = ("*const " if pointee_const else "*mut ") + rust
        pointee_const = i + 1 < len(parts) and parts[i + 1] == "const"
        i += 2 if pointee_const else 1
    return rust


def _strip_c_comments(text):
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return re.sub(r"//[^\n]*", "", text)


def header_functions():
    text = _strip_c_comments(open(HEADER).read())
    out = {}
    for m in re.finditer(r"^([A-Za-z_][\w\s\*]*?)\b(rt_[a-z0-9_]+)\s*\(([^)]*)\)\s*;", text, flags=re.M):
        ret, name, args = m.group(1).strip(), m.group(2), m.group(3)
        params = []
        for a in [x.strip() for x in args.split(",") if x.strip()]:
            pm = re.match(r"^(.*?)([A-Za-z_]\w*)$", a)
            params.append(c_to_rust(pm.group(1).strip()))
        out[name] = (c_to_rust(ret), params)
    return out


def rust_functions():
    text = open(FFI).read()
    block = re.search(r'extern\s+"C"\s*\{(.*)\n\}', text, flags=re.S).group(1)
    block = re.sub(r"//[^\n]*", "", block)
    out = {}
    for m in re.finditer(r"pub fn (rt_[a-z0-9_]+)\s*\(([^)]*)\)\s*(->\s*([^;]+))?;", block, flags=re.S):
        name, args, ret = m.group(1), m.group(2), (m.group(4) or "()").strip()
        params = []
        for a in [x.strip() for x in args.split(",") if x.strip()]:
            params.append(" ".join(a.split(":", 1)[1].split()))
        out[name] = (" ".join(ret.split()), params)
    return out


def test_c_to_rust_translation_rules():
    assert c_to_rust("int") == "c_int"
    assert c_to_rust("const char*") == "*const c_char"
    assert c_to_rust("rt_buf**") == "*mut *mut RtBuf"
    assert c_to_rust("const float* const*") == "*const *const f32"
    assert c_to_rust("float* const*") == "*const *mut f32"
    assert c_to_rust("rt_buf* const*") == "*const *mut RtBuf"
    assert c_to_rust("const rt_buf* const*") == "*const *const RtBuf"
    assert c_to_rust("const rt_mlp_config*") == "*const RtMlpConfig"


def test_crate_files_exist():
    for f in ("Cargo.toml", "build.rs", os.path.join("src", "ffi.rs"), os.path.join("src", "lib.rs")):
        assert os.path.isfile(os.path.join(CRATE, f)), f
    cargo = open(os.path.join(CRATE, "Cargo.toml")).read()
    assert 'links = "rtensor_hip"' in cargo
    assert "rustc-link-lib=dylib=rtensor_hip" in open(os.path.join(CRATE, "build.rs")).read()


def test_extern_block_matches_header_exactly():
    h, r = header_functions(), rust_functions()
    assert len(h) >= 60
    assert sorted(h) == sorted(r), (sorted(set(h) - set(r)), sorted(set(r) - set(h)))
    for name in h:
        assert h[name] == r[name], (name, h[name], r[name])
    # the two entry points an earlier written-out block had left out
    assert "rt_mlp_activation" in r and "rt_mlp_delta" in r


def test_enum_constants_match_header():
    text = _strip_c_comments(open(HEADER).read())
    want = {k: int(v) for k, v in re.findall(r"\b(RT_[A-Z0-9_]+)\s*=\s*(\d+)", text)}
    got = {k: int(v) for k, v in re.findall(r"pub const (RT_[A-Z0-9_]+): c_int = (\d+);", open(FFI).read())}
    assert want and want == got


def test_config_struct_fields_match_header():
    text = _strip_c_comments(open(HEADER).read())
    body = re.search(r"typedef struct \{(.*?)\}\s*rt_mlp_config;", text, flags=re.S).group(1)
    c_fields = [(n, c_to_rust(t)) for t, n in re.findall(r"(\w+)\s+(\w+)\s*;", body)]
    rs = re.search(r"pub struct RtMlpConfig \{(.*?)\}", open(FFI).read(), flags=re.S).group(1)
    r_fields = re.findall(r"pub (\w+): (\w+),", rs)
    assert c_fields == r_fields


def test_safe_wrapper_calls_only_declared_entry_points():
    lib = open(os.path.join(CRATE, "src", "lib.rs")).read()
    used = set(re.findall(r"ffi::(rt_[a-z0-9_]+)", lib))
    assert used <= set(header_functions())
    # the rtensor::gpu surface the wrapper mirrors (mod.rs:263-564, 1341-1561, 1672)
    for fn in ("new", "info", "zeros", "upload", "download", "sync", "from_params", "step", "forward_only",
               "logits", "last_loss", "weights", "grads", "batch_size", "dispatches_por_passo", "upload_labels"):
        assert re.search(rf"pub fn {fn}\b", lib), fn
