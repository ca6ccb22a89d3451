"""The Rust crate (ferrum-cpu_amd/rust/ferrum_hip) against the C header, on
the CPU: no Rust toolchain exists on this image, so its FFI block is checked
here -- one declaration per entry point of include/ferrum_hip.h with the same
parameter count and C-compatible types, and the same constants -- and its
safe wrappers are checked to hold the context lock across every foreign call."""
import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "ferrum_hip.h")
CRATE = os.path.join(ROOT, "ferrum-cpu_amd", "rust", "ferrum_hip")

C_TO_RUST = {"int": "c_int", "long": "c_long", "void": "c_void", "char": "c_char", "size_t": "usize",
             "uint32_t": "u32", "uint64_t": "u64", "int32_t": "i32", "int8_t": "i8", "uint8_t": "u8", "float": "f32",
             "double": "f64"}


def header_decls():
    s = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    out = {}
    for ret, name, args in re.findall(r"\n\s*((?:const\s+)?[a-zA-Z_][\w\s\*]*?\**)\s*\b(fh_\w+)\s*\(([^;{]*?)\)\s*;", s):
        params = [] if args.strip() == "void" else [" ".join(a.split()) for a in args.split(",")]
        out[name] = (" ".join(ret.split()), params)
    return out


def rust_type(c):
    c = " ".join(c.split())
    const = c.startswith("const ")
    if const:
        c = c[6:]
    stars, t = c.count("*"), c.replace("*", "").strip()
    r = C_TO_RUST.get(t, t)
    if stars == 0:
        return r
    out = ("*const " if const else "*mut ") + r
    for _ in range(stars - 1):
        out = "*mut " + out
    return out


def crate_decls():
    s = open(os.path.join(CRATE, "src", "lib.rs")).read()
    block = s[s.index('extern "C" {'):]
    block = block[:block.index("\n    }\n")]
    out = {}
    for name, params, ret in re.findall(r"pub fn (fh_\w+)\((.*?)\)(?:\s*->\s*([^;]+))?;", block):
        ps = [p.split(":", 1)[1].strip() for p in params.split(",") if p.strip()]
        out[name] = (ret.strip() if ret else "c_void", ps)
    return out


def test_every_header_entry_point_is_declared_with_its_types():
    h, r = header_decls(), crate_decls()
    assert set(h) == set(r), (sorted(set(h) - set(r)), sorted(set(r) - set(h)))
    for name, (ret, params) in h.items():
        rret, rparams = r[name]
        assert rust_type(ret) == rret, (name, ret, rret)
        assert len(params) == len(rparams), name
        for p, rp in zip(params, rparams):
            ctype = re.match(r"(.*?)\w+$", p).group(1)
            assert rust_type(ctype) == rp, (name, p, rp)


def test_constants_match_the_header():
    h = open(HEADER).read()
    s = open(os.path.join(CRATE, "src", "lib.rs")).read()
    consts = dict(re.findall(r"pub const (FH_\w+): c_int = (\d+);", s))
    assert len(consts) >= 20
    for name, value in consts.items():
        m = re.search(rf"\b{name}\s*=\s*(\d+)", h)
        assert m and m.group(1) == value, name


def test_struct_layouts_follow_the_header():
    s = open(os.path.join(CRATE, "src", "lib.rs")).read()
    h = open(HEADER).read()
    sp = re.search(r"pub struct fh_sampling_params \{(.*?)\}", s, re.S).group(1)
    assert re.findall(r"pub (\w+):", sp) == ["temperature", "top_k", "top_p", "repetition_penalty"]
    hb = re.search(r"typedef struct \{([^{}]*?)\} fh_gpt2_block;", h, re.S).group(1)
    hb = re.sub(r"/\*.*?\*/", "", hb, flags=re.S)
    names = re.findall(r"\*\s*(\w+)", hb)
    rb = re.search(r"pub struct fh_gpt2_block \{(.*?)\}", s, re.S).group(1)
    assert re.findall(r"pub (\w+):", rb) == names


def test_safe_calls_hold_the_context_lock_across_the_foreign_call():
    """No `*self.ctx.lock()...` copy that drops the guard before the call: the
    only lock sites bind the guard to a local that outlives the call."""
    s = open(os.path.join(CRATE, "src", "lib.rs")).read()
    assert "*self.ctx.lock()" not in s
    lock_sites = [m.start() for m in re.finditer(r"self\.lock\(\)", s)]
    assert len(lock_sites) == 2  # with_raw and call
    for i in lock_sites:
        body = s[i:s.index("\n    }\n", i)]
        assert body.startswith("self.lock();") and "let c = guard.0;" in body and "drop(guard);" in body
        assert body.index("f(c)") < body.index("drop(guard)")
    # every foreign call in a safe wrapper goes through call() / with_raw()
    # (fh_ctx_destroy runs in Drop, with exclusive access)
    for m in re.finditer(r"unsafe \{ sys::fh_(\w+)\(c[,)]", s):
        if m.group(1) == "ctx_destroy":
            continue
        pre = s[max(0, m.start() - 200):m.start()]
        assert "call(|c|" in pre or "with_raw" in pre, m.group(1)


def test_crate_files_exist():
    for f in ("Cargo.toml", "build.rs", os.path.join("src", "lib.rs")):
        assert os.path.isfile(os.path.join(CRATE, f)), f
    toml = open(os.path.join(CRATE, "Cargo.toml")).read()
    assert 'name = "ferrum_hip"' in toml and 'links = "ferrum_hip"' in toml
