"""The Rust tier (rust/hip_tier/ffi.rs) binds exactly the C ABI the header
declares: every `extern "C"` function has the header's name, arity, argument
types (pointer constness, integer and float widths) and return type, and every
#[repr(C)] struct has the header struct's fields in the same order and types.
No cargo is in the image, so this parse is the check that the binding a
wave-engine maintainer adds (src/hip_tier beside src/cpu, src/wgpu_tier,
src/candle_tier; selected by --hip, src/cli.rs:208-210) matches the library."""
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
RUST = ROOT / "rust" / "hip_tier"

C_TO_RUST = {
    "float": "f32", "double": "f64", "int32_t": "i32", "int64_t": "i64", "uint64_t": "u64",
    "size_t": "usize", "int": "c_int", "char": "c_char", "void": "c_void",
    "wha_layout": "WhaLayout", "wha_wave_shape": "WhaWaveShape", "wha_wave_weights": "WhaWaveWeights",
    "wha_wave_cache": "WhaWaveCache", "wha_wave_grads": "WhaWaveGrads", "wha_wave_kv_cache": "WhaWaveKvCache",
}


def _strip_c_comments(text):
    return re.sub(r"/\*.*?\*/", "", re.sub(r"//[^\n]*", "", text, flags=re.S), flags=re.S)


def c_type(decl):
    """'const float* q' -> '*const f32'; 'size_t' -> 'usize' (name optional)."""
    decl = decl.strip()
    stars = decl.count("*")
    words = re.findall(r"[A-Za-z_]\w*", decl.replace("*", " * "))
    const = "const" in words
    words = [w for w in words if w not in ("const", "struct")]
    base = words[0]
    if base not in C_TO_RUST:
        raise AssertionError(f"unmapped C type in {decl!r}")
    t = C_TO_RUST[base]
    if stars == 0:
        return t
    assert stars == 1, decl
    return ("*const " if const else "*mut ") + t


def header_functions():
    text = _strip_c_comments("".join(p.read_text() for p in sorted((ROOT / "include").glob("*.h"))))
    out = {}
    for m in re.finditer(r"([A-Za-z_][\w\s\*]*?)\b(wha_\w+)\s*\(([^)]*)\)\s*;", text, flags=re.S):
        ret, name, params = m.group(1), m.group(2), m.group(3).strip()
        args = [] if params in ("", "void") else [c_type(p) for p in params.split(",")]
        r = c_type(ret)
        out[name] = (args, None if r == "c_void" else r)
    return out


def header_structs():
    text = _strip_c_comments("".join(p.read_text() for p in sorted((ROOT / "include").glob("*.h"))))
    out = {}
    for m in re.finditer(r"typedef\s+struct\s+\w+\s*\{(.*?)\}\s*(\w+)\s*;", text, flags=re.S):
        fields = []
        for stmt in m.group(1).split(";"):
            stmt = stmt.strip()
            if not stmt:
                continue
            # 'int32_t B, H, T, D' or 'const float* harmonic_raw'
            first, *rest = [s.strip() for s in stmt.split(",")]
            tm = re.match(r"(.*?)(\w+)$", first)
            base = tm.group(1)
            fields.append(c_type(base))
            base_no_star = base.replace("*", "")
            for _ in rest:
                fields.append(c_type(base_no_star) if "*" not in base else c_type(base))
        out[C_TO_RUST[m.group(2)]] = fields
    return out


def _rust_text():
    return re.sub(r"//[^\n]*", "", (RUST / "ffi.rs").read_text())


def rust_functions():
    text = _rust_text()
    block = re.search(r'extern\s+"C"\s*\{(.*)\n\}', text, flags=re.S).group(1)
    out = {}
    for m in re.finditer(r"pub fn (\w+)\s*\(([^)]*)\)\s*(->\s*([^;]+))?;", block, flags=re.S):
        name, params, ret = m.group(1), m.group(2), m.group(4)
        args = []
        for p in (x.strip() for x in params.split(",")):
            if p:
                args.append(" ".join(p.split(":", 1)[1].split()))
        out[name] = (args, " ".join(ret.split()) if ret else None)
    return out


def rust_structs():
    text = _rust_text()
    out = {}
    for m in re.finditer(r"#\[repr\(C\)\]\s*(?:#\[derive\([^)]*\)\]\s*)?pub struct (\w+)\s*\{(.*?)\}", text,
                         flags=re.S):
        fields = [" ".join(f.split(":", 1)[1].split()) for f in m.group(2).split(",") if f.strip()]
        out[m.group(1)] = fields
    return out


def test_parsers_see_the_whole_abi():
    hf, rf = header_functions(), rust_functions()
    assert len(hf) >= 30 and "wha_attn_fwd" in hf and "wha_timing_read" in hf
    assert hf["wha_attn_fwd"] == (["*const f32"] * 3 + ["*mut f32"] * 2 + ["*const WhaLayout", "f32", "*mut c_void"],
                                  "c_int")
    assert hf["wha_last_error"] == ([], "*const c_char")
    assert len(rf) >= 30


def test_every_header_function_is_bound_with_matching_types():
    hf, rf = header_functions(), rust_functions()
    assert set(rf) == set(hf), (f"only in the header: {sorted(set(hf) - set(rf))}; "
                                f"only in ffi.rs: {sorted(set(rf) - set(hf))}")
    for name, (args, ret) in hf.items():
        rargs, rret = rf[name]
        assert len(rargs) == len(args), f"{name}: arity {len(rargs)} in ffi.rs, {len(args)} in the header"
        for i, (a, b) in enumerate(zip(args, rargs)):
            assert a == b, f"{name} argument {i}: header {a}, ffi.rs {b}"
        assert ret == rret, f"{name} return: header {ret}, ffi.rs {rret}"


def test_repr_c_structs_match_the_header():
    hs, rs = header_structs(), rust_structs()
    assert set(hs) == set(rs), (sorted(hs), sorted(rs))
    for name, fields in hs.items():
        assert rs[name] == fields, f"{name}: header {fields}, ffi.rs {rs[name]}"


@pytest.mark.parametrize("path", ["mod.rs", "wave.rs", "kv.rs", "device.rs"])
def test_every_ffi_call_in_the_tier_is_declared(path):
    """Calls the other modules make through ffi:: name functions ffi.rs declares."""
    declared = set(rust_functions())
    text = (RUST / path).read_text()
    for m in re.finditer(r"ffi::(wha_\w+)\s*\(", text):
        assert m.group(1) in declared, f"{path} calls undeclared {m.group(1)}"


def test_build_rs_links_the_library():
    text = (ROOT / "rust" / "build.rs").read_text()
    assert "CARGO_FEATURE_HIP" in text and "rustc-link-lib=dylib=wave_hip_attn" in text
