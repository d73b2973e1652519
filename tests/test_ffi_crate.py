"""The Rust binding crate (mivi-v4_amd/mivi-hip-sys) against include/mivi_hip.h
(CPU only; the image has no Rust toolchain to compile the crate): every
function the header declares is in the crate's extern block and nothing else
is, with the same number of parameters and the same parameter and return
types under the C-to-Rust type mapping."""
from __future__ import annotations

import os
import re

from conftest import ROOT

HEADER = os.path.join(ROOT, "include", "mivi_hip.h")
CRATE = os.path.join(ROOT, "mivi-v4_amd", "mivi-hip-sys")

C_TO_RUST = {
    "int32_t": "i32", "uint32_t": "u32", "uint64_t": "u64", "size_t": "usize", "float": "f32", "void": "()",
    "char": "c_char", "uint8_t": "u8", "mivi_error": "MiviError", "mivi_model": "MiviModel",
    "mivi_model_info": "MiviModelInfo", "mivi_prefix_cache": "MiviPrefixCache",
    "mivi_sampler_config": "MiviSamplerConfig",
}


def c_type_to_rust(t: str) -> str:
    t = " ".join(t.split())
    stars = t.count("*")
    base = t.replace("*", "").strip()
    const = base.startswith("const ")
    base = base.replace("const ", "").strip()
    rust = C_TO_RUST[base]
    if stars == 0:
        return rust
    if rust == "()":
        rust = "c_void"
    out = rust
    for i in range(stars):
        # the innermost pointer carries the const of the pointee
        q = "*const" if (const and i == 0) else "*mut"
        out = f"{q} {out}"
    return out


def header_functions():
    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    text = re.sub(r"#[^\n]*", "", text)
    out = {}
    for m in re.finditer(r"([A-Za-z_][\w\s\*]*?)\b((?:mivi_hip|mivi_synth)_\w+)\s*\(([^)]*)\)\s*;", text):
        ret, name, params = m.group(1).strip(), m.group(2), m.group(3).strip()
        plist = [] if params in ("", "void") else [p.strip() for p in params.split(",")]
        types = []
        for p in plist:
            p = " ".join(p.split())
            pm = re.match(r"(.*?[\s\*])(\w+)$", p)
            types.append(c_type_to_rust(pm.group(1)))
        out[name] = (c_type_to_rust(ret), types)
    return out


def crate_functions():
    text = open(os.path.join(CRATE, "src", "lib.rs")).read()
    text = re.sub(r"//[^\n]*", "", text)
    out = {}
    for m in re.finditer(r"pub fn ((?:mivi_hip|mivi_synth)_\w+)\s*\(([^)]*)\)\s*(->\s*([^;]+))?;", text, flags=re.S):
        name, params = m.group(1), m.group(2)
        ret = " ".join(m.group(4).split()) if m.group(4) else "()"
        types = []
        for p in [p for p in params.split(",") if p.strip()]:
            types.append(" ".join(p.split(":", 1)[1].split()))
        out[name] = (ret, types)
    return out


def test_type_mapping():
    assert c_type_to_rust("const float* ") == "*const f32"
    assert c_type_to_rust("mivi_model** ") == "*mut *mut MiviModel"
    assert c_type_to_rust("const mivi_model* ") == "*const MiviModel"
    assert c_type_to_rust("void* ") == "*mut c_void"


def test_crate_files_present():
    for f in ("Cargo.toml", "build.rs", os.path.join("src", "lib.rs")):
        assert os.path.exists(os.path.join(CRATE, f)), f
    toml = open(os.path.join(CRATE, "Cargo.toml")).read()
    assert 'name = "mivi-hip-sys"' in toml and 'links = "mivi_hip"' in toml


def test_extern_block_matches_header_symbol_for_symbol():
    h = header_functions()
    r = crate_functions()
    assert len(h) >= 45
    assert sorted(h) == sorted(r), (sorted(set(h) - set(r)), sorted(set(r) - set(h)))
    for name, (ret, types) in h.items():
        rret, rtypes = r[name]
        assert len(types) == len(rtypes), (name, types, rtypes)
        assert types == rtypes, (name, types, rtypes)
        assert ret == rret, (name, ret, rret)


def test_safe_wrappers_have_the_reference_signatures():
    # mivi_quant::quantized_matvec (lib.rs:75-82), quantized_matmul_rows
    # (lib.rs:136-151), dequantize_slice (lib.rs:35), try_matvec_* (q4_k_m.rs:217,
    # q6_k.rs:202, q8_0.rs:127)
    text = " ".join(open(os.path.join(CRATE, "src", "lib.rs")).read().split())
    for sig in (
        "pub fn quantized_matvec(out: &mut [f32], ggml_type: GgmlType, weights: &[u8], x: &[f32], n: usize, "
        "d: usize) -> Result<()>",
        "pub fn quantized_matmul_rows(out: &mut [f32], ggml_type: GgmlType, weights: &[u8], inputs: &[f32], "
        "batch: usize, rows: usize, cols: usize) -> Result<()>",
        "pub fn dequantize_slice(ggml_type: GgmlType, bytes: &[u8], out: &mut [f32]) -> Result<()>",
        "pub fn try_matvec_q4_k_m(out: &mut [f32], weights: &[u8], x: &[f32], n: usize, d: usize) -> Result<()>",
        "pub fn try_matvec_q6_k(out: &mut [f32], weights: &[u8], x: &[f32], n: usize, d: usize) -> Result<()>",
        "pub fn try_matvec_q8_0(out: &mut [f32], weights: &[u8], x: &[f32], n: usize, d: usize) -> Result<()>",
    ):
        assert sig in text, sig
    # the QuantError variants in the reference's declaration order (types.rs:5-15)
    i = [text.index(v) for v in ("UnsupportedType(u32)", "BufferTooSmall {", "DimensionMisaligned {",
                                  "ArithmeticOverflow,")]
    assert i == sorted(i)
