"""The Rust binding of the boundary (rust/lb-ternary-hip/src/ffi.rs, not
compiled here: no Rust toolchain) against include/lbt.h: every declared
function is bound once with the same parameter names and the Rust type each C
type maps to (pointer levels and constness included), and the #[repr(C)]
structs have the header's fields in the header's order and types."""
import re
from pathlib import Path

REPO = Path(__file__).resolve().parent.parent
HEADER = REPO / "include" / "lbt.h"
FFI = REPO / "rust" / "lb-ternary-hip" / "src" / "ffi.rs"

SCALAR = {"int": "c_int", "size_t": "usize", "float": "f32", "double": "f64", "char": "c_char", "void": "c_void",
          "uint8_t": "u8", "int8_t": "i8", "uint16_t": "u16", "int32_t": "i32", "uint32_t": "u32",
          "uint64_t": "u64", "int64_t": "i64"}


def rust_name(c: str) -> str:
    if c in SCALAR:
        return SCALAR[c]
    assert c.startswith("lbt_"), c
    special = {"lbt_q8head": "LbtQ8Head", "lbt_bf16": "LbtBf16"}
    return special.get(c, "".join(p.capitalize() for p in c.split("_")))


def c_type_to_rust(decl: str) -> str:
    """`const lbt_weight* const* ws` -> `*const *const LbtWeight` (name dropped)."""
    toks = re.findall(r"const|\*|\w+", decl)
    base_const = False
    if toks[0] == "const":
        base_const = True
        toks = toks[1:]
    base = toks[0]
    rest = toks[1:]
    if rest and re.fullmatch(r"\w+", rest[-1]) and rest[-1] != "const":
        rest = rest[:-1]  # parameter name
    t = rust_name(base)
    pointee_const = base_const
    i = 0
    while i < len(rest):
        assert rest[i] == "*", decl
        t = ("*const " if pointee_const else "*mut ") + t
        pointee_const = i + 1 < len(rest) and rest[i + 1] == "const"
        i += 2 if pointee_const else 1
    return t


def c_decls():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    text = re.sub(r"#.*", "", text)
    out = {}
    for m in re.finditer(r"^([\w\s\*]+?)\b(lbt_\w+)\s*\(([^)]*)\)\s*;", text, flags=re.M):
        ret, name, params = m.group(1).strip(), m.group(2), m.group(3).strip()
        plist = [] if params in ("", "void") else [p.strip() for p in params.split(",")]
        names = [re.findall(r"\w+", p)[-1] for p in plist]
        out[name] = (c_type_to_rust(ret + " r") if ret != "void" else None,
                     [(n, c_type_to_rust(p)) for n, p in zip(names, plist)])
    return out


def rust_decls():
    text = FFI.read_text()
    block = text[text.index('extern "C" {'):]
    block = re.sub(r"//.*", "", block)
    out = {}
    for m in re.finditer(r"pub fn (lbt_\w+)\s*\((.*?)\)\s*(->\s*([^;]+?))?\s*;", block, flags=re.S):
        name, params, ret = m.group(1), m.group(2), m.group(4)
        plist = [p.strip() for p in params.split(",") if p.strip()]
        args = []
        for p in plist:
            n, t = p.split(":", 1)
            args.append((n.strip(), " ".join(t.split())))
        assert name not in out, f"{name} bound twice"
        out[name] = (" ".join(ret.split()) if ret else None, args)
    return out


def c_structs():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    out = {}
    for m in re.finditer(r"typedef struct (lbt_\w+) \{(.*?)\} \w+;", text, flags=re.S):
        fields = []
        for f in m.group(2).split(";"):
            f = f.strip()
            if not f:
                continue
            arr = re.match(r"(\w+)\s+(\w+)\[(\d+)\]", f)
            if arr:
                fields.append((arr.group(2), f"[{rust_name(arr.group(1))}; {arr.group(3)}]"))
            else:
                t, n = f.split()
                fields.append((n, rust_name(t)))
        out[rust_name(m.group(1))] = fields
    return out


def rust_structs():
    text = FFI.read_text()
    out = {}
    for m in re.finditer(r"pub struct (\w+) \{(.*?)\}", text, flags=re.S):
        fields = re.findall(r"pub (\w+): ([^,\n]+),", m.group(2))
        if fields:
            out[m.group(1)] = [(n, " ".join(t.split())) for n, t in fields]
    return out


def test_every_function_bound_with_matching_types():
    c, r = c_decls(), rust_decls()
    assert len(c) > 70
    assert set(c) == set(r), (set(c) ^ set(r))
    for name, (cret, cargs) in c.items():
        rret, rargs = r[name]
        assert cret == rret, (name, cret, rret)
        assert cargs == rargs, (name, cargs, rargs)


def test_structs_match_header():
    c, r = c_structs(), rust_structs()
    assert set(c) == {"LbtSampleParams", "LbtConfig", "LbtProf"}
    for name, fields in c.items():
        assert r[name] == fields, (name, fields, r[name])


def test_status_codes_match_header():
    text = HEADER.read_text()
    rs = FFI.read_text()
    for name, val in re.findall(r"#define (LBT_\w+) \(?(-?\d+)\)?", text):
        assert re.search(rf"pub const {name}: c_int = {val};", rs), name


def test_mapping_examples():
    assert c_type_to_rust("const lbt_weight* const* ws") == "*const *const LbtWeight"
    assert c_type_to_rust("float* const* outs") == "*const *mut f32"
    assert c_type_to_rust("lbt_ctx** out") == "*mut *mut LbtCtx"
    assert c_type_to_rust("const char* r") == "*const c_char"


# ---- the `burn` facade: lb_model::BitNet's own signatures --------------------
# The reference's declarations (crates/lb-model/src/model.rs:149, :234, :305)
# and the calls lb-server / lb-run make (lb-server/src/main.rs:104-107,153,
# lb-model/src/bin/lb-run.rs:94-106), normalised: what the facade must accept.
REF_SIGS = {
    "load": "pub fn load(dir: &Path, device: &Device) -> Result<Self>",
    "new_cache": "pub fn new_cache(&self) -> KvCache",
    "forward": "pub fn forward(&self, tokens: &[u32], cache: &mut KvCache, all_logits: bool) -> Tensor<2>",
}
REF_MODEL = Path("/root/reference/crates/lb-model/src/model.rs")


def facade_sigs():
    text = (REPO / "rust" / "lb-ternary-hip" / "src" / "bitnet.rs").read_text()
    body = text[text.index("impl BitNet {"):]
    out = {}
    for m in re.finditer(r"(pub fn (\w+)\((.*?)\)\s*->\s*([^{]+?))\s*\{", body, flags=re.S):
        out[m.group(2)] = " ".join(m.group(1).split())
    return out


def norm(sig: str) -> str:
    # anyhow::Result and Result are the same type in lb-model (use anyhow::Result)
    return sig.replace("anyhow::Result", "Result")


def test_burn_facade_has_the_reference_signatures():
    got = facade_sigs()
    for name, sig in REF_SIGS.items():
        assert norm(got[name]) == sig, (name, got[name])
    text = (REPO / "rust" / "lb-ternary-hip" / "src" / "bitnet.rs").read_text()
    assert re.search(r"pub struct KvCache \{[^}]*pub len: usize,[^}]*pub cap: usize,", text, flags=re.S)


def test_reference_signatures_are_current():
    """REF_SIGS restates the reference's declarations (checked where the
    reference tree is present; it is not on the GPU box)."""
    if not REF_MODEL.exists():
        import pytest

        pytest.skip("reference tree not present")
    text = " ".join(REF_MODEL.read_text().split())
    for sig in REF_SIGS.values():
        assert sig in text, sig
