"""The Rust `-sys` declarations that the integration guide gives a maintainer agree
with include/thrml_hip.h: every declared C function appears in the Rust
extern block with the same parameter count, and every descriptor struct has
the same fields in the same order (a mismatch would corrupt every call made
through that binding).  CPU only: text comparison."""
import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _split_params(s):
    s = s.strip()
    if not s or s == "void":
        return []
    return [p.strip() for p in s.split(",") if p.strip()]


def _c_header():
    src = open(os.path.join(ROOT, "include", "thrml_hip.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    src = re.sub(r"//[^\n]*", "", src)
    funcs = {}
    for m in re.finditer(r"\b(thrml_[a-z0-9_]+)\s*\(([^()]*)\)\s*;", src):
        funcs[m.group(1)] = _split_params(m.group(2))
    structs = {}
    for m in re.finditer(r"typedef\s+struct\s*\{(.*?)\}\s*(thrml_[a-z0-9_]+)\s*;", src, flags=re.S):
        fields = []
        for decl in m.group(1).split(";"):
            decl = decl.strip()
            if not decl:
                continue
            # "uint32_t n_visible, n_hidden" or "const float *biases"
            head, *rest = decl.split(",")
            names = [re.findall(r"([A-Za-z_][A-Za-z0-9_]*)\s*(?:\[[^\]]*\])?$", head.strip())[0]]
            names += [r.strip().lstrip("*").strip() for r in rest]
            fields += names
        structs[m.group(2)] = fields
    return funcs, structs


def _rust_block():
    doc = open(os.path.join(ROOT, "INTEGRATION.md")).read()
    blocks = re.findall(r"```rust\n(.*?)```", doc, flags=re.S)
    assert blocks, "the integration guide has no rust block"
    src = re.sub(r"//[^\n]*", "", "\n".join(blocks))
    funcs = {}
    for m in re.finditer(r"pub fn (thrml_[a-z0-9_]+)\s*\(([^()]*)\)", src):
        funcs[m.group(1)] = _split_params(m.group(2))
    structs = {}
    for m in re.finditer(r"pub struct (thrml_[a-z0-9_]+)\s*\{(.*?)\}", src, flags=re.S):
        structs[m.group(1)] = re.findall(r"pub\s+([a-z_0-9]+)\s*:", m.group(2))
    return funcs, structs


def test_rust_extern_block_matches_header_functions():
    cf, _ = _c_header()
    rf, _ = _rust_block()
    assert len(cf) >= 30
    missing = sorted(set(cf) - set(rf))
    assert not missing, f"declared in the header, absent from the integration guide: {missing}"
    extra = sorted(set(rf) - set(cf))
    assert not extra, f"in the integration guide, not in the header: {extra}"
    bad = {n: (len(cf[n]), len(rf[n])) for n in cf if len(cf[n]) != len(rf[n])}
    assert not bad, f"parameter counts (header, rust) differ: {bad}"


def test_rust_structs_match_header_structs():
    _, cs = _c_header()
    _, rs = _rust_block()
    assert cs, "no descriptor structs parsed from the header"
    for name, fields in cs.items():
        assert name in rs, f"struct {name} missing from the integration guide"
        assert rs[name] == fields, f"{name}: header {fields} vs rust {rs[name]}"
