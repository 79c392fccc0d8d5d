"""INTEGRATION.md's Rust binding block mirrors include/fwhip.h: every entry
point the header declares appears with the same number of arguments, and every
struct with the same fields in the same order (no compiler for the Rust side
here, so the text is checked)."""
import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _header():
    src = open(os.path.join(ROOT, "include", "fwhip.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return re.sub(r"^#.*$", "", src, flags=re.M)


def _rust():
    doc = open(os.path.join(ROOT, "INTEGRATION.md")).read()
    m = re.search(r"```rust\n(.*?)```", doc, re.S)
    assert m, "no rust block"
    return re.sub(r"//[^\n]*", "", m.group(1))


def _split_args(args):
    args = args.strip()
    if args in ("", "void"):
        return []
    return [a for a in args.split(",") if a.strip()]


def header_functions():
    out = {}
    for m in re.finditer(r"\b(fwhip_[a-z0-9_]+)\s*\(([^()]*)\)\s*;", _header()):
        out[m.group(1)] = len(_split_args(m.group(2)))
    return out


def rust_functions():
    out = {}
    for m in re.finditer(r"pub fn (fwhip_[a-z0-9_]+)\s*\(([^()]*)\)", _rust()):
        out[m.group(1)] = len(_split_args(m.group(2)))
    return out


def header_structs():
    out = {}
    for m in re.finditer(r"typedef struct (fwhip_[a-z0-9_]+)\s*\{(.*?)\}\s*\1\s*;", _header(), re.S):
        fields = []
        for decl in m.group(2).split(";"):
            decl = decl.strip()
            if not decl:
                continue
            # "const float *a, *b" / "int32_t family[N]" -> names in order
            first, *rest = decl.split(",")
            names = [re.sub(r"\[.*\]", "", first).split()[-1]] + [re.sub(r"\[.*\]", "", r).strip() for r in rest]
            fields += [n.lstrip("*") for n in names]
        out[m.group(1)] = fields
    return out


def rust_structs():
    out = {}
    for m in re.finditer(r"pub struct (fwhip_[a-z0-9_]+)\s*\{(.*?)\}", _rust(), re.S):
        out[m.group(1)] = re.findall(r"pub ([a-z0-9_]+)\s*:", m.group(2))
    return out


def test_every_entry_point_is_bound_with_its_arity():
    h, r = header_functions(), rust_functions()
    assert len(h) > 50
    missing = sorted(set(h) - set(r))
    assert not missing, missing
    wrong = {n: (h[n], r[n]) for n in h if h[n] != r[n]}
    assert not wrong, wrong


def test_every_struct_has_the_header_fields_in_order():
    h, r = header_structs(), rust_structs()
    assert "fwhip_dec_layer" in h and "fwhip_exec_record" in h
    for name, fields in h.items():
        assert name in r, name
        assert r[name] == fields, (name, fields, r[name])
