"""The committed Zig binding (integration/zig/src/gpu/hip.zig) against the C
header it binds (include/tomoul_hip.h): the same set of functions, and for
each one the same arity, return type, integer widths and pointer constness.
There is no Zig toolchain in this image, so this parse is the check a Zig
compile would otherwise make at the call boundary.  CPU only."""
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "tomoul_hip.h")
ZIG = os.path.join(ROOT, "integration", "zig", "src", "gpu", "hip.zig")

# C scalar -> Zig scalar
SCALARS = {"int": "c_int", "int64_t": "i64", "uint64_t": "u64", "size_t": "usize", "float": "f32", "void": "void"}
# pointee C type -> Zig element type
ELEMS = {"float": "f32", "int8_t": "i8", "uint8_t": "u8", "uint16_t": "u16", "int64_t": "i64", "uint64_t": "u64",
         "int": "c_int", "char": "u8", "void": "anyopaque"}
HANDLES = {"tml_prepared_t", "tml_tl_t"}


def _strip_comments(text):
    text = re.sub(r"/\*.*?\*/", " ", text, flags=re.S)
    return re.sub(r"//[^\n]*", " ", text)


def c_functions():
    text = _strip_comments(open(HEADER).read())
    out = {}
    for m in re.finditer(r"\b(const\s+char\s*\*|int64_t|int|void)\s*(tml_\w+)\s*\(([^)]*)\)\s*;", text):
        ret, name, params = m.group(1), m.group(2), m.group(3)
        ps = [] if params.strip() in ("", "void") else [p.strip() for p in params.split(",")]
        out[name] = (" ".join(ret.split()), ps)
    return out


def zig_functions():
    text = open(ZIG).read()
    out = {}
    for m in re.finditer(r'extern "c" fn (tml_\w+)\(([^)]*)\)\s*([^;]+);', text):
        name, params, ret = m.group(1), m.group(2), m.group(3).strip()
        ps = [] if not params.strip() else [p.split(":", 1)[1].strip() for p in params.split(",")]
        out[name] = (ret, ps)
    return out


def c_param_type(p):
    """'const float *A' -> ('const float', 1); 'int64_t M' -> ('int64_t', 0)."""
    p = re.sub(r"\b\w+$", "", p).strip()  # drop the parameter name
    stars = p.count("*")
    return " ".join(p.replace("*", " ").split()), stars


def zig_matches(ctype, stars, z):
    """Whether the Zig type z binds the C type (ctype with `stars` pointers)."""
    const = ctype.startswith("const ")
    base = ctype[6:] if const else ctype
    if stars == 0:
        if base in HANDLES:
            return z in ("Prepared", "TlFile")
        return SCALARS.get(base) == z
    if base in HANDLES:  # tml_prepared_t *out / tml_tl_t *out
        return stars == 1 and not const and z in ("*Prepared", "*TlFile")
    if stars != 1:
        return False
    z = z[1:] if z.startswith("?") else z  # nullable or not: same ABI
    zconst = re.search(r"\bconst\b", z) is not None
    elem = re.sub(r"^(\[\*(:0)?\]|\*)\s*(const\s+)?", "", z)
    if base == "char" and const:
        return z in ("[*:0]const u8",)
    if base == "void":
        return elem == "anyopaque" and z.startswith("*") and zconst == const
    return (z.startswith("[*]") or z.startswith("*")) and elem == ELEMS[base] and zconst == const


def c_return_matches(cret, zret):
    if cret == "const char *" or cret == "const char*":
        return zret in ("[*:0]const u8", "?[*:0]const u8")
    return SCALARS.get(cret) == zret


def test_every_header_function_is_bound():
    c, z = c_functions(), zig_functions()
    assert len(c) >= 39, sorted(c)
    assert set(c) == set(z), (sorted(set(c) - set(z)), sorted(set(z) - set(c)))


@pytest.mark.parametrize("name", sorted(c_functions()))
def test_signature_matches(name):
    cret, cps = c_functions()[name]
    zret, zps = zig_functions()[name]
    assert c_return_matches(" ".join(cret.replace("*", " *").split()), zret), (name, cret, zret)
    assert len(cps) == len(zps), (name, cps, zps)
    for cp, zp in zip(cps, zps):
        ctype, stars = c_param_type(cp)
        assert zig_matches(ctype, stars, zp), (name, cp, zp)


def test_checker_rejects_mismatches():
    # planted mistakes the parse must catch: a narrowed size, dropped const,
    # wrong element type, lost nullability of a handle out-pointer
    assert not zig_matches("int64_t", 0, "c_int")
    assert not zig_matches("const float", 1, "[*]f32")
    assert not zig_matches("float", 1, "[*]const f32")
    assert not zig_matches("const int8_t", 1, "[*]const u8")
    assert not zig_matches("const void", 1, "*anyopaque")
    assert not zig_matches("tml_prepared_t", 1, "*anyopaque")
    assert zig_matches("const float", 1, "?[*]const f32") and zig_matches("void", 1, "?*anyopaque")
