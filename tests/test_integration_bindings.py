"""The Rust bindings written out for maintainers agree with the C header.

The integration guide at the repository root holds the `src/sys.rs` a
maintainer would add to the reference (crates/rhizome-gdr-hip); no Rust
toolchain exists here to compile it.  This test parses both texts and checks,
declaration by declaration, what a `#[repr(C)]` binding depends on: every
constant's value, every struct's fields in order with their C types, and
every function's parameters and result.
"""
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "rhizome_gdr.h")
DOC = os.path.join(ROOT, "INTEGRATION.md")

# C type (const, base, pointer depth) -> Rust type in sys.rs
SCALARS = {"int32_t": "i32", "uint32_t": "u32", "int64_t": "i64", "uint64_t": "u64", "size_t": "usize", "float": "f32",
           "double": "f64", "rhz_status": "i32"}
POINTEES = {"void": "c_void", "char": "c_char", "int32_t": "i32", "uint32_t": "u32", "float": "f32", "size_t": "usize"}


def c_to_rust(ctype):
    t = ctype.strip()
    const = t.startswith("const ")
    if const:
        t = t[len("const "):].strip()
    ptr = t.endswith("*")
    base = t.rstrip("*").strip()
    if not ptr:
        assert not const, ctype
        if base.startswith("rhz_") and base.endswith("_args"):
            return base  # a struct held by value
        return SCALARS[base]
    inner = POINTEES.get(base, base)  # struct pointers keep the struct's name
    return ("*const " if const else "*mut ") + inner


def strip_c_comments(text):
    return re.sub(r"/\*.*?\*/", "", text, flags=re.S)


def parse_header():
    text = strip_c_comments(open(HEADER).read())
    consts = {}
    for body in re.findall(r"typedef enum \w+ \{(.*?)\}", text, flags=re.S):
        for name, value in re.findall(r"(RHZ_\w+)\s*=\s*(\d+)", body):
            consts[name] = int(value)
    for name, value in re.findall(r"#define (RHZ_\w+) (\d+)", text):
        consts[name] = int(value)
    structs = {}
    for name, body in re.findall(r"typedef struct (\w+) \{(.*?)\} \1;", text, flags=re.S):
        fields = []
        for decl in body.split(";"):
            decl = " ".join(decl.split())
            if not decl:
                continue
            m = re.fullmatch(r"(.+?)\s*(\w+)", decl)
            fields.append((m.group(2), c_to_rust(m.group(1))))
        structs[name] = fields
    funcs = {}
    for ret, name, params in re.findall(r"(rhz_status|int32_t|const char\*)\s+(rhz_\w+)\(([^)]*)\);", text):
        ps = []
        for p in params.split(","):
            p = " ".join(p.split())
            if p in ("void", ""):
                continue
            m = re.fullmatch(r"(.+?)\s*(\w+)", p)
            ps.append((m.group(2), c_to_rust(m.group(1))))
        funcs[name] = (ps, c_to_rust(ret))
    return consts, structs, funcs


def sys_rs_block():
    doc = open(DOC).read()
    i = doc.index("### src/sys.rs")
    start = doc.index("```rust", i) + len("```rust")
    return doc[start:doc.index("```", start)]


def parse_rust():
    text = re.sub(r"//[^\n]*", "", sys_rs_block())
    consts = {n: int(v) for n, v in re.findall(r"pub const (RHZ_\w+): i32 = (\d+);", text)}
    structs = {}
    for name, body in re.findall(r"#\[repr\(C\)\]\s*pub struct (\w+) \{(.*?)\}", text, flags=re.S):
        fields = []
        for f in body.split(","):
            f = " ".join(f.split())
            if f:
                m = re.fullmatch(r"pub (\w+): (.+)", f)
                fields.append((m.group(1), m.group(2)))
        structs[name] = fields
    funcs = {}
    for name, params, ret in re.findall(r"pub fn (rhz_\w+)\(([^)]*)\)\s*->\s*([^;]+);", text, flags=re.S):
        ps = []
        for p in params.split(","):
            p = " ".join(p.split())
            if p:
                m = re.fullmatch(r"(\w+): (.+)", p)
                ps.append((m.group(1), m.group(2)))
        funcs[name] = (ps, ret.strip())
    return consts, structs, funcs


@pytest.fixture(scope="module")
def both():
    return parse_header(), parse_rust()


def test_header_parses(both):
    (consts, structs, funcs), _ = both
    # guards the parser itself: everything the header declares was found
    assert len(structs) == 8 and len(funcs) == 19 and consts["RHZ_ERR_HIP"] == 4


def test_every_constant(both):
    (cc, _, _), (rc, _, _) = both
    assert rc == cc


def test_every_struct_field_in_order(both):
    (_, cs, _), (_, rs, _) = both
    assert sorted(rs) == sorted(cs)
    for name in cs:
        assert rs[name] == cs[name], name


def test_every_function_signature(both):
    (_, _, cf), (_, _, rf) = both
    assert sorted(rf) == sorted(cf)
    for name, (params, ret) in cf.items():
        rparams, rret = rf[name]
        assert [t for _, t in rparams] == [t for _, t in params], name
        assert rret == ret, name



# ---- the safe drop-ins (src/lib.rs) behave as the reference and the tested
# C++ layer do (rhizome_amd/host/rhizome_delta.cpp)

def dropin_rust():
    doc = open(DOC).read()
    i = doc.index("### src/lib.rs: the drop-ins")
    end = doc.index("## 3.", i)
    blocks = re.findall(r"```rust\n(.*?)```", doc[i:end], flags=re.S)
    assert len(blocks) == 2
    return "\n".join(blocks)


def rust_fn(text, name):
    """The body of `pub fn name` up to its matching closing brace."""
    i = text.index(f"pub fn {name}(")
    j = text.index("{", text.index(")", i))
    depth = 0
    for k in range(j, len(text)):
        depth += {"{": 1, "}": -1}.get(text[k], 0)
        if depth == 0:
            return text[j:k + 1]
    raise AssertionError(f"unbalanced braces in {name}")


def test_dropins_braces_balance():
    text = re.sub(r"//[^\n]*", "", dropin_rust())
    assert text.count("{") == text.count("}")
    assert text.count("(") == text.count(")")


def test_empty_sequence_returns_init():
    # delta.rs:135,153: with T = 0 the loop never runs and init comes back
    body = re.sub(r"//[^\n]*", "", rust_fn(dropin_rust(), "try_gated_delta_sequential"))
    m = re.search(r"if t == 0 \{\s*return Ok\(\(Vec::new\(\), init\.clone\(\)\)\);\s*\}", body)
    assert m, "T = 0 must return init unchanged"
    # the early return comes before any device work
    assert m.start() < body.index("DeviceBuf")
    assert "vec![0.0; d * d]" not in body


def test_lengths_checked_as_the_slicing_needs():
    text = re.sub(r"//[^\n]*", "", dropin_rust())
    # the reference never calls is_consistent (delta.rs:133-230)
    assert "is_consistent" not in text
    req = rust_fn(text, "require_inputs") if "pub fn require_inputs(" in text else None
    if req is None:
        i = text.index("fn require_inputs(")
        req = text[i:text.index("\n}\n", i)]
    for cond in ("inp.q.len() < t * d", "inp.k.len() < t * d", "inp.v.len() < t * d",
                 "inp.beta.len() < t", "inp.segment.len() < t"):
        assert cond in req, cond
    # every sequence-level drop-in uses it
    for fn in ("try_gated_delta_sequential", "gated_delta_multistep"):
        assert "require_inputs(" in rust_fn(text, fn), fn


def test_multistep_runs_in_windows():
    # one rhz_gdr_multistep call takes at most RHZ_MULTISTEP_MAX positions;
    # each window starts from the previous window's last snapshot
    body = re.sub(r"//[^\n]*", "", rust_fn(dropin_rust(), "gated_delta_multistep"))
    assert "sys::RHZ_MULTISTEP_MAX" in body
    assert re.search(r"while t0 < n \{", body)
    assert re.search(r"let m = window\.min\(n - t0\);", body)
    assert re.search(r"steps: m as i32", body)
    assert re.search(r"state: if t0 == 0 \{ f\(&s0, 0\) \} else \{ f\(&snaps, \(t0 - 1\) \* d \* d\) \}", body)
    assert re.search(r"states: f\(&snaps, t0 \* d \* d\)", body)
    assert "t0 += m;" in body
    # no path hands n > RHZ_MULTISTEP_MAX to the ABI in one call
    assert "steps: n as i32" not in body
