"""The Rust `-sys` binding that INTEGRATION.md specifies must match the C ABI it mirrors.

No Rust toolchain exists in this image, so the binding is checked as text: every
`#[repr(C)]` struct of INTEGRATION.md's Rust block is laid out by the C rules (field names,
types, offsets, total size) and compared with the same struct in include/nanocamelid_gpu.h
and with the ctypes structure in nanocamelid_amd/_ffi.py; every `extern "C"` function is
compared with the header's prototype (argument count, each argument's type and constness,
return type) and with the ctypes signature table; every `pub const` with the header's
`#define`.  A field added to the header and not to the document (the way a caller's struct
ends up smaller than what nc_model_get_config writes) fails here.
"""
import ctypes as C
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "nanocamelid_gpu.h")
DOC = os.path.join(ROOT, "INTEGRATION.md")

# scalar types: canonical name -> (size, alignment)
SCALARS = {"i8": 1, "u8": 1, "i16": 2, "u16": 2, "i32": 4, "u32": 4, "i64": 8, "u64": 8, "f32": 4, "f64": 8,
           "usize": 8, "char": 1, "void": 0}
C_NAMES = {"int8_t": "i8", "uint8_t": "u8", "int16_t": "i16", "uint16_t": "u16", "int32_t": "i32",
           "uint32_t": "u32", "int64_t": "i64", "uint64_t": "u64", "float": "f32", "double": "f64",
           "size_t": "usize", "int": "i32", "char": "char", "void": "void"}
RUST_NAMES = {"i8": "i8", "u8": "u8", "i16": "i16", "u16": "u16", "i32": "i32", "u32": "u32", "i64": "i64",
              "u64": "u64", "f32": "f32", "f64": "f64", "usize": "usize", "c_int": "i32", "c_char": "char",
              "c_void": "void"}
# functions of the header that the crate leaves out on purpose (INTEGRATION.md says why:
# benchmark-only entry points of the synthetic configs and debug hooks)
LEFT_OUT = {"nc_generate_speculative_oracle", "nc_synth_size", "nc_synth_write", "nc_uniform_prompt",
            "nc_oracle_draft", "nc_bench_matmul", "nc_session_kernel_timing", "nc_session_timing_enable",
            "nc_debug_expf", "nc_session_fill_kv", "nc_synth_kv_values", "nc_session_stage_timing",
            "nc_debug_temperature_paths", "nc_debug_pass_graphs"}


def _strip_c_comments(text):
    text = re.sub(r"/\*.*?\*/", " ", text, flags=re.S)
    return re.sub(r"//[^\n]*", " ", text)


def _rust_block():
    doc = open(DOC).read()
    blocks = re.findall(r"```rust\n(.*?)```", doc, flags=re.S)
    src = [b for b in blocks if 'extern "C"' in b]
    assert len(src) == 1, "INTEGRATION.md must hold exactly one Rust block with the extern \"C\" declarations"
    return re.sub(r"//[^\n]*", " ", src[0])


# ---------------------------------------------------------------- types
def _canon_c(ty):
    ty = ty.replace("*", " * ").split()
    # split at '*': base part, then pointer levels; 'const' before the first '*' qualifies the pointee
    levels, cur = [], []
    for t in ty:
        if t == "*":
            levels.append(cur)
            cur = []
        else:
            cur.append(t)
    base_words = levels[0] if levels else cur
    const_base = "const" in base_words
    base = [w for w in base_words if w not in ("const", "struct")]
    assert len(base) == 1, ty
    b = C_NAMES.get(base[0], base[0])
    # one flag per pointer level, innermost first: is the object that level points to const
    chain = [const_base] + ["const" in lv for lv in levels[1:]] if levels else []
    return (b, tuple(chain))


def _canon_rust(ty):
    ty = ty.strip()
    chain = []
    while ty.startswith("*"):
        m = re.match(r"^\*(const|mut)\s+(.*)$", ty)
        chain.append(m.group(1) == "const")
        ty = m.group(2).strip()
    m = re.match(r"^\[\s*(\w+)\s*;\s*(\d+)\s*\]$", ty)
    if m:
        return ("array", RUST_NAMES.get(m.group(1), m.group(1)), int(m.group(2)))
    # Rust's chain lists the outermost pointer first; the pointee of the innermost is the base
    return (RUST_NAMES.get(ty, ty), tuple(reversed(chain)))


# ---------------------------------------------------------------- structs
def _c_structs():
    text = _strip_c_comments(open(HEADER).read())
    out = {}
    for name, body in re.findall(r"typedef\s+struct\s+(\w+)\s*\{(.*?)\}\s*\w+\s*;", text, flags=re.S):
        fields = []
        for stmt in body.split(";"):
            stmt = stmt.strip()
            if not stmt:
                continue
            m = re.match(r"^(\w+)\s+(.*)$", stmt)
            base = C_NAMES[m.group(1)]
            for var in m.group(2).split(","):
                var = var.strip()
                am = re.match(r"^(\w+)\s*\[\s*(\d+)\s*\]$", var)
                if am:
                    fields.append((am.group(1), ("array", base, int(am.group(2)))))
                else:
                    fields.append((var, (base, ())))
        out[name] = fields
    return out


def _rust_structs():
    src = _rust_block()
    out = {}
    for name, body in re.findall(r"#\[repr\(C\)\][^\n]*?\n?\s*(?:#\[[^\]]*\]\s*)*pub struct (\w+)\s*\{(.*?)\}",
                                 src, flags=re.S):
        fields = []
        for part in re.split(r",(?![^\[]*\])", body):
            part = part.strip()
            if not part:
                continue
            m = re.match(r"^(?:pub\s+)?(\w+)\s*:\s*(.+)$", part, flags=re.S)
            fields.append((m.group(1), _canon_rust(m.group(2))))
        out[name] = fields
    return out


def _size_align(t):
    if t[0] == "array":
        s = SCALARS[t[1]]
        return s * t[2], s
    if t[1]:
        return 8, 8
    s = SCALARS[t[0]]
    return s, s


def _layout(fields):
    off, align, offs = 0, 1, []
    for name, t in fields:
        s, a = _size_align(t)
        off = (off + a - 1) // a * a
        offs.append((name, off, s))
        off += s
        align = max(align, a)
    return offs, (off + align - 1) // align * align


def test_rust_structs_match_header_layout():
    cs, rs = _c_structs(), _rust_structs()
    # opaque handles are zero-sized in Rust and incomplete in C: only the data structs are compared
    data_structs = {n: f for n, f in rs.items() if not (len(f) == 1 and f[0][0] == "_p")}
    assert {"nc_model_config", "nc_load_opts", "nc_verify_result", "nc_decode_stats"} <= set(data_structs)
    for name, rfields in data_structs.items():
        assert name in cs, f"{name}: not a struct of the header"
        cfields = cs[name]
        assert [f[0] for f in rfields] == [f[0] for f in cfields], f"{name}: field names or order differ"
        for (fname, rt), (_, ct) in zip(rfields, cfields):
            assert rt == ct, f"{name}.{fname}: Rust {rt} vs C {ct}"
        rl, rsize = _layout(rfields)
        cl, csize = _layout(cfields)
        assert rl == cl and rsize == csize, f"{name}: Rust layout {rsize} B vs C {csize} B"
    # every header struct that crosses the crate's boundary is mirrored
    for name in cs:
        if name != "nc_synth_spec":  # benchmark-only, left out with nc_synth_*
            assert name in data_structs, f"header struct {name} has no Rust mirror"


def test_model_config_is_144_bytes_everywhere():
    from nanocamelid_amd import _ffi as F
    _, rsize = _layout(_rust_structs()["nc_model_config"])
    _, csize = _layout(_c_structs()["nc_model_config"])
    assert rsize == csize == C.sizeof(F.ModelConfig) == 144


@pytest.mark.parametrize("name,cls", [("nc_model_config", "ModelConfig"), ("nc_load_opts", "LoadOpts"),
                                      ("nc_verify_result", "VerifyResult"), ("nc_decode_stats", "DecodeStats"),
                                      ("nc_synth_spec", "SynthSpec")])
def test_ctypes_structs_match_header(name, cls):
    from nanocamelid_amd import _ffi as F
    st = getattr(F, cls)
    cfields = _c_structs()[name]
    assert [f[0] for f in st._fields_] == [f[0] for f in cfields]
    layout, size = _layout(cfields)
    assert C.sizeof(st) == size
    for (fname, off, _), (cf, ct) in zip(layout, st._fields_):
        assert getattr(st, fname).offset == off, f"{cls}.{fname} offset"
        ctsize = C.sizeof(ct)
        assert ctsize == _size_align(dict(cfields)[fname])[0], f"{cls}.{fname} size"


# ---------------------------------------------------------------- functions
def _c_functions():
    text = _strip_c_comments(open(HEADER).read())
    text = re.sub(r"#[^\n]*", " ", text)
    out = {}
    for ret, name, args in re.findall(r"([A-Za-z_][\w\s\*]*?)\b(nc_\w+)\s*\(([^;{]*?)\)\s*;", text, flags=re.S):
        ret = ret.split(";")[-1].split("}")[-1].strip()
        arglist = [] if args.strip() in ("", "void") else [a.strip() for a in args.split(",")]
        params = []
        for a in arglist:
            m = re.match(r"^(.*?)(\w+)$", a, flags=re.S)
            params.append(_canon_c(m.group(1)))
        out[name] = (_canon_c(ret), params)
    return out


def _rust_functions():
    src = _rust_block()
    ext = re.search(r'extern "C"\s*\{(.*)\}', src, flags=re.S).group(1)
    out = {}
    for name, args, ret in re.findall(r"pub fn (nc_\w+)\s*\(([^)]*)\)\s*(?:->\s*([^;]+))?;", ext, flags=re.S):
        params = []
        for a in [x.strip() for x in args.split(",") if x.strip()]:
            params.append(_canon_rust(a.split(":", 1)[1]))
        out[name] = (_canon_rust(ret) if ret.strip() else ("void", ()), params)
    return out


def test_rust_functions_match_header_prototypes():
    cf, rf = _c_functions(), _rust_functions()
    assert len(rf) >= 40
    for name, (rret, rparams) in rf.items():
        assert name in cf, f"{name}: declared in INTEGRATION.md, not in the header"
        cret, cparams = cf[name]
        assert len(rparams) == len(cparams), f"{name}: {len(rparams)} arguments vs {len(cparams)} in the header"
        for i, (ra, ca) in enumerate(zip(rparams, cparams)):
            assert ra == ca, f"{name} argument {i}: Rust {ra} vs C {ca}"
        assert rret == cret, f"{name} return: Rust {rret} vs C {cret}"
    missing = set(cf) - set(rf) - LEFT_OUT
    assert not missing, f"header functions without a Rust declaration: {sorted(missing)}"


def test_ctypes_signatures_match_header_arity_and_scalars():
    from nanocamelid_amd import _ffi as F
    cf = _c_functions()
    # ctypes aliases c_uint64 and c_size_t to one class on x86-64 Linux: both are 8-byte unsigned
    kinds = {C.c_int32: ("i32", ()), C.c_int: ("i32", ()), C.c_int64: ("i64", ()), C.c_uint32: ("u32", ()),
             C.c_uint64: ("u64", ()), C.c_float: ("f32", ()), C.c_double: ("f64", ())}
    same = {("usize", ()): ("u64", ())}
    for name, (ret, args) in F.SIGNATURES.items():
        assert name in cf, name
        cret, cparams = cf[name]
        assert len(args) == len(cparams), f"{name}: ctypes arity {len(args)} vs {len(cparams)}"
        for i, (a, ca) in enumerate(zip(args, cparams)):
            if ca[1]:  # a pointer in C: any ctypes pointer type (or c_void_p / c_char_p)
                assert a in (C.c_void_p, C.c_char_p) or issubclass(a, C._Pointer), f"{name} arg {i}"
            else:
                assert kinds.get(a) == same.get(ca, ca), f"{name} arg {i}: ctypes {a} vs C {ca}"


def test_rust_constants_match_header_defines():
    text = open(HEADER).read()
    defines = {n: int(v) for n, v in re.findall(r"#define\s+(NC_\w+)\s+\(?(-?\d+)\)?", text)}
    consts = dict(re.findall(r"pub const (NC_\w+)\s*:\s*\w+\s*=\s*(-?\d+)\s*;", _rust_block()))
    assert consts, "no constants in the Rust block"
    for n, v in consts.items():
        assert n in defines and defines[n] == int(v), n
    assert set(defines) - {"NANOCAMELID_GPU_H"} <= set(consts), sorted(set(defines) - set(consts))


def test_checker_fails_on_a_dropped_field():
    # the layout check itself: a mirror without the five rope-scaling fields is 120 bytes
    rf = _rust_structs()["nc_model_config"]
    short = [f for f in rf if not f[0].startswith("rope_scaling")]
    assert _layout(short)[1] == 120 != _layout(_c_structs()["nc_model_config"])[1]
