"""The Rust crate's raw bindings against include/smoe.h, on the CPU.

No Rust toolchain is installed here, so the crate cannot be compiled; this
test instead parses `streamoe_amd/rust/streammoe-hip/src/sys.rs` and the
header and requires them to agree exactly: every function (name, argument
names, argument types with pointer constness, return type), every struct
(field order, names and types), every status / option constant and
SMOE_MAX_K. It also checks that each `sys::` call and struct literal in
`src/lib.rs` names something sys.rs declares and passes as many arguments
(or fields) as it declares."""
import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "smoe.h")
CRATE = os.path.join(ROOT, "streamoe_amd", "rust", "streammoe-hip")

C_BASE = {"int": "c_int", "int32_t": "i32", "uint32_t": "u32", "int64_t": "i64", "uint64_t": "u64",
          "uint16_t": "u16", "float": "f32", "char": "c_char", "void": "c_void"}


def strip_c_comments(s):
    s = re.sub(r"/\*.*?\*/", " ", s, flags=re.S)
    return re.sub(r"//[^\n]*", " ", s)


def c_type_to_rust(decl):
    """'const void* const* norm_w' -> ('norm_w', '*const *const c_void')."""
    toks = re.findall(r"[A-Za-z_][A-Za-z0-9_]*|\*", decl)
    name = toks[-1] if len(toks) > 1 and toks[-1] != "*" and not (len(toks) == 1) else None
    if name is not None and (toks[-1] in C_BASE or toks[-1] == "const"):
        name = None
    body = toks[:-1] if name is not None else toks
    const = False
    base = None
    i = 0
    while i < len(body) and body[i] != "*":
        if body[i] == "const":
            const = True
        else:
            assert base is None, decl
            base = body[i]
        i += 1
    t = C_BASE.get(base, base)
    while i < len(body):
        assert body[i] == "*", decl
        t = ("*const " if const else "*mut ") + t
        const = i + 1 < len(body) and body[i + 1] == "const"
        i += 2 if const else 1
    return name, t


def header_api():
    src = strip_c_comments(open(HEADER).read())
    funcs = {}
    code = re.sub(r"^\s*#[^\n]*", " ", src, flags=re.M)
    for stmt in code.split(";"):
        stmt = re.split(r"[{}]", stmt)[-1]
        m = re.fullmatch(r"\s*([A-Za-z_][\w\s\*]*?)\b(smoe_\w+)\s*\(([^)]*)\)\s*", stmt)
        if not m or "typedef" in m.group(1):
            continue
        ret, name, args = m.group(1), m.group(2), m.group(3).strip()
        _, rret = c_type_to_rust(ret.strip())
        params = [] if args in ("", "void") else [c_type_to_rust(a.strip()) for a in args.split(",")]
        funcs[name] = (params, rret)
    structs = {}
    for m in re.finditer(r"typedef\s+struct\s*\{([^}]*)\}\s*(\w+)\s*;", src):
        fields = [c_type_to_rust(f.strip()) for f in m.group(1).split(";") if f.strip()]
        structs[m.group(2)] = fields
    consts = {k: int(v) for k, v in re.findall(r"\b(SMOE_(?:OK|ERR_\w+|OPT_\w+))\s*=\s*(\d+)", src)}
    consts["SMOE_MAX_K"] = int(re.search(r"#define\s+SMOE_MAX_K\s+(\d+)", src).group(1))
    consts["SMOE_ABI_VERSION"] = int(re.search(r"#define\s+SMOE_ABI_VERSION\s+(\d+)", src).group(1))
    return funcs, structs, consts


def norm(t):
    return re.sub(r"\s+", " ", t.strip()).replace("* ", "*").replace("*const", "*const ").replace(
        "*mut", "*mut ").replace("  ", " ")


def split_top(s, sep=","):
    out, depth, cur = [], 0, ""
    for ch in s:
        if ch in "([{<":
            depth += 1
        elif ch in ")]}>" and depth:
            depth -= 1
        if ch == sep and depth == 0:
            out.append(cur)
            cur = ""
        else:
            cur += ch
    if cur.strip():
        out.append(cur)
    return [x.strip() for x in out if x.strip()]


def sys_api():
    src = re.sub(r"//[^\n]*", " ", open(os.path.join(CRATE, "src", "sys.rs")).read())
    block = re.search(r'extern\s+"C"\s*\{(.*)\n\}', src, flags=re.S).group(1)
    funcs = {}
    for m in re.finditer(r"pub\s+fn\s+(\w+)\s*\(([^)]*)\)\s*(?:->\s*([^;]+))?;", block):
        params = []
        for a in split_top(m.group(2)):
            n, t = a.split(":", 1)
            params.append((n.strip(), norm(t)))
        funcs[m.group(1)] = (params, norm(m.group(3) or "()"))
    structs = {}
    for m in re.finditer(r"pub\s+struct\s+(\w+)\s*\{([^}]*)\}", src):
        fields = []
        for f in split_top(m.group(2)):
            n, t = f.split(":", 1)
            fields.append((n.replace("pub", "").strip(), norm(t)))
        structs[m.group(1)] = fields
    consts = {k: int(v) for k, v in re.findall(r"pub\s+const\s+(\w+)\s*:\s*\w+\s*=\s*(\d+)\s*;", src)}
    return funcs, structs, consts


def test_header_parser_reads_known_declarations():
    funcs, structs, consts = header_api()
    assert funcs["smoe_destroy"] == ([("h", "*mut smoe_handle")], "c_int")
    assert funcs["smoe_create"][0][2] == ("out", "*mut *mut smoe_handle")
    assert funcs["smoe_moe_decode_layers"][0][3] == ("norm_w", "*const *const c_void")
    assert funcs["smoe_strerror"] == ([("status", "c_int")], "*const c_char")
    assert funcs["smoe_abi_version"] == ([], "u32")
    assert structs["smoe_binding"] == [("base", "*const c_void"), ("offset", "u64")]
    assert consts["SMOE_ERR_IO"] == 13 and consts["SMOE_MAX_K"] == 16
    assert len(funcs) >= 30


def test_sys_functions_match_header():
    hf, _, _ = header_api()
    rf, _, _ = sys_api()
    assert sorted(rf) == sorted(hf), (set(hf) ^ set(rf))
    for name, (params, ret) in hf.items():
        rparams, rret = rf[name]
        assert [norm(t) for _, t in params] == [t for _, t in rparams], name
        assert [n for n, _ in params] == [n for n, _ in rparams], name
        assert norm(ret) == rret, (name, ret, rret)


def test_sys_structs_match_header():
    _, hs, _ = header_api()
    _, rs, _ = sys_api()
    for name, fields in hs.items():
        assert name in rs, name
        assert [(n, norm(t)) for n, t in fields] == rs[name], name
    # The opaque handle is a zero-sized repr(C) type on the Rust side.
    assert rs["smoe_handle"] == [("_private", "[u8; 0]")]


def test_sys_constants_match_header():
    _, _, hc = header_api()
    _, _, rc = sys_api()
    assert hc == rc


def test_lib_calls_match_sys_arity():
    rf, rs, _ = sys_api()
    lib = re.sub(r"//[^\n]*", " ", open(os.path.join(CRATE, "src", "lib.rs")).read())
    called = set()
    for m in re.finditer(r"sys::(smoe_\w+)\s*([({])", lib):
        name, opener = m.group(1), m.group(2)
        if re.search(r"->\s*$", lib[:m.start()]):
            continue  # a return type followed by the function body
        closer = ")" if opener == "(" else "}"
        depth, i = 1, m.end()
        while depth:
            c = lib[i]
            depth += c == opener
            depth -= c == closer
            i += 1
        inner = lib[m.end():i - 1]
        if opener == "(":
            assert name in rf, name
            assert len(split_top(inner)) == len(rf[name][0]), (name, inner)
            called.add(name)
        else:
            assert name in rs, name
            got = [f.split(":", 1)[0].strip() for f in split_top(inner)]
            assert got == [n for n, _ in rs[name]], (name, got)
    # The safe layer reaches every entry point that does work on the device
    # or the layer files (the synthetic-data helpers and raw topk/softmax
    # steps stay in sys).
    for must in ("smoe_create", "smoe_destroy", "smoe_qmv", "smoe_qmv_argmax", "smoe_qmm", "smoe_router",
                 "smoe_experts_decode", "smoe_moe_decode_layer", "smoe_moe_decode_layers",
                 "smoe_moe_decode_layers_noalloc", "smoe_moe_decode_tokens", "smoe_moe_prefill",
                 "smoe_layer_file_layout", "smoe_load_file"):
        assert must in called, must


def test_cargo_manifest_links_libsmoe():
    cargo = open(os.path.join(CRATE, "Cargo.toml")).read()
    assert re.search(r'^name\s*=\s*"streammoe-hip"', cargo, flags=re.M)
    assert re.search(r'^links\s*=\s*"smoe"', cargo, flags=re.M)
    build = open(os.path.join(CRATE, "build.rs")).read()
    assert "rustc-link-lib=dylib=smoe" in build
