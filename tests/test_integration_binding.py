"""The Java FFM binding in INTEGRATION.md, checked against include/nva.h without a JDK.

The reference builds with maven.compiler.release 21 (pom.xml:21), where java.lang.foreign is a
preview API.  The class must therefore use Java 21's names, bind every export of the C ABI with
a descriptor whose layouts match the C prototype, cast every ``invokeExact`` to the handle's
return type (a bare-statement call has return type void and throws WrongMethodTypeException),
pass as many arguments as the prototype has, and lay its structs out exactly as the C structs.

``check_binding`` returns the list of problems; the planted mistakes at the end must each be
reported, so the checker itself is pinned.
"""

import ctypes
import os
import re

import pytest

from nanollvm_amd import _native as N

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "nva.h")
INTEGRATION = os.path.join(ROOT, "INTEGRATION.md")
HIP_HEADER = "/opt/rocm/include/hip/hip_runtime_api.h"

# HIP runtime functions the class binds (hip_runtime_api.h); hipError_t and hipMemcpyKind are
# C enums (int), size_t is 64-bit.
HIP_PROTOS = {
    "hipMalloc": ("JAVA_INT", ["ADDRESS", "JAVA_LONG"]),
    "hipFree": ("JAVA_INT", ["ADDRESS"]),
    "hipMemcpy": ("JAVA_INT", ["ADDRESS", "ADDRESS", "JAVA_LONG", "JAVA_INT"]),
}
HIP_C = {
    "hipMalloc": "hipError_t hipMalloc(void** ptr, size_t size);",
    "hipFree": "hipError_t hipFree(void* ptr);",
    "hipMemcpy": "hipError_t hipMemcpy(void* dst, const void* src, size_t sizeBytes, "
                 "hipMemcpyKind kind);",
}

LAYOUT_BYTES = {"JAVA_INT": 4, "JAVA_FLOAT": 4, "JAVA_LONG": 8, "JAVA_DOUBLE": 8, "ADDRESS": 8,
                "JAVA_BYTE": 1}
# Java struct name -> the ctypes mirror of the C struct (ctypes lays out like the C compiler).
STRUCTS = {"DESC": N.AttnDesc, "NORM": N.RmsNormDesc, "SEQ": N.Seq, "STEP_META": N.StepMetaOut}


def c_layout(ctype: str) -> str:
    t = ctype.strip()
    if "*" in t:
        return "ADDRESS"
    t = re.sub(r"\bconst\b", "", t).split()[0]
    return {"int": "JAVA_INT", "int32_t": "JAVA_INT", "nva_status": "JAVA_INT",
            "int64_t": "JAVA_LONG", "float": "JAVA_FLOAT", "double": "JAVA_DOUBLE",
            "uint8_t": "JAVA_BYTE"}[t]


def header_protos(text: str) -> dict:
    """name -> (return layout, [argument layouts]) of every function nva.h declares."""
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    out = {}
    for m in re.finditer(r"(nva_status|void\s*\*|const\s+char\s*\*)\s*(nva_\w+)\s*\(([^;{]*?)\)\s*;",
                         text, flags=re.S):
        ret, name, args = m.group(1), m.group(2), " ".join(m.group(3).split())
        argl = [] if args.strip() in ("", "void") else [c_layout(a.rsplit(" ", 1)[0] if "*" not in a
                                                                 else a) for a in args.split(",")]
        out[name] = (c_layout(ret), argl)
    return out


def java_block(md: str) -> str:
    m = re.search(r"```java\n(.*?)```", md, flags=re.S)
    assert m, "no java block in INTEGRATION.md"
    return m.group(1)


def balanced(text: str, i: int) -> tuple:
    """(contents, end) of the parenthesised group whose '(' is at text[i]."""
    assert text[i] == "("
    depth = 0
    for j in range(i, len(text)):
        if text[j] == "(":
            depth += 1
        elif text[j] == ")":
            depth -= 1
            if depth == 0:
                return text[i + 1:j], j + 1
    raise ValueError("unbalanced parentheses")


def split_top(args: str) -> list:
    parts, depth, cur = [], 0, ""
    for ch in args:
        if ch in "([{":
            depth += 1
        elif ch in ")]}":
            depth -= 1
        if ch == "," and depth == 0:
            parts.append(cur.strip())
            cur = ""
        else:
            cur += ch
    if cur.strip():
        parts.append(cur.strip())
    return parts


def java_handles(java: str) -> dict:
    """handle variable -> (library loader, symbol, return layout or None, [argument layouts])."""
    out = {}
    for m in re.finditer(r"MethodHandle\s+(\w+)\s*=\s*(h|hip)\(\s*\"(\w+)\"\s*,\s*"
                         r"FunctionDescriptor\.(of|ofVoid)\s*(?=\()", java):
        body, _ = balanced(java, m.end())
        lay = [re.sub(r"\s+", "", x) for x in split_top(body)]
        ret = None if m.group(4) == "ofVoid" else lay.pop(0)
        out[m.group(1)] = (m.group(2), m.group(3), ret, lay)
    return out


def java_structs(java: str) -> dict:
    """struct name -> [(offset, size, field name or None for padding)]."""
    out = {}
    for m in re.finditer(r"StructLayout\s+(\w+)\s*=\s*MemoryLayout\.structLayout\s*(?=\()", java):
        body, _ = balanced(java, m.end())
        off, fields = 0, []
        for item in split_top(body):
            pm = re.fullmatch(r"MemoryLayout\.paddingLayout\((\d+)\)", item)
            if pm:
                size, name = int(pm.group(1)), None
            else:
                fm = re.fullmatch(r"(\w+)\.withName\(\"(\w+)\"\)", item)
                assert fm, f"unparsed struct member {item!r}"
                size, name = LAYOUT_BYTES[fm.group(1)], fm.group(2)
            fields.append((off, size, name))
            off += size
        out[m.group(1)] = fields
    return out


def check_binding(java: str, header: str) -> list:
    errs = []
    protos = header_protos(header)
    handles = java_handles(java)
    bound = {}
    for var, (lib, sym, ret, args) in handles.items():
        want = protos.get(sym) if lib == "h" else HIP_PROTOS.get(sym)
        if want is None:
            errs.append(f"{var}: {sym} is not declared by {'nva.h' if lib == 'h' else 'HIP'}")
            continue
        if (ret, args) != want:
            errs.append(f"{var}: descriptor {ret}{args} != C prototype {want[0]}{want[1]}")
        bound.setdefault(sym, []).append(var)
    for sym in protos:
        if sym not in bound:
            errs.append(f"{sym} has no downcall handle")
    for sym, vars_ in bound.items():
        if len(vars_) > 1:
            errs.append(f"{sym} is bound twice: {vars_}")

    # Every invokeExact: cast to the handle's return type, arity of the prototype.
    for m in re.finditer(r"(\w+)\.invokeExact\s*(?=\()", java):
        var = m.group(1)
        if var not in handles:
            errs.append(f"invokeExact on unknown handle {var}")
            continue
        _, sym, ret, args = handles[var]
        before = java[:m.start()].rstrip()
        cast = re.search(r"\((int|long|float|double|MemorySegment)\)$", before)
        want = {"JAVA_INT": "int", "JAVA_LONG": "long", "JAVA_FLOAT": "float",
                "JAVA_DOUBLE": "double", "ADDRESS": "MemorySegment", None: None}[ret]
        got = cast.group(1) if cast else None
        if got != want:
            line = java[:m.start()].count("\n") + 1
            errs.append(f"line {line}: {var}.invokeExact cast ({got}) does not match the "
                        f"handle's return type ({want}); a bare statement has type void")
        call, _ = balanced(java, m.end())
        n = len(split_top(call))
        if n != len(args):
            line = java[:m.start()].count("\n") + 1
            errs.append(f"line {line}: {var}.invokeExact passes {n} arguments, {sym} takes "
                        f"{len(args)}")

    # Java 21 preview names only (the Java 22 final API renamed them).
    for pat, what in ((r"\.allocateFrom\s*\(", "allocateFrom (Java 22)"),
                      (r"\.getString\s*\(", "getString (Java 22)"),
                      (r"\.setString\s*\(", "setString (Java 22)"),
                      (r"\.allocate\s*\(\s*[A-Z_]+\s*,", "allocate(layout, count) (Java 22)")):
        for m in re.finditer(pat, java):
            errs.append(f"line {java[:m.start()].count(chr(10)) + 1}: {what}")

    # Struct layouts against the C structs (through their ctypes mirrors).
    structs = java_structs(java)
    for jname, cstruct in STRUCTS.items():
        if jname not in structs:
            errs.append(f"struct layout {jname} missing")
            continue
        fields = structs[jname]
        named = {n: (o, s) for o, s, n in fields if n}
        if [n for _, _, n in fields if n] != [f for f, _ in cstruct._fields_]:
            errs.append(f"{jname}: fields {list(named)} != C fields "
                        f"{[f for f, _ in cstruct._fields_]}")
        for f, ft in cstruct._fields_:
            if f in named:
                o, s = named[f]
                co = getattr(cstruct, f).offset
                if (o, s) != (co, ctypes.sizeof(ft)):
                    errs.append(f"{jname}.{f}: offset/size {(o, s)} != C {(co, ctypes.sizeof(ft))}")
                if o % s:
                    errs.append(f"{jname}.{f}: offset {o} not aligned to {s}")
        total = sum(s for _, s, _ in fields)
        if total != ctypes.sizeof(cstruct):
            errs.append(f"{jname}: {total} bytes != C sizeof {ctypes.sizeof(cstruct)}")

    # Raw offsets written into struct segments: e (nva_seq) and m (nva_step_meta).
    for var, jname in (("e", "SEQ"), ("m", "STEP_META")):
        by_off = {o: (s, n) for o, s, n in structs.get(jname, []) if n}
        for mm in re.finditer(rf"\b{var}\.(set|get)\(\s*(\w+)\s*,\s*(\d+)\s*[,)]", java):
            lay, off = mm.group(2), int(mm.group(3))
            if off not in by_off or by_off[off][0] != LAYOUT_BYTES.get(lay):
                errs.append(f"{var}.{mm.group(1)}({lay}, {off}) hits no {jname} field of that size")
    return errs


@pytest.fixture(scope="module")
def texts():
    with open(INTEGRATION) as f:
        java = java_block(f.read())
    with open(HEADER) as f:
        header = f.read()
    return java, header


def test_header_parse_matches_ctypes_binding(texts):
    """The header parser sees exactly the symbols the ctypes binding declares (which
    test_abi.py checks against the library's exports), with the same arity."""
    protos = header_protos(texts[1])
    assert set(protos) == set(N.SIGNATURES)
    for name, (ret, args) in protos.items():
        assert len(args) == len(N.SIGNATURES[name][0]), name


def test_hip_prototypes_match_runtime_header():
    if not os.path.exists(HIP_HEADER):
        pytest.skip("ROCm headers not installed")
    with open(HIP_HEADER) as f:
        text = " ".join(f.read().split())
    for name, proto in HIP_C.items():
        assert " ".join(proto.split()) in text, name


def test_java_binding_matches_header(texts):
    errs = check_binding(*texts)
    assert not errs, "\n".join(errs)


def test_java_binding_binds_kv_layer(texts):
    """KvCacheArena.getKeyCache/getValueCache (KvCacheArena.java:111-124) go through
    nva_kv_layer."""
    java = texts[0]
    assert re.search(r"KV_LAYER\.invokeExact", java)
    assert "getKeyCache" in java and "getValueCache" in java


def test_build_uses_enable_preview():
    with open(INTEGRATION) as f:
        md = f.read()
    assert "--enable-preview" in md


PLANTED = [
    ("statement-form invokeExact", lambda j: j.replace(
        "st = (int) KV_DESTROY.invokeExact(kv);", "KV_DESTROY.invokeExact(kv);")),
    ("wrong cast", lambda j: j.replace("(MemorySegment) CTX_STREAM.invokeExact",
                                       "(int) CTX_STREAM.invokeExact")),
    ("missing argument", lambda j: j.replace(
        "LINEAR.invokeExact(ctx, attnOut, rows, in, weight, out, bias, y)",
        "LINEAR.invokeExact(ctx, attnOut, rows, in, weight, out, y)")),
    ("int for int64_t", lambda j: j.replace(
        'h("nva_kv_write", FunctionDescriptor.of(JAVA_INT,\n      ADDRESS, JAVA_INT, JAVA_INT, '
        'JAVA_LONG', 'h("nva_kv_write", FunctionDescriptor.of(JAVA_INT,\n      ADDRESS, JAVA_INT, '
        'JAVA_INT, JAVA_INT')),
    ("Java 22 allocateFrom", lambda j: j.replace("arena.allocateArray(JAVA_INT, headDims)",
                                                 "arena.allocateFrom(JAVA_INT, headDims)")),
    ("Java 22 getString", lambda j: j.replace("getUtf8String(0)", "getString(0)")),
    ("missing padding", lambda j: j.replace(
        'JAVA_INT.withName("num_blocks"),\n      MemoryLayout.paddingLayout(4));',
        'JAVA_INT.withName("num_blocks"));')),
    ("unbound export", lambda j: re.sub(r"static final MethodHandle KV_LAYER = h\(.*?\)\);\n", "",
                                        j, flags=re.S)),
    ("wrong struct offset", lambda j: j.replace("e.set(JAVA_INT, 24, table.length);",
                                                "e.set(JAVA_INT, 20, table.length);")),
]


@pytest.mark.parametrize("name,mutate", PLANTED, ids=[p[0] for p in PLANTED])
def test_checker_catches_planted_mistake(texts, name, mutate):
    java, header = texts
    bad = mutate(java)
    assert bad != java, f"planted mistake '{name}' did not apply"
    assert check_binding(bad, header), f"checker missed: {name}"
