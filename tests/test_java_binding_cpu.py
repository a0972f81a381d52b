"""The Java FFM binding (java/backend-hip/.../HipAttentionLibrary.java) against the C ABI it
binds (include/jmodels_attn.h): every export of the header has exactly one downcall descriptor,
with the same arity and, parameter by parameter, the value layout FFM needs for the C type
(int32/uint32 JAVA_INT, uint64 JAVA_LONG, float JAVA_FLOAT, pointers ADDRESS), return type
included; and the LAYER / LAYER_SPEC struct layouts match the header's structs field by field.
No JDK is installed here, so the Java is parsed, not compiled."""

import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
JAVA = os.path.join(ROOT, "java", "backend-hip", "src", "main", "java", "com", "integrallis",
                    "models", "backend", "hip", "HipAttentionLibrary.java")
HEADER = os.path.join(ROOT, "include", "jmodels_attn.h")


def _strip_c(text):
    return re.sub(r"/\*.*?\*/", "", text, flags=re.S)


def _layout_of_c(param):
    p = " ".join(param.replace("const", " ").split())
    if "*" in p:
        return "ADDRESS"
    base = p.split()[0]
    return {"int32_t": "JAVA_INT", "uint32_t": "JAVA_INT", "uint64_t": "JAVA_LONG",
            "float": "JAVA_FLOAT", "void": None}[base]


def header_exports():
    text = _strip_c(open(HEADER).read())
    text = "\n".join(ln for ln in text.splitlines() if not ln.lstrip().startswith("#"))
    out = {}
    for m in re.finditer(r"JMODELS_ATTN_API\s+(.*?)\b(jmodels_attn_\w+)\s*\((.*?)\)\s*;", text, re.S):
        ret, name, params = m.group(1), m.group(2), m.group(3)
        params = [p.strip() for p in params.split(",")]
        if params == ["void"]:
            params = []
        out[name] = (_layout_of_c(ret + " x"), [_layout_of_c(p) for p in params])
    return out


def _split_args(s):
    depth, cur, parts = 0, "", []
    for ch in s:
        if ch == "(":
            depth += 1
        elif ch == ")":
            depth -= 1
        if ch == "," and depth == 0:
            parts.append(cur.strip())
            cur = ""
        else:
            cur += ch
    if cur.strip():
        parts.append(cur.strip())
    return parts


def java_downcalls():
    text = open(JAVA).read()
    text = re.sub(r"//[^\n]*", "", text)
    consts = {}
    for m in re.finditer(r"private static final FunctionDescriptor (\w+)\s*=\s*(.*?);", text, re.S):
        consts[m.group(1)] = m.group(2)

    def parse(expr):
        expr = " ".join(expr.split())
        if expr in consts:
            return parse(consts[expr])
        m = re.fullmatch(r"FunctionDescriptor\.(of|ofVoid)\((.*)\)", expr)
        assert m, expr
        args = _split_args(m.group(2))
        if m.group(1) == "ofVoid":
            return None, args
        return args[0], args[1:]

    body = text[text.index("static final Map<String, FunctionDescriptor> DOWNCALLS"):]
    body = body[:body.index(");\n\n")]
    out = {}
    for m in re.finditer(r'entry\(\s*"(\w+)",\s*(.*?)\)(?=,\s*entry\(|\s*$)', body + " ", re.S):
        name, expr = m.group(1), m.group(2)
        assert name not in out, f"{name} bound twice"
        out[name] = parse(expr)
    return out


def test_every_export_has_a_matching_downcall():
    exports = header_exports()
    downcalls = java_downcalls()
    assert len(exports) >= 35
    assert sorted(downcalls) == sorted(exports), (set(exports) ^ set(downcalls))
    for name, (ret, params) in exports.items():
        jret, jparams = downcalls[name]
        assert jret == ret, f"{name}: returns {jret}, header {ret}"
        assert len(jparams) == len(params), f"{name}: {len(jparams)} parameters, header {len(params)}"
        for i, (a, b) in enumerate(zip(jparams, params)):
            assert a == b, f"{name} parameter {i}: {a}, header {b}"


def _c_struct(name):
    text = _strip_c(open(HEADER).read())
    m = re.search(r"typedef struct %s \{(.*?)\} %s;" % (name, name), text, re.S)
    fields = []
    for line in m.group(1).split(";"):
        line = " ".join(line.replace("const", " ").split())
        if not line:
            continue
        fields.append((line.split()[-1].lstrip("*"), "ADDRESS" if "*" in line else _layout_of_c(line)))
    return fields


def _java_struct(const):
    text = open(JAVA).read()
    m = re.search(r"public static final StructLayout %s\s*=\s*MemoryLayout\.structLayout\((.*?)\);" % const,
                  text, re.S)
    return [(f, lay) for lay, f in re.findall(r"(\w+)\.withName\(\"(\w+)\"\)", m.group(1))]


def test_struct_layouts_match_the_header():
    assert _java_struct("LAYER") == _c_struct("jmodels_attn_layer")
    assert _java_struct("LAYER_SPEC") == _c_struct("jmodels_attn_layer_spec")


def test_constants_match_the_header():
    text = open(JAVA).read()
    header = _strip_c(open(HEADER).read())
    hdefs = dict(re.findall(r"#define JMODELS_ATTN_(\w+)\s+(\d+)u?\b", header))
    caps = {n: 1 << int(s) for n, _, s in
            re.findall(r"#define JMODELS_ATTN_(CAP_\w+)\s+\((\d+)ull\s*<<\s*(\d+)\)", header)}
    for name, value in caps.items():
        m = re.search(r"public static final long %s = 1L << (\d+);" % name, text)
        assert m and 1 << int(m.group(1)) == value, name
    assert re.search(r"ABI_VERSION = %s;" % hdefs["ABI_VERSION"], text)
    for name in ("OK", "NULL_POINTER", "INVALID_SHAPE", "BUFFER_TOO_SMALL", "PANIC", "DEVICE_ERROR",
                 "OUT_OF_RANGE", "UNAVAILABLE", "NON_FINITE", "NOT_CAPTURABLE"):
        m = re.search(r"public static final int %s = (\d+);" % name, text)
        assert m and m.group(1) == hdefs[name], name
