"""The Deno.dlopen binding written out in INTEGRATION.md against the C ABI in include/tsc.h.

A maintainer who adds the TypeScript host copies that symbol table; Deno is not in this image, so
nothing runs it.  This test keeps it honest mechanically: the table names exactly the functions
tsc.h declares, each with tsc.h's parameter count, and every parameter and result uses the Deno FFI
type of its C type (pointers and arrays: "pointer" or "buffer"; int32_t / int: "i32"; int64_t:
"i64"; size_t: "usize"; float: "f32"; void result: "void")."""
import re
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]


def _c_decls() -> dict:
    text = (ROOT / "include" / "tsc.h").read_text()
    text = re.sub(r"/\*.*?\*/", " ", text, flags=re.S)
    text = re.sub(r"//[^\n]*", " ", text)
    decls = {}
    for m in re.finditer(r"([A-Za-z_][\w\s\*]*?)\b(tsc_\w+)\s*\(([^;{]*?)\)\s*;", text):
        ret, name, params = m.group(1).strip(), m.group(2), m.group(3).strip()
        plist = [] if params in ("", "void") else [p.strip() for p in params.split(",")]
        decls[name] = (ret, plist)
    return decls


def _deno_table() -> dict:
    text = (ROOT / "INTEGRATION.md").read_text()
    m = re.search(r"Deno\.dlopen\(.*?, \{\n(.*?)\n\}( as const)?\);", text, flags=re.S)
    assert m, "no Deno.dlopen block in INTEGRATION.md"
    body = m.group(1)
    table = {}
    for e in re.finditer(r"(tsc_\w+)\s*:\s*\{\s*parameters:\s*\[(.*?)\]\s*,\s*result:\s*\"(\w+)\"",
                         body, flags=re.S):
        params = re.findall(r"\"(\w+)\"", e.group(2))
        table[e.group(1)] = (params, e.group(3))
    return table


def _ffi_types(c_type: str) -> set:
    t = c_type.replace("const", "").strip()
    if "*" in t or "[" in t:
        return {"pointer", "buffer"}
    t = re.sub(r"\s+\w+$", "", t).strip() if " " in t else t  # drop the parameter name
    return {"int32_t": {"i32"}, "int": {"i32"}, "int64_t": {"i64"}, "size_t": {"usize"},
            "float": {"f32"}, "uint32_t": {"u32"}, "void": {"void"}}[t]


def test_deno_table_matches_header():
    decls, table = _c_decls(), _deno_table()
    assert len(decls) >= 40, sorted(decls)
    assert set(table) == set(decls), (sorted(set(decls) - set(table)), sorted(set(table) - set(decls)))
    for name, (ret, params) in decls.items():
        dparams, dres = table[name]
        assert len(dparams) == len(params), (name, params, dparams)
        for cp, dp in zip(params, dparams):
            assert dp in _ffi_types(cp), (name, cp, dp)
        want_res = {"pointer"} if "*" in ret else _ffi_types(ret)
        assert dres in want_res, (name, ret, dres)


def test_header_parser_sees_multiline_declarations():
    decls = _c_decls()
    ret, params = decls["tsc_map_build"]
    assert ret == "int" and len(params) == 14
    assert decls["tsc_version"] == ("int", [])
    assert decls["tsc_last_error"][0] == "const char*"
