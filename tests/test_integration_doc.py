"""The bindings INTEGRATION.md shows a maintainer agree with the library.

Every ``lib.<name>.argtypes = [...]`` / ``.restype = ...`` assignment in the
document's python listings must equal vates_amd._lib's signature table, every
call of an entry point written out in the document (listings and inline code)
must pass as many arguments as the table lists, and every declaration in
include/vmi.h must have as many parameters as the table lists.
"""
import ctypes
import re
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]


def _split_args(s: str) -> list:
    """Top-level comma split of an argument list (brackets nest)."""
    out, depth, cur = [], 0, ""
    for ch in s:
        if ch in "([{":
            depth += 1
        elif ch in ")]}":
            depth -= 1
        if ch == "," and depth == 0:
            out.append(cur.strip())
            cur = ""
        else:
            cur += ch
    if cur.strip():
        out.append(cur.strip())
    return out


def _balanced(text: str, start: int) -> str:
    """The text between the bracket at ``start`` and its partner."""
    open_ch = text[start]
    close_ch = {"(": ")", "[": "]"}[open_ch]
    depth = 0
    for i in range(start, len(text)):
        if text[i] == open_ch:
            depth += 1
        elif text[i] == close_ch:
            depth -= 1
            if depth == 0:
                return text[start + 1:i]
    raise AssertionError(f"unbalanced {open_ch} at {start}")


def _type_key(t) -> str:
    """Comparable name of a ctypes type (structures by name and fields)."""
    if isinstance(t, type) and issubclass(t, ctypes.Structure):
        return t.__name__ + str([(n, _type_key(ft)) for n, ft in t._fields_])
    if hasattr(t, "_type_") and t.__name__.startswith("LP_"):
        return "POINTER(" + _type_key(t._type_) + ")"
    return {ctypes.c_int32: "c_int", ctypes.c_uint32: "c_uint"}.get(t, t.__name__)


def doc_bindings(text: str) -> dict:
    """name -> {"argtypes": [...], "restype": t} from the python listings."""
    import vates_amd._lib as L
    ns = {k: getattr(ctypes, k) for k in dir(ctypes) if k.startswith("c_") or k == "POINTER"}
    ns.update(ctypes=ctypes, QMat=L.QMat, MoeLayerDesc=L.MoeLayerDesc)
    found = {}
    for block in re.findall(r"```python\n(.*?)```", text, flags=re.S):
        for m in re.finditer(r"lib\.(vmi_\w+)\.argtypes\s*=\s*\[", block):
            body = _balanced(block, m.end() - 1)
            found.setdefault(m.group(1), {})["argtypes"] = eval("[" + body + "]", ns)  # noqa: S307 (doc listing)
        for m in re.finditer(r"lib\.(vmi_\w+)\.restype\s*=\s*([\w.]+)", block):
            found.setdefault(m.group(1), {})["restype"] = eval(m.group(2), ns)  # noqa: S307
    return found


def doc_calls(text: str) -> list:
    """(name, argument count, context) of every entry point call written out."""
    calls = []
    for block in re.findall(r"```python\n(.*?)```", text, flags=re.S):
        for m in re.finditer(r"lib\.(vmi_\w+)\(", block):
            calls.append((m.group(1), len(_split_args(_balanced(block, m.end() - 1))), "listing"))
    prose = re.sub(r"```.*?```", "", text, flags=re.S)
    for code in re.findall(r"`([^`]+)`", prose):
        for m in re.finditer(r"\b(vmi_\w+)\(", code):
            inner = _balanced(code, m.end() - 1)
            calls.append((m.group(1), len(_split_args(inner)), code))
    return calls


def header_arity() -> dict:
    text = re.sub(r"/\*.*?\*/", "", (ROOT / "include" / "vmi.h").read_text(), flags=re.S)
    out = {}
    for m in re.finditer(r"^[\w\s\*]+?\b(vmi_\w+)\s*\(", text, flags=re.M):
        params = _split_args(_balanced(text, m.end() - 1))
        out[m.group(1)] = 0 if params in ([], ["void"]) else len(params)
    return out


def check_document(text: str) -> list:
    """Every disagreement between the document and the signature table."""
    import vates_amd._lib as L
    problems = []
    for name, b in doc_bindings(text).items():
        if name not in L._SIGNATURES:
            problems.append(f"{name}: not an entry point")
            continue
        res, args = L._SIGNATURES[name]
        if "argtypes" in b and [_type_key(t) for t in b["argtypes"]] != [_type_key(t) for t in args]:
            problems.append(f"{name}.argtypes: document {len(b['argtypes'])} args, library {len(args)}")
        if "restype" in b and _type_key(b["restype"]) != _type_key(res):
            problems.append(f"{name}.restype differs")
    for name, n, ctx in doc_calls(text):
        if name not in L._SIGNATURES:
            problems.append(f"{name}: not an entry point ({ctx})")
        elif n != len(L._SIGNATURES[name][1]):
            problems.append(f"{name} called with {n} args, library takes {len(L._SIGNATURES[name][1])} ({ctx})")
    return problems


def test_integration_bindings_match_library():
    text = (ROOT / "INTEGRATION.md").read_text()
    assert len(doc_bindings(text)) >= 6 and len(doc_calls(text)) >= 10
    assert check_document(text) == []


def test_checker_catches_a_stale_binding():
    # a listing with a dropped argument and an inline call with one too few
    stale = ("```python\nlib.vmi_lm_head.argtypes = [c_void_p, c_int, c_int, c_void_p, ctypes.c_float, c_void_p,"
             " c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_size_t, c_void_p]\n```\n"
             "| x | `vmi_spec_commit(record, hid, hidden, K, H, x, pos, mtp_len, mtp_pos, stream)` |\n")
    problems = check_document(stale)
    assert any("vmi_lm_head.argtypes" in p for p in problems)
    assert any("vmi_spec_commit called with 10" in p for p in problems)


def test_header_parameter_counts_match_library():
    import vates_amd._lib as L
    arity = header_arity()
    assert set(arity) == set(L._SIGNATURES)
    for name, (_, args) in L._SIGNATURES.items():
        assert arity[name] == len(args), (name, arity[name], len(args))
