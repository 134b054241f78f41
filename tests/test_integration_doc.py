"""The integration guide's Mojo bindings against the C ABI (no GPU, no Mojo):
every `external_call["t2h_…", R](…)` in the guide names a function that
include/t2h.h declares and passes as many arguments as the declaration takes,
so the bindings a maintainer copies cannot drift from the library. The Mojo
itself cannot be compiled here; this checks what can be checked from the
text."""
import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GUIDE = "INTEGRATION.md"


def split_top(args: str):
    """Split an argument list at the commas outside (), [] and {}."""
    out, depth, cur = [], 0, ""
    for ch in args:
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


def declared():
    src = open(os.path.join(ROOT, "include", "t2h.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    decls = {}
    for m in re.finditer(r"\b(?:int32_t|int64_t|const char\*)\s+(t2h_\w+)\s*\(([^)]*)\)\s*;", src):
        params = split_top(m.group(2))
        decls[m.group(1)] = 0 if params == ["void"] else len(params)
    return decls


def calls():
    doc = open(os.path.join(ROOT, GUIDE)).read()
    found = []
    for m in re.finditer(r'external_call\["(t2h_\w+)",\s*[^\]]*\]?\]\(', doc):
        i, depth = m.end(), 1
        while depth:
            depth += {"(": 1, ")": -1}.get(doc[i], 0)
            i += 1
        found.append((m.group(1), doc[m.end():i - 1]))
    return found


def test_bindings_match_the_header():
    decls = declared()
    assert len(decls) >= 30
    found = calls()
    assert len(found) >= 15
    for name, args in found:
        assert name in decls, f"{GUIDE} calls {name}, which include/t2h.h does not declare"
        n = len(split_top(args))
        assert n == decls[name], f"{GUIDE} passes {n} arguments to {name}; t2h.h declares {decls[name]}"
