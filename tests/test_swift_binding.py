"""The Swift package against the C header it binds (CPU only).

No Swift toolchain exists in this image, so the package under swift/ is never
compiled here.  This test keeps it from drifting away from include/rwkv_hip.h:
every rwkv_* / rwkvq_* function the Swift sources call must be declared in the
header with the same number of parameters, and every other rwkv_* / rwkvq_*
name they use must be a type the header defines.
"""
import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "rwkv_hip.h")
SWIFT = os.path.join(ROOT, "swift", "Sources")
NAME = re.compile(r"\b(rwkvq?_[A-Za-z0-9_]+)\b")


def _strip_c_comments(src):
    src = re.sub(r"/\*.*?\*/", " ", src, flags=re.S)
    return re.sub(r"//[^\n]*", " ", src)


def _split_top(args):
    """Top-level comma-separated pieces of an argument / parameter list."""
    parts, depth, cur, i = [], 0, [], 0
    while i < len(args):
        c = args[i]
        if c == '"':   # string literal (Swift interpolation `\( … )` stays inside)
            j = i + 1
            while j < len(args) and args[j] != '"':
                j += 2 if args[j] == "\\" else 1
            cur.append(args[i:j + 1])
            i = j + 1
            continue
        if c in "([{":
            depth += 1
        elif c in ")]}":
            depth -= 1
        if c == "," and depth == 0:
            parts.append("".join(cur))
            cur = []
        else:
            cur.append(c)
        i += 1
    parts.append("".join(cur))
    return [p.strip() for p in parts if p.strip()]


def header_api():
    src = _strip_c_comments(open(HEADER).read())
    funcs = {}
    for m in re.finditer(r"\b(rwkvq?_[A-Za-z0-9_]+)\s*\(([^;{}]*?)\)\s*;", src):
        params = _split_top(m.group(2))
        funcs[m.group(1)] = 0 if params in ([], ["void"]) else len(params)
    types = set(re.findall(r"\}\s*(rwkvq?_[A-Za-z0-9_]+)\s*;", src))
    types |= set(re.findall(r"typedef\s+(?:struct|enum)\s+\w+\s+(rwkvq?_[A-Za-z0-9_]+)\s*;", src))
    return funcs, types


def swift_calls():
    """(file, name, argument count or None for a bare use) of every rwkv_* /
    rwkvq_* name in the Swift sources."""
    out = []
    for dirpath, _, files in os.walk(SWIFT):
        for fn in files:
            if not fn.endswith(".swift"):
                continue
            path = os.path.join(dirpath, fn)
            src = re.sub(r"//[^\n]*", " ", open(path).read())
            for m in NAME.finditer(src):
                j = m.end()
                while j < len(src) and src[j] in " \t":
                    j += 1
                if j < len(src) and src[j] == "(":
                    depth, k = 0, j
                    while True:
                        if src[k] == "(":
                            depth += 1
                        elif src[k] == ")":
                            depth -= 1
                            if depth == 0:
                                break
                        k += 1
                    out.append((os.path.relpath(path, ROOT), m.group(1), len(_split_top(src[j + 1:k]))))
                else:
                    out.append((os.path.relpath(path, ROOT), m.group(1), None))
    return out


def test_header_parses():
    funcs, types = header_api()
    assert funcs["rwkv_wkv7_seq_fwd"] > 10 and funcs["rwkv_last_error"] == 0
    assert {"rwkv_dtype", "rwkv_status", "rwkv_counters", "rwkvq_file", "rwkvq_manifest"} <= types


def test_swift_calls_match_the_header():
    funcs, types = header_api()
    calls = swift_calls()
    assert len({n for _, n, a in calls if a is not None and n in funcs}) >= 25
    bad = []
    for path, name, nargs in calls:
        if name in funcs:
            if nargs is not None and nargs != funcs[name]:
                bad.append(f"{path}: {name} called with {nargs} arguments, declared with {funcs[name]}")
        elif name in types:
            if nargs not in (None, 0):   # a zero-initialised C struct
                bad.append(f"{path}: type {name} constructed with {nargs} arguments")
        else:
            bad.append(f"{path}: {name} is not declared in include/rwkv_hip.h")
    assert not bad, "\n".join(bad)
