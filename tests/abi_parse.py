"""Parse the C ABI prototypes of a kernel_set header directory.

Every ``KS_API <ret> ks_name(<params>);`` becomes (name -> return type,
parameter types in order, file:line), with comments removed, whitespace
collapsed, ``*`` attached to the type and parameter names dropped, so two
headers that declare the same ABI compare equal however they are formatted.
"""
from __future__ import annotations

import os
import re

_DECL = re.compile(r"\bKS_API\b(.*?)\b(ks_\w+)\s*\((.*?)\)\s*;", re.S)


def _strip_comments(src: str) -> str:
    src = re.sub(r"/\*.*?\*/", lambda m: "\n" * m.group(0).count("\n"), src, flags=re.S)
    return re.sub(r"//[^\n]*", "", src)


def norm_type(t: str) -> str:
    t = re.sub(r"\s+", " ", t.strip())
    return re.sub(r"\s*\*\s*", "*", t)


def param_type(p: str) -> str:
    p = norm_type(p)
    if p in ("", "void"):
        return p
    m = re.match(r"^(.*?[\*\s])([A-Za-z_]\w*)$", p)  # "<type> <name>" or "<type>*<name>"
    if m and m.group(1).strip():
        return norm_type(m.group(1))
    return p


def prototypes(inc_dir: str) -> dict:
    out = {}
    for fn in sorted(os.listdir(inc_dir)):
        if not fn.endswith(".h"):
            continue
        src = _strip_comments(open(os.path.join(inc_dir, fn)).read())
        for m in _DECL.finditer(src):
            l0 = src[:m.start()].count("\n") + 1
            l1 = src[:m.end()].count("\n") + 1
            params = [param_type(x) for x in m.group(3).split(",")] if m.group(3).strip() else []
            if params == ["void"]:
                params = []
            out[m.group(2)] = {
                "ret": norm_type(m.group(1)),
                "params": params,
                "header": f"include/kernel_set/{fn}:{l0}" + (f"-{l1}" if l1 != l0 else ""),
            }
    return out
