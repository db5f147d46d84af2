"""Writes tests/golden/abi_signatures.json: the expected C ABI of this build.

Entries for symbols the reference declares are read from the reference
headers (cklxx/kernel-set include/kernel_set/*.h, under /root/reference when
this script runs); each keeps its reference file:line as "ref". The extension
entry points, which have no reference counterpart, are taken from this
repository's headers and marked "ref": "extension". Only symbols this build
implements are listed.

Usage: python tests/golden/make_abi_table.py [reference_root]
"""
import json
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
from tests.abi_parse import prototypes  # noqa: E402


def main():
    ref_root = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    ref = prototypes(os.path.join(ref_root, "include", "kernel_set"))
    ours = prototypes(os.path.join(ROOT, "include", "kernel_set"))
    table = {}
    for name in sorted(ours):
        if name in ref:
            e = dict(ref[name])
            e["ref"] = e.pop("header")
        else:
            e = dict(ours[name])
            e.pop("header")
            e["ref"] = "extension"
        table[name] = e
    with open(os.path.join(HERE, "abi_signatures.json"), "w") as f:
        json.dump(table, f, indent=1, sort_keys=True)
        f.write("\n")
    print(f"{len(table)} prototypes ({sum(v['ref'] != 'extension' for v in table.values())} from the reference)")


if __name__ == "__main__":
    main()
