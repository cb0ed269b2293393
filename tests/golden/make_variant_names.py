"""Writes variant_names.json: for each example, the function names that enter
the reference's Materialize pass (examples/<ex>/IR/05_after_enumerate_broadcast.mlir)
and the materialized names it emitted (06_after_canonicalize.mlir), in file
order.  Run in a checkout that has the reference tree:

    python tests/golden/make_variant_names.py /root/reference
"""
import json
import os
import re
import sys

EXAMPLES = ("mm", "bmm_2Dmesh", "split_k_mm_gather", "flashattn", "mqa_decode",
            "mamba_chunk_scan")
FUNC = re.compile(r"func\.func (?:private )?@([A-Za-z0-9_]+)")


def names(path):
    with open(path) as f:
        return FUNC.findall(f.read())


def main(ref):
    out = {}
    for ex in EXAMPLES:
        ir = os.path.join(ref, "examples", ex, "IR")
        out[ex] = {
            "funcs": names(os.path.join(ir, "05_after_enumerate_broadcast.mlir")),
            "variants": names(os.path.join(ir, "06_after_canonicalize.mlir")),
        }
    dst = os.path.join(os.path.dirname(os.path.abspath(__file__)), "variant_names.json")
    with open(dst, "w") as f:
        json.dump(out, f, indent=1)
        f.write("\n")
    print(dst, {k: len(v["variants"]) for k, v in out.items()})


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
