"""Writes eden_codebooks.json: the reference's Lloyd-Max N(0,1) codebooks B1..B4
(/root/reference/src/eden.rs:15-44) as IEEE binary32 bit patterns.

Runs in the build container only (it reads the reference's source as text;
the fixture it writes is 30 numbers).  Each decimal literal is rounded to the
nearest binary32 directly (round half to even), as rustc does for an f32
literal; going through a float64 first could round twice.

    python tests/golden/make_codebooks.py [/root/reference]
"""
import json
import os
import re
import sys
from fractions import Fraction

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "eden_codebooks.json")


def f32_nearest(lit: str) -> np.float32:
    """The binary32 nearest to the decimal `lit` (ties to even mantissa)."""
    exact = Fraction(lit)
    c = np.float32(float(exact))
    cands = {c, np.nextafter(c, np.float32(np.inf)), np.nextafter(c, np.float32(-np.inf))}
    best = None
    for x in sorted(cands, key=float):
        d = abs(Fraction(float(x)) - exact)
        if best is None or d < best[0] or (d == best[0] and int(np.array(x).view(np.uint32)) % 2 == 0):
            best = (d, x)
    return np.float32(best[1])


def parse_tables(src: str):
    tables = {}
    for name in ("B1", "B2", "B3", "B4"):
        m = re.search(r"const\s+" + name + r"\s*:\s*\[f32;\s*(\d+)\]\s*=\s*\[(.*?)\];", src, re.S)
        if not m:
            raise SystemExit(f"{name} not found")
        n = int(m.group(1))
        lits = [t.strip() for t in m.group(2).replace("\n", " ").split(",") if t.strip()]
        if len(lits) != n:
            raise SystemExit(f"{name}: {len(lits)} literals, declared {n}")
        tables[name] = lits
    return tables


def main():
    ref = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    path = os.path.join(ref, "src", "eden.rs")
    src = open(path).read()
    start = src[:src.index("const B1")].count("\n") + 1
    tables = parse_tables(src)
    out = {"source": f"src/eden.rs:{start}-{start + 29}",
           "note": "binary32 bits of each literal, rounded directly from the decimal (ties to even)"}
    for name, lits in tables.items():
        vals = [f32_nearest(x) for x in lits]
        out[name] = {"decimal": lits, "f32_bits": [f"0x{int(np.array(v).view(np.uint32)):08x}" for v in vals]}
    with open(OUT, "w") as f:
        json.dump(out, f, indent=1)
        f.write("\n")
    print(f"wrote {OUT}")


if __name__ == "__main__":
    main()
