"""Writes sign_hash.json: the statement sequence of the reference's two ±1 sign
hashes, read from their source text, and the signs that sequence gives.

    rademacher_diag(seed, i)   /root/reference/src/eden.rs   (the EDEN diagonal)
    tail_rademacher(b, d)      /root/reference/src/rotate.rs (the tail fold)

Runs in the build container only: it reads the reference's source as text,
parses each function body into a list of 64-bit operations (the initial
method chain, the `x ^= x >> n` / `x = x.wrapping_mul(c)` statements, and the
final `if x & m == v { a } else { b }`), and refuses any statement of another
shape.  The fixture holds that list (constants, shifts, order, sign rule) and
the signs it produces for the (seed, i) and (block, dim) pairs the scan path
uses; it holds no source text.

    python tests/golden/make_sign_hash.py [/root/reference]
"""
import json
import os
import re
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "sign_hash.json")
MASK64 = (1 << 64) - 1

# the pairs the path evaluates: EDEN prefix (dim 64) and EdenB1 mid band
# (dim 128) diagonals at the seeds the tests and the bench use; the tail fold
# at up to 9 blocks x 64 dims (rotate.rs:73-93)
DIAG_SEEDS = (1, 7)
DIAG_LEN = 128
TAIL_BLOCKS = 9
TAIL_DIMS = 64


def function_text(src, name):
    """(parameter names, body text without comments, first line, last line)."""
    m = re.search(r"fn\s+" + name + r"\s*\(([^)]*)\)\s*->\s*f32\s*\{", src)
    if not m:
        raise SystemExit(f"fn {name} not found")
    params = [p.split(":")[0].strip() for p in m.group(1).split(",") if p.strip()]
    depth, i = 1, m.end()
    while depth:
        c = src[i]
        depth += (c == "{") - (c == "}")
        i += 1
    body = src[m.end():i - 1]
    first = src[:m.start()].count("\n") + 1
    last = src[:i].count("\n") + 1
    body = "\n".join(line.split("//")[0] for line in body.splitlines())
    return params, body, first, last


def parse_operand(tok, params):
    tok = tok.strip()
    lit = re.fullmatch(r"(0x[0-9A-Fa-f_]+|\d[\d_]*)(u64)?", tok)
    if lit:
        return {"const": f"0x{int(lit.group(1).replace('_', ''), 0):016x}"}
    arg = re.fullmatch(r"\(?\s*(\w+)\s+as\s+u64\s*\)?", tok)
    if arg and arg.group(1) in params:
        return {"arg": params.index(arg.group(1))}
    if tok in params:
        return {"arg": params.index(tok)}
    raise SystemExit(f"operand not understood: {tok!r}")


def parse_chain(expr, params, var):
    """`atom(.wrapping_mul(o)|.wrapping_add(o))*` -> ops; the atom is an
    argument (start) or the hash variable (continue)."""
    expr = re.sub(r"\s+", " ", expr).strip()
    m = re.match(r"(\(\s*\w+\s+as\s+u64\s*\)|\w+)", expr)
    if not m:
        raise SystemExit(f"chain not understood: {expr!r}")
    ops = []
    atom = m.group(1)
    if atom == var:
        pass
    else:
        ops.append({"op": "load", **parse_operand(atom, params)})
    rest = expr[m.end():]
    for call in re.finditer(r"\s*\.\s*wrapping_(mul|add)\s*\(([^()]*)\)", rest):
        ops.append({"op": call.group(1), **parse_operand(call.group(2), params)})
    consumed = "".join(c.group(0) for c in re.finditer(r"\s*\.\s*wrapping_(mul|add)\s*\(([^()]*)\)", rest))
    if consumed.replace(" ", "") != rest.replace(" ", ""):
        raise SystemExit(f"chain not fully understood: {expr!r}")
    return ops


def parse_function(src, name):
    params, body, first, last = function_text(src, name)
    parts = [p.strip() for p in body.split(";")]
    *stmts, tail = parts
    m = re.fullmatch(r"let\s+mut\s+(\w+)\s*=\s*(.*)", stmts[0], re.S)
    if not m:
        raise SystemExit(f"{name}: first statement not understood: {stmts[0]!r}")
    var = m.group(1)
    ops = parse_chain(m.group(2), params, var)
    for s in stmts[1:]:
        s1 = re.sub(r"\s+", " ", s).strip()
        xs = re.fullmatch(rf"{var} \^= {var} >> (\d+)", s1)
        if xs:
            ops.append({"op": "xor_shr", "n": int(xs.group(1))})
            continue
        asg = re.fullmatch(rf"{var} = (.*)", s1)
        if asg:
            ops.extend(parse_chain(asg.group(1), params, var))
            continue
        raise SystemExit(f"{name}: statement not understood: {s1!r}")
    t = re.sub(r"\s+", " ", tail).strip()
    cond = re.fullmatch(rf"if {var} & (\w+) == (\w+) \{{ (-?[\d.]+) \}} else \{{ (-?[\d.]+) \}}", t)
    if not cond:
        raise SystemExit(f"{name}: result expression not understood: {t!r}")
    sign = {"mask": int(cond.group(1), 0), "equals": int(cond.group(2), 0),
            "then": float(cond.group(3)), "else": float(cond.group(4))}
    return {"params": params, "lines": [first, last], "ops": ops, "sign": sign}


def evaluate(fn, args):
    """Runs a parsed function's operations in 64-bit wrapping arithmetic."""
    x = 0
    for op in fn["ops"]:
        o = op["op"]
        if o == "xor_shr":
            x ^= x >> op["n"]
            continue
        v = int(op["const"], 16) if "const" in op else args[op["arg"]]
        if o == "load":
            x = v & MASK64
        elif o == "mul":
            x = (x * v) & MASK64
        elif o == "add":
            x = (x + v) & MASK64
        else:
            raise ValueError(o)
    s = fn["sign"]
    return s["then"] if (x & s["mask"]) == s["equals"] else s["else"]


def signs(fn, a, n):
    return "".join("+" if evaluate(fn, (a, i)) > 0 else "-" for i in range(n))


def main():
    ref = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    eden = open(os.path.join(ref, "src", "eden.rs")).read()
    rot = open(os.path.join(ref, "src", "rotate.rs")).read()
    diag = parse_function(eden, "rademacher_diag")
    tail = parse_function(rot, "tail_rademacher")
    out = {
        "source": {"rademacher_diag": "src/eden.rs:%d-%d" % tuple(diag["lines"]),
                   "tail_rademacher": "src/rotate.rs:%d-%d" % tuple(tail["lines"])},
        "note": ("operations parsed from the reference's function bodies, applied in order to a 64-bit "
                 "register with wrapping arithmetic; 'load' takes an argument, 'mul'/'add' a constant or an "
                 "argument, 'xor_shr' is x ^= x >> n; the result is sign.then when (x & mask) == equals, "
                 "else sign.else. values: '+' for +1.0, '-' for -1.0, index = the second argument"),
        "functions": {"rademacher_diag": diag, "tail_rademacher": tail},
        "values": {
            "rademacher_diag": {str(s): signs(diag, s, DIAG_LEN) for s in DIAG_SEEDS},
            "tail_rademacher": [signs(tail, b, TAIL_DIMS) for b in range(TAIL_BLOCKS)],
        },
    }
    with open(OUT, "w") as f:
        json.dump(out, f, indent=1)
        f.write("\n")
    print(f"wrote {OUT}")


if __name__ == "__main__":
    main()
