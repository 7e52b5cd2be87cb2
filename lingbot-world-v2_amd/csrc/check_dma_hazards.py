"""Build check for the gfx950 assembly of the attention kernels: no LDS copy issued from inline
asm (global_load_lds_*) may read an SGPR that a VALU instruction wrote fewer than 5 wait states
before it, along any path into the copy.

The hardware needs those wait states between a VALU write of an SGPR and a vector memory
instruction that reads it (as an address base); the compiler inserts them for its own
instructions but not for the operands of inline asm, and a copy that reads a stale base faults.
The walk goes backwards from each copy over the instructions before it, each one wait state
(s_nop N: N + 1), and at a label forks into the fall-through and every branch to that label.

usage: python check_dma_hazards.py file.s ...   (exit status 1 and the sites, if any)"""
import re
import sys

WAIT = 5
BRANCH = re.compile(r"s_c?branch")


def sgprs(tok):
    tok = tok.strip()
    m = re.match(r"s\[(\d+):(\d+)\]$", tok)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.match(r"s(\d+)$", tok)
    return {int(m.group(1))} if m else set()


def valu_sgpr_writes(name, ops):
    """SGPRs a VALU instruction writes: an SGPR first operand (v_readlane, v_readfirstlane,
    v_cmp_*_e64 ...), and the carry or condition output of the ops that have one."""
    w = set()
    if ops:
        w |= sgprs(ops[0])
    if len(ops) > 1 and ("_co_" in name or "mad_u64" in name or "mad_i64" in name
                         or "div_scale" in name or "addc" in name or "subb" in name):
        w |= sgprs(ops[1])
    return w


def parse(path):
    """Functions as lists of ('label', name) / ('inst', name, ops, line)."""
    funcs, cur = [], None
    for ln, raw in enumerate(open(path), 1):
        t = raw.split(";")[0].strip()
        if not t:
            continue
        if t.endswith(":") and not t.startswith("."):
            cur = []
            funcs.append(cur)
            continue
        if cur is None:
            continue
        if t.endswith(":"):
            cur.append(("label", t[:-1]))
            continue
        if t.startswith("."):
            continue
        parts = t.split(None, 1)
        ops = [o.strip() for o in parts[1].split(",")] if len(parts) > 1 else []
        cur.append(("inst", parts[0], ops, ln))
    return funcs


def check_func(f, path):
    labels = {e[1]: i for i, e in enumerate(f) if e[0] == "label"}
    branches = {}
    for i, e in enumerate(f):
        if e[0] == "inst" and BRANCH.match(e[1]) and e[2]:
            branches.setdefault(e[2][0], []).append(i)
    bad = []

    def walk(i, budget, reads, seen):
        # instructions before index i (exclusive), with `budget` wait states left to check
        while budget > 0 and i > 0:
            i -= 1
            e = f[i]
            if e[0] == "label":
                for b in branches.get(e[1], []):
                    if (b, budget) not in seen:
                        seen.add((b, budget))
                        r = walk(b + 1, budget, reads, seen)
                        if r:
                            return r
                continue
            name, ops, ln = e[1], e[2], e[3]
            if name in ("s_branch", "s_endpgm", "s_setpc_b64"):
                return None  # no fall-through into what follows
            if name.startswith("v_") and valu_sgpr_writes(name, ops) & reads:
                return ln
            if name == "s_nop":
                budget -= int(ops[0], 0) + 1 if ops else 1
            else:
                budget -= 1
        return None

    for i, e in enumerate(f):
        if e[0] != "inst" or not e[1].startswith("global_load_lds"):
            continue
        reads = set()
        for o in e[2][1:]:
            reads |= sgprs(o)
        if not reads:
            continue
        hit = walk(i, WAIT, reads, set())
        if hit is not None:
            bad.append(f"{path}:{e[3]}: {e[1]} {', '.join(e[2])} reads an SGPR written by the VALU "
                       f"instruction at line {hit}, fewer than {WAIT} wait states before")
    return bad


def main(paths):
    bad = []
    for p in paths:
        for f in parse(p):
            bad += check_func(f, p)
    for b in bad:
        print(b)
    return 1 if bad else 0


if __name__ == "__main__":
    sys.exit(main(sys.argv[1:]))
