#!/usr/bin/env python3
"""Static check of the generated prefill tile loop (prefill_mx_asm.inc): every
register an instruction writes must be a declared clobber or an output of
the asm statement, so the compiler never keeps a value of its own in a
register the loop overwrites (exec, which the claim narrows to one lane,
is restored by the statement itself).  Run by the build after the
generator."""
from __future__ import annotations

import os
import re
import sys

HERE = os.path.dirname(os.path.abspath(__file__))

RESTORED = {"exec"}


def outputs(hip=os.path.join(HERE, "paged_prefill_mx.hip")):
    """Registers bound to outputs ("={...}") or read-write operands ("+{...}")
    of the asm statement, read from its operand list in the kernel source."""
    text = open(hip).read()
    out = set()
    for spec in re.findall(r'"[=+]\{([^}]+)\}"', text):
        out.update(regs(spec))
    return out


NO_DEST = ("s_waitcnt", "s_nop", "s_barrier", "s_branch", "s_cbranch", "s_cmp", "s_bitcmp",
           "ds_write", "s_endpgm", "global_store", "buffer_store")


def regs(tok: str):
    """Registers named by one operand token (v3, a[4:7], s[8:9], vcc, m0...)."""
    tok = tok.strip().rstrip(",")
    m = re.fullmatch(r"([vas])\[(\d+):(\d+)\]", tok)
    if m:
        return [f"{m.group(1)}{i}" for i in range(int(m.group(2)), int(m.group(3)) + 1)]
    m = re.fullmatch(r"([vas])(\d+)", tok)
    if m:
        return [tok]
    if tok in ("vcc", "m0", "scc", "exec"):
        return [tok]
    return []


def dests(ins: str):
    op, _, rest = ins.partition(" ")
    direct = op.startswith("buffer_load") and rest.rstrip().endswith(" lds")  # writes LDS only
    if not rest or op.endswith(":") or direct or any(op.startswith(p) for p in NO_DEST):
        out = []
    else:
        first = rest.split(",")[0]
        out = regs(first)
        if op.startswith("v_permlane32_swap"):  # swaps both operands
            out += regs(rest.split(",")[1])
    if op.startswith("v_cmp") and op.endswith("_e32") or re.match(r"v_cmp_\w+ vcc", ins):
        out += ["vcc"]
    if op.startswith("s_") and not op.startswith(("s_waitcnt", "s_nop", "s_barrier", "s_branch", "s_cbranch")):
        out += ["scc"]
    return out


def parse_inc(path):
    text = open(path).read()
    blocks = {}
    for name in ("NVS_PREFILL_MX_ASM_PAGED", "NVS_PREFILL_MX_ASM_LOCAL", "NVS_PREFILL_MX_ASM_PAGED_F16",
                 "NVS_PREFILL_MX_ASM_LOCAL_F16"):
        m = re.search(rf"#define {name} \\\n(.*?)\n  \"\"", text, re.S)
        lines = re.findall(r'"(.*?)\\n"', m.group(1))
        blocks[name] = lines
    m = re.search(r"#define NVS_PREFILL_MX_CLOBBERS (.*)", text)
    clob = set(re.findall(r'"([^"]+)"', m.group(1)))
    return blocks, clob


def check(path=os.path.join(HERE, "prefill_mx_asm.inc")):
    blocks, clob = parse_inc(path)
    allowed = clob | outputs() | RESTORED | {"scc"}  # scc: clobbered too
    bad = []
    for name, lines in blocks.items():
        for ln in lines:
            for r in dests(ln):
                if r not in allowed:
                    bad.append((name, ln, r))
    return bad


if __name__ == "__main__":
    path = sys.argv[1] if len(sys.argv) > 1 else os.path.join(HERE, "prefill_mx_asm.inc")
    bad = check(path)
    for name, ln, r in bad[:20]:
        print(f"{name}: writes undeclared {r}: {ln}")
    print(f"{len(bad)} undeclared writes")
    sys.exit(1 if bad else 0)
