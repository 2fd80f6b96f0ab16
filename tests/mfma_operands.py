"""MFMA operand integrity check over gfx950 assembly (test helper).

Invariant: every register of an MFMA's A or B operand tuple carries the value
the kernel's source gave that tuple. Walking back from the MFMA, each
register's value comes either from a load that wrote the whole tuple (a
global, buffer or LDS load; read-modify-writes of the register in between,
such as the decode attention's current-key insert or its value mask, keep
that origin) or from VALU instructions that built the tuple register by
register (the P pieces). A tuple whose registers mix both origins, or come
from different loads, has had part of a loaded operand overwritten before
the MFMA read it.

This catches a register-allocation error of the ROCm 7.2 compiler seen in
the decode attention's earlier source: with the P split through
v_cvt_pk_bf16_f32 and several prologue heads per wave (3-8 query heads per
kv head), two registers of the last value tile were reused as temporaries
between its load and the P.V MFMA, and the outputs were wrong on MI355X.
"""
import re

_REG = re.compile(r"\bv\[(\d+):(\d+)\]|\bv(\d+)\b")
_NO_VDST = ("global_store", "buffer_store", "ds_write", "s_", "v_cmp", "global_atomic",
            "buffer_atomic", "v_accvgpr_write", "v_readfirstlane", "v_readlane", "v_mfma")
_LOADS = ("global_load", "ds_read", "buffer_load")


def _regs(text):
    out = []
    for m in _REG.finditer(text):
        if m.group(1):
            out += list(range(int(m.group(1)), int(m.group(2)) + 1))
        else:
            out.append(int(m.group(3)))
    return out


def _parse(lines):
    insts = []
    for line in lines:
        s = line.strip()
        if not s or s.startswith((";", ".")) or s.endswith(":"):
            continue
        s = s.split(";")[0].strip()
        op, _, args = s.partition(" ")
        insts.append((op, [a.strip() for a in args.split(",")] if args.strip() else []))
    return insts


def _writes(op, ops):
    if not ops or op.startswith(_NO_VDST):
        return []
    return _regs(ops[0])


def _origin(insts, idx, reg):
    j = idx - 1
    while j >= 0:
        op, ops = insts[j]
        if reg in _writes(op, ops):
            if op.startswith(_LOADS):
                return ("load", j)
            if reg not in _regs(",".join(ops[1:])):
                return ("valu", j)
            # a read-modify-write keeps the register's origin
        j -= 1
    return ("entry", -1)


def functions(asm_text):
    """(symbol, lines) of every function in an assembly listing."""
    name, body = None, []
    for line in asm_text.splitlines():
        m = re.match(r"^(_Z\w+):", line)
        if m:
            name, body = m.group(1), []
        elif name is not None:
            body.append(line)
            if line.startswith(".Lfunc_end"):
                yield name, body
                name = None


def check_function(lines):
    """(MFMA count, [(mfma text, origins)] of operands with mixed origins)."""
    insts = _parse(lines)
    count, bad = 0, []
    for idx, (op, ops) in enumerate(insts):
        if not op.startswith("v_mfma"):
            continue
        count += 1
        for operand in ops[1:3]:
            regs = _regs(operand)
            if not regs:
                continue
            origins = [_origin(insts, idx, r) for r in regs]
            kinds = {o[0] for o in origins}
            loads = {o[1] for o in origins if o[0] == "load"}
            if ("load" in kinds and len(kinds) > 1) or len(loads) > 1:
                bad.append((op + " " + ", ".join(ops),
                            [(k, " ".join([insts[j][0]] + insts[j][1]) if j >= 0 else "")
                             for k, j in origins]))
    return count, bad
