"""Static check of the grouped GEMM's asm weight loads.

The weight loads of grouped_gemm_kernel are inline-asm
`buffer_load_dwordx4 v[a:b], ...` and (MX scales) `buffer_load_ubyte v, ...`
(no `lds` modifier): the compiler does not
know they are still in flight, so nothing may read or overwrite their
destination registers until an explicit `s_waitcnt vmcnt(...)`.  This walks
every control-flow path from each such load (following branches) to the
first vmcnt wait that covers it and reports any instruction on the way that
names one of the destination registers -- a copy, a spill, an MFMA reading
it too early, or a reuse of the register.
"""
import re


def _regs(tok):
    m = re.fullmatch(r"v\[(\d+):(\d+)\]", tok)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.fullmatch(r"v(\d+)", tok)
    return {int(m.group(1))} if m else set()


_VMEM = ("buffer_", "global_", "flat_", "scratch_", "tbuffer_")
_VMCNT = re.compile(r"vmcnt\((\d+)\)")


def violations(asm_text):
    """[(kernel, line, instruction)] for every hazard found.

    vmcnt counts vector-memory instructions (loads, stores and LDS DMA alike
    on gfx9) and they complete in issue order, so `s_waitcnt vmcnt(N)` has
    landed a load once at least N vector-memory instructions were issued
    after it on the path walked; a wait with a larger N does not end the
    walk."""
    lines = [ln.split(";")[0].strip() for ln in asm_text.split("\n")]
    labels = {}
    for i, ln in enumerate(lines):
        m = re.match(r"^([.\w]+):$", ln)
        if m:
            labels[m.group(1)] = i
    bad, kern = [], None
    for i, ln in enumerate(lines):
        m = re.match(r"^(_Z\w+):$", ln)
        if m:
            kern = m.group(1)
        m = re.match(r"buffer_load_(?:dwordx4|ubyte) (v\[\d+:\d+\]|v\d+), ", ln)
        if not m or ln.endswith(" lds"):
            continue
        dst = _regs(m.group(1))
        stack, seen, found = [(i + 1, 0)], set(), False
        while stack and not found:
            j, k = stack.pop()
            while j < len(lines) and (j, k) not in seen:
                seen.add((j, k))
                t = lines[j]
                if t.startswith("s_waitcnt"):
                    w = _VMCNT.search(t)
                    if w and int(w.group(1)) <= k:
                        break
                if t.startswith("s_endpgm"):
                    bad.append((kern, i + 1, "reaches s_endpgm with the load in flight"))
                    found = True
                    break
                if t.startswith("s_branch"):
                    j = labels[t.split()[1]]
                    continue
                if t.startswith("s_cbranch"):
                    stack.append((labels[t.split()[1]], k))
                if t and not t.endswith(":") and not t.startswith("."):
                    if not (t.startswith("buffer_load_dwordx4") or t.startswith("buffer_load_ubyte")):
                        ops = re.split(r"[ ,]+", t)[1:]
                        if set().union(set(), *[_regs(o) for o in ops]) & dst:
                            bad.append((kern, j + 1, t))
                            found = True
                            break
                    if t.startswith(_VMEM):
                        k = min(k + 1, 64)
                j += 1
    return bad


def _sregs(tok):
    m = re.fullmatch(r"s\[(\d+):(\d+)\]", tok)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.fullmatch(r"s(\d+)", tok)
    return {int(m.group(1))} if m else set()


def sgpr_hazards(asm_text, states=5):
    """[(kernel, line, instruction)] for every asm weight load whose scalar
    operands (descriptor, soffset) were written by a VALU instruction
    (v_readfirstlane, v_cmp, ...) fewer than `states` wait states before it:
    the hardware needs 5, and the compiler does not pad before inline asm.
    Walks back along the fall-through path (s_nop N counts N + 1)."""
    lines = [ln.split(";")[0].strip() for ln in asm_text.split("\n")]
    bad, kern = [], None
    for i, ln in enumerate(lines):
        m = re.match(r"^(_Z\w+):$", ln)
        if m:
            kern = m.group(1)
        m = re.match(r"buffer_load_(?:dwordx4|ubyte) (?:v\[\d+:\d+\]|v\d+), v\d+, (s\[\d+:\d+\]), (s\d+) offen", ln)
        if not m:
            continue
        want = _sregs(m.group(1)) | _sregs(m.group(2))
        ws, j = 0, i - 1
        while j >= 0 and ws < states:
            t = lines[j]
            j -= 1
            if not t or t.startswith(".") or t.endswith(":") or t.startswith(";"):
                continue
            ops = re.split(r"[ ,]+", t)
            if ops[0] == "s_nop":
                ws += int(ops[1], 0) + 1
                continue
            if ops[0].startswith("v_") and len(ops) > 1 and _sregs(ops[1]) & want:
                bad.append((kern, i + 1, f"{t}  ->  {ln}"))
                break
            ws += 1
    return bad
