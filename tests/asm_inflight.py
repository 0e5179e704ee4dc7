"""Checker for the kernels' untracked loads, over their gfx950 assembly.

The sip and gulp kernels issue their payload loads as inline-asm buffer
loads that the compiler does not track, and complete them with explicit
`s_waitcnt vmcnt(N)` where the data is used. That is sound only while the
register allocator leaves a load's destination registers alone until the
wait: a spill, copy or reuse of such a register in between reads stale data,
and the load's late write then lands on whatever the compiler put there.

`analyse(asm)` walks a kernel's control-flow graph with, per block, the
loads that may still be in flight (loads retire in issue order;
`s_waitcnt vmcnt(N)` retires all but the newest N) and reports every
instruction that reads or writes one of their destination registers. The
walk is path-sensitive in the 64-bit scalar constants (`s_mov_b64 X, -1|0`)
that the compiler uses to steer `s_cbranch_vccnz`, and treats
`s_cbranch_execz` as never taken and `s_cbranch_execnz` as always taken
where exec is known to be full (outside every `saveexec` region: the
kernels run whole waves), so the branches of a wave-uniform if/else of two
load variants are not mixed.
"""

from __future__ import annotations

import re
from collections import defaultdict

_CAP = 64
_VMEM = ("buffer_", "global_", "scratch_", "flat_")
_NO_SDEST = ("s_cbranch", "s_branch", "s_waitcnt", "s_nop", "s_cmp", "s_bitcmp", "s_setprio", "s_barrier",
             "s_sleep", "s_endpgm")


def _vregs(tok: str) -> list[str]:
    m = re.match(r"v\[(\d+):(\d+)\]", tok)
    if m:
        return [f"v{k}" for k in range(int(m.group(1)), int(m.group(2)) + 1)]
    return [tok] if re.match(r"v\d+$", tok) else []


def _sregs(tok: str) -> set[int]:
    m = re.match(r"s\[(\d+):(\d+)\]", tok)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.match(r"s(\d+)$", tok)
    return {int(m.group(1))} if m else set()


def _blocks(text: str) -> list[tuple[str, list[str]]]:
    out, cur, label = [], [], "entry"
    for line in text.splitlines():
        ln = line.split(";")[0].strip()
        if not ln or (ln.startswith(".") and not ln.endswith(":")):
            continue
        if ln.endswith(":"):
            if cur or label:
                out.append((label, cur))
            cur, label = [], ln[:-1]
            continue
        cur.append(ln)
        if ln.startswith(("s_branch", "s_cbranch", "s_endpgm", "s_setpc")):
            out.append((label, cur))
            cur, label = [], None
    if cur or label:
        out.append((label, cur))
    return [(lab if lab else f"anon{k}", ins) for k, (lab, ins) in enumerate(out)]


def _run(blocks, k, consts, loads, issues):
    consts, loads, vcc = dict(consts), dict(loads), None
    for n, ln in enumerate(blocks[k][1]):
        t = ln.replace(",", " ").split()
        op = t[0]
        if op == "s_mov_b64" and len(t) > 2 and t[2] in ("-1", "0"):
            d = _sregs(t[1])
            for key in [key for key in consts if key != "exec" and set(key) & d]:
                consts.pop(key)
            consts[tuple(sorted(d))] = int(t[2])
        elif op == "s_andn2_b64" and t[1] == "vcc" and t[2] == "exec":
            key = tuple(sorted(_sregs(t[3])))
            vcc = (0 if consts[key] == -1 else 1) if key in consts else None
        elif op.startswith("s_") and not op.startswith(_NO_SDEST) and len(t) > 1:
            d = _sregs(t[1])
            for key in [key for key in consts if key != "exec" and set(key) & d]:
                consts.pop(key)
            if t[1].startswith("vcc"):
                vcc = None
        elif op.startswith("v_cmp") or (len(t) > 1 and t[1].startswith("vcc")):
            vcc = None
        depth = consts.get("exec", 0)
        if "saveexec" in op:
            consts["exec"] = min(depth + 1, 8)
        elif op == "s_or_b64" and len(t) > 2 and t[1] == "exec" and t[2] == "exec":
            consts["exec"] = max(depth - 1, 0)
        elif (len(t) > 1 and t[1] == "exec" and op.startswith("s_")) or op.startswith("v_cmpx"):
            consts["exec"] = max(depth, 1)
        if op.startswith("s_waitcnt"):
            m = re.search(r"vmcnt\((\d+)\)", ln)
            if m:
                loads = {x: v for x, v in loads.items() if v[0] < int(m.group(1))}
            continue
        toks = re.findall(r"v\[\d+:\d+\]|v\d+", ln)
        if issues is not None and loads:
            pend = {r: lid for lid, (_, ds) in loads.items() for r in ds}
            for tok in toks:
                for r in _vregs(tok):
                    if r in pend:
                        issues.append((blocks[k][0], n, ln, pend[r]))
        if op.startswith(_VMEM):
            # (a load to LDS, as global_load_lds_* or a buffer load with the
            # lds modifier, writes no VGPR: its first operand is its address)
            is_load = "load" in op and "lds" not in op and not re.search(r"\slds\b", ln)
            loads = {x: (min(c + 1, _CAP), ds) for x, (c, ds) in loads.items()}
            loads[(k, n)] = (0, frozenset(_vregs(toks[0])) if (is_load and toks) else frozenset())
    return consts, loads, vcc


def analyse(text: str):
    """-> (hazards, blocks reached, blocks): hazards are (block label,
    instruction index, instruction, (load block, load index))."""
    blocks = _blocks(text)
    idx = {lab: k for k, (lab, _) in enumerate(blocks)}

    def succs(k, vcc, exec_full):
        last = blocks[k][1][-1] if blocks[k][1] else ""
        nxt = [k + 1] if k + 1 < len(blocks) else []
        if last.startswith("s_branch"):
            return [idx[last.split()[1]]]
        if last.startswith("s_cbranch_execz") and exec_full:
            return nxt
        if last.startswith("s_cbranch_execnz") and exec_full:
            return [idx[last.split()[1]]]
        if last.startswith("s_cbranch_vccnz") and vcc is not None:
            return [idx[last.split()[1]]] if vcc else nxt
        if last.startswith("s_cbranch_vccz") and vcc is not None:
            return nxt if vcc else [idx[last.split()[1]]]
        if last.startswith("s_cbranch"):
            return [idx[last.split()[1]]] + nxt
        if last.startswith(("s_endpgm", "s_setpc")):
            return []
        return nxt

    def join(a, b):
        out = dict(a)
        for lid, (c, ds) in b.items():
            out[lid] = (min(out[lid][0], c), ds) if lid in out else (c, ds)
        return out

    state = defaultdict(dict)  # block -> {constants: in-flight loads}
    state[0][()] = {}
    work = [(0, ())]
    while work:
        k, ck = work.pop()
        consts, loads, vcc = _run(blocks, k, dict(ck), state[k][ck], None)
        key = tuple(sorted(consts.items(), key=repr))
        for s in succs(k, vcc, consts.get("exec", 0) == 0):
            cur = state[s].get(key)
            new = loads if cur is None else join(cur, loads)
            if cur is None or new != cur:
                state[s][key] = new
                work.append((s, key))
    hazards: list = []
    for k in state:
        for ck, loads in state[k].items():
            _run(blocks, k, dict(ck), loads, hazards)
    return sorted(set(hazards)), len(state), len(blocks)


def kernels(asm: str, pattern: str):
    """-> {mangled name: its body text} for the kernels whose name matches."""
    out = {}
    for m in re.finditer(r"^(_Z[^:\s]+):", asm, re.M):
        if re.search(pattern, m.group(1)):
            out[m.group(1)] = asm[m.end():asm.find(".Lfunc_end", m.end())]
    return out


def metadata(asm: str) -> dict:
    """-> {kernel name: {vgpr_count, sgpr_count, agpr_count, vgpr_spill_count,
    sgpr_spill_count, private_segment_fixed_size, group_segment_fixed_size}}
    from the code object's metadata block of an assembly file (one entry of
    its kernel list per kernel, the keys in any order)."""
    out = {}
    block = asm[asm.find(".amdgpu_metadata"):asm.find(".end_amdgpu_metadata")]
    for entry in re.split(r"\n  - \.", block)[1:]:
        name = re.search(r"\.name:\s+(_Z\S+)", entry)
        if not name:
            continue
        fields = {}
        for key in ("vgpr_count", "sgpr_count", "agpr_count", "vgpr_spill_count", "sgpr_spill_count",
                    "private_segment_fixed_size", "group_segment_fixed_size"):
            mm = re.search(r"(?:^|\s)\.?" + key + r":\s+(\d+)", entry)
            if mm:
                fields[key] = int(mm.group(1))
        out[name.group(1)] = fields
    return out
