"""Scan AMDGPU assembly for loops that contain s_barrier and leave through an
exec-mask exit (a divergent loop).

The compiler builds such a loop when the exit of a barrier-containing loop
looks per-lane to it (a value read from LDS or through a flat pointer); the
lanes of one wave can then run different iterations around the same barrier
instance.  In the persistent layer kernel this once turned the ticket loop into
a loop that re-ran a task with a stale ticket for every lane but thread 0,
while lane 0 waited for them: a hang.

Loops and their nesting come from the compiler's block comments
("in Loop: Header=...", "Parent Loop ...", "Loop Header").
"""

from __future__ import annotations

import re
import sys

_BLOCK = re.compile(r"^(\.LBB\d+_\d+:|; %bb\.\d+:)")
_LOOP_REF = re.compile(r"(?:Parent Loop|Header=) ?(BB\d+_\d+)")
_EXEC_EXIT = re.compile(r"s_cbranch_exec(?:z|nz) \.L(BB\d+_\d+)$")


def _scan_function(lines: list[str]) -> list[tuple[str, list[str]]]:
    blocks, cur = [], None
    for line in lines:
        if _BLOCK.match(line):
            cur = {"label": line.split(":")[0], "loops": set(), "bar": 0, "exits": []}
            blocks.append(cur)
        if cur is None:
            continue
        if ";" in line:
            cur["loops"].update(_LOOP_REF.findall(line))
            if "Loop Header" in line and cur["label"].startswith(".L"):
                cur["loops"].add(cur["label"][2:])
        if "s_barrier" in line:
            cur["bar"] += 1
        m = _EXEC_EXIT.search(line)
        if m:
            cur["exits"].append(m.group(1))
    parent = {}
    for b in blocks:
        name = b["label"][2:]
        if b["label"].startswith(".L") and name in b["loops"]:
            parent[name] = [x for x in b["loops"] if x != name]

    def closure(ls):
        out, todo = set(ls), list(ls)
        while todo:
            for q in parent.get(todo.pop(), []):
                if q not in out:
                    out.add(q)
                    todo.append(q)
        return out

    for b in blocks:
        b["loops"] = closure(b["loops"])
    label_loops = {b["label"][2:]: b["loops"] for b in blocks if b["label"].startswith(".L")}
    bad = []
    for h in sorted(set().union(*[b["loops"] for b in blocks]) if blocks else set()):
        members = [b for b in blocks if h in b["loops"]]
        if not any(b["bar"] for b in members):
            continue
        outs = [t for b in members for t in b["exits"] if h not in label_loops.get(t, set())]
        if outs:
            bad.append((h, outs[:3]))
    return bad


def scan(text: str, kernel_substr: str = "") -> dict:
    """{kernel symbol: [(loop header, [exit targets])]} for every offending loop
    of the kernels whose symbol contains ``kernel_substr``."""
    report = {}
    for f in re.split(r"\n(?=_Z\S+:)", text):
        lines = f.splitlines()
        if not lines or kernel_substr not in lines[0]:
            continue
        name = lines[0].split(":")[0]
        if not name.startswith("_Z"):
            continue
        report[name] = _scan_function(lines)
    return report


if __name__ == "__main__":
    rep = scan(open(sys.argv[1]).read(), sys.argv[2] if len(sys.argv) > 2 else "")
    for k, v in rep.items():
        print(k[-70:], v)
    print("offending loops:", sum(len(v) for v in rep.values()))
