"""Checks, on the gfx950 assembly of this package's own HIP sources, that the
scalar-base HBM -> LDS DMAs (``global_load_lds_dword[x4] vOFF, s[a:b]``) take
their 64-bit base from wave-uniform values only.

The untracked DMA helpers in ``csrc/hip/common.hpp`` pass the tile base to
inline assembly through an ``"s"`` constraint.  If the compiler held that base
in a VGPR (a per-lane value, or one restored from a VGPR spill), it would have
to move it into SGPRs with ``v_readfirstlane``, which is only right if every
lane holds the same value.  This script follows each DMA's base SGPRs back
through the scalar instructions that computed them (a textual reaching-
definition walk, deep enough for the kernels' address arithmetic) and
classifies where each chain starts:

* a kernel-argument load (``s_load_*``) or a scalar constant,
* an SGPR that holds a dispatch value on entry (kernarg pointer, workgroup id),
* an SGPR spill restore (``v_readlane``: the SGPR was parked in one VGPR lane),
* ``v_readfirstlane`` of a VALU result: listed with the instruction that made
  that VGPR, so a reader can confirm it is uniform (the integer-division
  reciprocal estimate of a scalar, or the wave index from the thread id).

Any other VALU origin is reported as a failure, as is a kernel with DMAs and a
non-zero VGPR spill count or private segment.

Usage (compiles device code only; a few minutes per file):
    python aar-vlm_amd/check_dma_bases.py [flash_attn gemm_f32 ...]
"""
from __future__ import annotations

import collections
import re
import subprocess
import sys
import tempfile
from pathlib import Path

sys.path.insert(0, str(Path(__file__).resolve().parent))
import build  # noqa: E402

UNIFORM_READFIRSTLANE_SOURCES = ("v_cvt_u32_f32", "kernel-entry v0")
NO_DEST = ("s_cmp", "s_waitcnt", "s_barrier", "s_cbranch", "s_branch", "s_nop", "s_setprio", "s_endpgm",
           "s_bitcmp", "global_load_lds", "s_sleep", "global_store", "buffer_store", "ds_write", "s_sendmsg")


def emit_asm(stem: str, out: Path) -> None:
    src = build.HIP_DIR / f"{stem}.hip"
    flags = [f for f in build.HIP_FLAGS if f not in ("-fPIC",)] + build.HIP_FILE_FLAGS.get(stem, [])
    subprocess.run([build.HIPCC, *flags, "--cuda-device-only", "-S", "-o", str(out), str(src)], check=True,
                   stderr=subprocess.DEVNULL)


def _regs(tok: str) -> set:
    tok = tok.strip(",")
    for kind in ("s", "v"):
        m = re.match(rf"{kind}\[(\d+):(\d+)\]$", tok)
        if m:
            return {(kind, i) for i in range(int(m.group(1)), int(m.group(2)) + 1)}
        m = re.match(rf"{kind}(\d+)$", tok)
        if m:
            return {(kind, int(m.group(1)))}
    return set()


def _parse(ins: str):
    p = ins.replace(",", " ").split()
    op = p[0]
    if op.startswith(NO_DEST) or len(p) < 2:
        return op, set(), set()
    return op, _regs(p[1]), set().union(set(), *[_regs(t) for t in p[2:]])


def _functions(asm: str) -> dict[str, list[str]]:
    funcs, cur = {}, None
    for ln in asm.split("\n"):
        m = re.match(r"^([_A-Za-z][\w.$]*):", ln)
        if m:
            cur = m.group(1)
            funcs[cur] = []
            continue
        if cur and ln.startswith(".Lfunc_end"):
            cur = None
            continue
        if cur:
            s = ln.split(";")[0].strip()
            if s and not s.startswith(".") and not s.endswith(":"):
                funcs[cur].append(s)
    return funcs


def _spills(asm: str) -> dict[str, tuple[int, int]]:
    out, name = {}, None
    for ln in asm.split("\n"):
        m = re.match(r"\s+(?:-\s+)?\.name:\s+(\S+)", ln)
        if m:
            name = m.group(1)
            out[name] = [0, 0]
        m = re.match(r"\s+(?:-\s+)?\.(private_segment_fixed_size|vgpr_spill_count):\s+(\d+)", ln)
        if m and name:
            out[name][0 if m.group(1).startswith("private") else 1] = int(m.group(2))
    return {k: tuple(v) for k, v in out.items()}


def check(asm: str) -> tuple[collections.Counter, list[str]]:
    origins, failures = collections.Counter(), []
    spills = _spills(asm)
    for fname, ins in _functions(asm).items():
        parsed = [_parse(i) for i in ins]
        dmas = [k for k, i in enumerate(ins) if i.startswith("global_load_lds") and " s[" in i]
        if not dmas:
            continue
        if any(spills.get(fname, (0, 0))):
            failures.append(f"{fname}: scratch/VGPR spills {spills[fname]} in a kernel with scalar-base DMAs")
        for k in dmas:
            todo, seen = [(k, r, 0) for r in _regs(ins[k].split()[2])], set()
            while todo:
                pos, r, depth = todo.pop()
                if (pos, r) in seen or depth > 60:
                    continue
                seen.add((pos, r))
                for j in range(pos - 1, -1, -1):
                    op, dst, src = parsed[j]
                    if r not in dst:
                        continue
                    if op.startswith("s_load"):
                        origins["kernel argument (" + op + ")"] += 1
                    elif op.startswith("v_readlane"):
                        origins["SGPR spill restore (v_readlane)"] += 1
                    elif op.startswith("v_readfirstlane"):
                        v = next(iter(src), None)
                        made = next((ins[t].split()[0] for t in range(j - 1, -1, -1) if v in parsed[t][1]),
                                    f"kernel-entry v{v[1]}" if v else "?")
                        origins["v_readfirstlane of " + made] += 1
                        if not made.startswith(UNIFORM_READFIRSTLANE_SOURCES):
                            failures.append(f"{fname}: DMA base from v_readfirstlane of {made}: {ins[j]}")
                    elif op.startswith("v_"):
                        failures.append(f"{fname}: DMA base written by VALU {ins[j]}")
                    else:
                        scalar_src = [s for s in src if s[0] == "s"]
                        if not scalar_src:
                            origins["scalar constant"] += 1
                        todo.extend((j, s, depth + 1) for s in scalar_src)
                    break
                else:
                    origins["dispatch SGPR on entry (kernarg pointer, workgroup id)"] += 1
    return origins, failures


def main(stems: list[str]) -> int:
    bad = 0
    with tempfile.TemporaryDirectory() as d:
        for stem in stems:
            out = Path(d) / f"{stem}.s"
            emit_asm(stem, out)
            origins, failures = check(out.read_text())
            print(f"{stem}: base-register chain origins")
            for what, n in origins.most_common():
                print(f"  {n:6d}  {what}")
            for f in failures:
                print("  FAIL", f)
            bad += len(failures)
    print("ok" if not bad else f"{bad} failure(s)")
    return 1 if bad else 0


if __name__ == "__main__":
    sys.exit(main(sys.argv[1:] or ["flash_attn", "gemm_f32"]))
