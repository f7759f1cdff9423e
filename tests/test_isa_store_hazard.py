"""The gfx950 assembly of every kernel source: no store of more than 8 bytes is followed at once by
an instruction that overwrites its data registers.

Such a store still reads its data registers after it issues, and needs one wait state before
they are written again. The compiler inserts none for a buffer store whose offset is in an SGPR
(it treats that form as free of the hazard), and on gfx950 the key filter's 16-byte stores of
that form stored the next instruction's result in their first dword, in lanes 12..15 of each row
of 16. The kernels now use forms the compiler does protect; this scan keeps it so.

Compiles the device code only (``-S --offload-device-only``), about half a minute on 8 cores.
"""

from __future__ import annotations

import re
import shutil
import subprocess
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

import pytest

from vesper.kernels import build

STORE = re.compile(r"(buffer|global|flat|scratch)_store_(dwordx[34]|b96|b128)\s+(.*)")
DEST = re.compile(r"v_\S+\s+(?:v(\d+)\b|v\[(\d+):(\d+)\])")


def hazards(asm: str) -> tuple[int, list[str]]:
    """(stores wider than 8 bytes, those whose next instruction writes one of their data VGPRs)."""
    lines = [l.split(";")[0].strip() for l in asm.splitlines()]
    lines = [l for l in lines if l and not l.startswith(".") and not l.endswith(":")]
    wide, found = 0, []
    for i, line in enumerate(lines[:-1]):
        m = STORE.match(line)
        if not m:
            continue
        ops = [o.strip() for o in m.group(3).split(",")]
        data = ops[1] if m.group(1) != "buffer" else ops[0]
        r = re.fullmatch(r"v\[(\d+):(\d+)\]", data)
        if not r:
            continue
        lo, hi = int(r.group(1)), int(r.group(2))
        wide += 1
        d = DEST.match(lines[i + 1])
        if d:
            a = int(d.group(1) or d.group(2))
            b = int(d.group(1) or d.group(3))
            if a <= hi and b >= lo:
                found.append(f"{line}  ->  {lines[i + 1]}")
    return wide, found


def test_the_scan_finds_the_form_it_guards_against():
    bad = "buffer_store_dwordx4 v[72:75], v117, s[4:7], s33 offen\nv_mul_f32_e32 v72, v114, v80\n"
    assert hazards(bad) == (1, [bad.splitlines()[0] + "  ->  " + bad.splitlines()[1]])
    spaced = "buffer_store_dwordx4 v[72:75], v1, s[4:7], 0 offen\ns_nop 0\nv_mul_f32_e32 v72, v114, v80\n"
    assert hazards(spaced) == (1, [])
    other = "global_store_dwordx4 v[0:1], v[8:11], off\nv_mov_b32_e32 v12, 0\n"
    assert hazards(other) == (1, [])
    narrow = "buffer_store_dwordx2 v[8:9], v1, s[4:7], s3 offen\nv_mov_b32_e32 v8, 0\n"
    assert hazards(narrow) == (0, [])


@pytest.mark.skipif(shutil.which("hipcc") is None and not Path("/opt/rocm/bin/hipcc").exists(), reason="no hipcc")
def test_no_kernel_overwrites_the_data_of_a_wide_store(tmp_path):
    srcs = sorted(build.CSRC.glob("*.hip"))

    def asm_of(src: Path) -> str:
        out = tmp_path / (src.stem + ".s")
        cmd = [build.hipcc(), *build.HIP_FLAGS, "-I", str(build.CSRC), "-I", str(build.INCLUDE), "-S",
               "--offload-device-only", str(src), "-o", str(out)]
        proc = subprocess.run(cmd, capture_output=True, text=True, check=False)
        assert proc.returncode == 0, proc.stderr[-3000:]
        return out.read_text()

    with ThreadPoolExecutor(max_workers=len(srcs)) as pool:
        results = dict(zip((s.name for s in srcs), pool.map(asm_of, srcs)))
    total = 0
    for name, asm in results.items():
        wide, found = hazards(asm)
        total += wide
        assert not found, f"{name}: {len(found)} wide stores overwritten at once, e.g. {found[:3]}"
    assert total > 0  # the scan saw the kernels' stores
