"""The warp-specialized decode waits for its LDS reads with counted `s_waitcnt lgkmcnt(N)`: LDS
operations complete in order, but scalar memory loads share that counter and complete out of
order, so the counts are only right while no scalar load is in flight. The compiler may place
scalar loads (kernel arguments it reloads) anywhere; this test compiles the kernel to gfx950
assembly exactly as the library is built and checks that every scalar load is drained
(`lgkmcnt(0)`) before the next LDS operation or counted wait.

Inline-assembly statements that issue several LDS reads in a row must not give one read's
destination a register that a later read of the same statement uses as its address: the first
result may land while the later read still waits to issue. CPU only (hipcc cross-compiles).
"""
import pathlib
import re
import subprocess
import sys

import pytest

REPO = pathlib.Path(__file__).resolve().parent.parent
sys.path.insert(0, str(REPO / "qwen-mla-vllm_amd"))


def _assembly(tmp_path, source):
    import build as qbuild
    try:
        hipcc = qbuild.hipcc()
    except RuntimeError:
        pytest.skip("hipcc not available")
    extra = dict((s.name, e) for s, e in qbuild.SOURCES)[source]
    out = tmp_path / (source + ".s")
    cmd = [hipcc, *qbuild.COMMON_FLAGS, *extra, f"-I{REPO / 'include'}", f"-I{qbuild.CSRC}", "--cuda-device-only",
           "-S", str(qbuild.CSRC / source), "-o", str(out)]
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stderr[-2000:]
    return out.read_text().splitlines()


def _kernels(lines, pattern):
    starts = [i for i, l in enumerate(lines) if re.match(pattern, l)]
    for s in starts:
        e = next(i for i in range(s, len(lines)) if "s_endpgm" in lines[i])
        yield lines[s].split(":")[0], lines[s:e]


def _hazards(body):
    """(load line, LDS line, text) for every scalar load followed, along the straight-line code after
    it, by an LDS operation or a counted wait before an lgkmcnt(0). The scan follows fall-through
    only: it ends at an unconditional branch (the next line is not on that path)."""
    found = []
    for i, line in enumerate(body):
        if not re.search(r"\bs_(buffer_)?load_", line):
            continue
        for j in range(i + 1, len(body)):
            t = body[j]
            if "s_waitcnt" in t and "lgkmcnt(0)" in t:
                break
            if re.search(r"\bds_(read|write)", t) or re.search(r"lgkmcnt\([1-9]", t):
                found.append((i, j, t.strip()))
                break
            if re.match(r"\s*s_(branch|setpc_b64|endpgm)\b", t):
                break
    return found


def test_ws_scalar_loads_drained_before_lds(tmp_path):
    lines = _assembly(tmp_path, "qmla_ws.hip")
    n = 0
    for name, body in _kernels(lines, r"^_ZN4qmla2ws9ws_kernel\S*:"):
        n += 1
        hz = _hazards(body)
        assert not hz, f"{name}: scalar load in flight at an LDS operation: {hz[:3]}"
        assert any("lgkmcnt(" in l and "lgkmcnt(0)" not in l for l in body), "counted waits expected"
    assert n >= 1


def test_ro_scalar_loads_drained_before_lds(tmp_path):
    """The row-owner GLA decode counts its LDS waits the same way."""
    lines = _assembly(tmp_path, "qmla_ro.hip")
    n = 0
    for name, body in _kernels(lines, r"^_ZN4qmla2ro9ro_kernel\S*:"):
        n += 1
        hz = _hazards(body)
        assert not hz, f"{name}: scalar load in flight at an LDS operation: {hz[:3]}"
        assert any("lgkmcnt(" in l and "lgkmcnt(0)" not in l for l in body), "counted waits expected"
    assert n >= 1


def test_wsb_scalar_loads_drained_before_lds(tmp_path):
    """The bf16 warp-specialized decode counts its LDS waits the same way."""
    lines = _assembly(tmp_path, "qmla_wsb.hip")
    n = 0
    for name, body in _kernels(lines, r"^_ZN4qmla3wsb10wsb_kernel\S*:"):
        n += 1
        hz = _hazards(body)
        assert not hz, f"{name}: scalar load in flight at an LDS operation: {hz[:3]}"
        assert any("lgkmcnt(" in l and "lgkmcnt(0)" not in l for l in body), "counted waits expected"
        ov = _asm_read_overlaps(body)
        assert not ov, f"{name}: a read's destination is a later read's address: {ov[:2]}"
    assert n >= 1


def test_cs_scalar_loads_drained_before_lds(tmp_path):
    """The column-split decode (d_c 1792 and the rank-768 window) counts its LDS waits the same way;
    its inline-asm read statements keep their addresses too."""
    lines = _assembly(tmp_path, "qmla_cs.hip")
    n = 0
    for name, body in _kernels(lines, r"^_ZN4qmla2cs9cs_kernel\S*:"):
        n += 1
        hz = _hazards(body)
        assert not hz, f"{name}: scalar load in flight at an LDS operation: {hz[:3]}"
        assert any("lgkmcnt(" in l and "lgkmcnt(0)" not in l for l in body), "counted waits expected"
        ov = _asm_read_overlaps(body)
        assert not ov, f"{name}: a read's destination is a later read's address: {ov[:2]}"
    assert n >= 1


def test_hazard_check_sees_a_planted_overlap():
    body = ["s_load_dword s4, s[0:1], 0x10", "ds_read_b128 v[0:3], v4", "s_waitcnt lgkmcnt(0)"]
    assert _hazards(body)
    assert not _hazards(["s_load_dword s4, s[0:1], 0x10", "s_waitcnt lgkmcnt(0)", "ds_read_b128 v[0:3], v4"])


def _vregs(text):
    out = set()
    for m in re.finditer(r"v\[(\d+):(\d+)\]", text):
        out |= set(range(int(m.group(1)), int(m.group(2)) + 1))
    for m in re.finditer(r"\bv(\d+)\b", text):
        out.add(int(m.group(1)))
    return out


def _asm_read_overlaps(body):
    """(destination, later read) pairs inside one inline-asm statement whose registers overlap."""
    found = []
    block = None
    for line in body:
        t = line.strip()
        if t == ";;#ASMSTART":
            block = []
        elif t == ";;#ASMEND":
            reads = [x for x in (block or []) if x.startswith("ds_read")]
            for a in range(len(reads)):
                dst = _vregs(reads[a].split(None, 1)[1].split(",")[0])
                for b in range(a + 1, len(reads)):
                    if dst & _vregs(reads[b].split(None, 1)[1].split(",", 1)[1]):
                        found.append((reads[a], reads[b]))
            block = None
        elif block is not None:
            block.append(t)
    return found


def test_ws_multi_read_statements_keep_addresses(tmp_path):
    lines = _assembly(tmp_path, "qmla_ws.hip")
    for name, body in _kernels(lines, r"^_ZN4qmla2ws9ws_kernel\S*:"):
        ov = _asm_read_overlaps(body)
        assert not ov, f"{name}: a read's destination is a later read's address: {ov[:2]}"


def test_overlap_check_sees_a_planted_overlap():
    body = [";;#ASMSTART", "s_waitcnt lgkmcnt(0)", "ds_read_b32 v1, v2", "ds_read_b32 v3, v1", ";;#ASMEND"]
    assert _asm_read_overlaps(body)
    body[3] = "ds_read_b32 v3, v4"
    assert not _asm_read_overlaps(body)
