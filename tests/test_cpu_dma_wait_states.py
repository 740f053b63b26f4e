"""The inline-assembly global -> LDS transfers (csrc/common.h dma16 / dma16_at / dma4) keep the wait states the
hardware does not interlock, whatever the compiler's schedule: the sources that use them are compiled to gfx950
assembly here (hipcc -S, device only, the library's flags) and every `buffer_load ... lds` is checked for
  * >= 1 wait state after the last SALU write of M0 (its LDS destination), and
  * >= 5 wait states after a VALU write (v_readfirstlane / v_readlane) of any SGPR it reads (resource, offset),
counting one per instruction and N + 1 for `s_nop N`. Also under the alternative machine scheduler
`-amdgpu-sched-strategy=max-ilp`, which places instructions differently."""
import os
import re
import subprocess
from concurrent.futures import ThreadPoolExecutor

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "self_trainable_or_free_attn_amd", "csrc")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
SOURCES = ["attention.hip", "vsa_attn.hip", "vsa_rep.hip", "vsa_route.hip", "reps.hip"]


def _instructions(text):
    out = []
    for line in text.split("\n"):
        s = line.split(";")[0].strip()
        if not s or s.startswith(".") or s.endswith(":") or s.startswith("//"):
            continue
        out.append(s)
    return out


def _sgprs(tok):
    m = re.match(r"s\[(\d+):(\d+)\]$", tok)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.match(r"s(\d+)$", tok)
    return {int(m.group(1))} if m else set()


def _wait_states(inst):
    m = re.match(r"s_nop\s+(\d+)", inst)
    return int(m.group(1)) + 1 if m else 1


def violations(asm):
    """[(reason, instruction)] of the LDS-DMA instructions in `asm` that miss a wait state (a linear scan of the
    instructions before each one; control flow is not followed)."""
    insts = _instructions(asm)
    bad = []
    for i, s in enumerate(insts):
        ops = s.split()
        if not (ops[0].startswith("buffer_load") and ops[-1] == "lds"):
            continue
        reads = set()
        for tok in ops[2:4]:
            reads |= _sgprs(tok.strip(","))
        waits, m0_seen = 0, False
        for j in range(i - 1, -1, -1):
            p = insts[j].split()
            op, dst = p[0], (p[1].strip(",") if len(p) > 1 else "")
            valu_sgpr = op in ("v_readfirstlane_b32", "v_readlane_b32")
            if not m0_seen and dst == "m0":
                m0_seen = True
                need = 5 if valu_sgpr else 1
                if waits < need:
                    bad.append((f"M0 written by {op} {waits} wait states before", s))
            if valu_sgpr and waits < 5 and _sgprs(dst) & reads:
                bad.append((f"SGPR written by {op} {waits} wait states before", s))
            waits += _wait_states(insts[j])
            if waits >= 5 and (m0_seen or i - j > 400):
                break
    return bad


def _compile(src, extra):
    cmd = [HIPCC, "-O3", "-std=c++17", "--offload-arch=gfx950", "-Xclang", "-target-feature", "-Xclang",
           "-packed-fp32-ops", "--cuda-device-only", "-S", "-x", "hip", os.path.join(CSRC, src), "-o", "-", *extra]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-2000:]
    return r.stdout


def test_scanner_flags_a_missing_wait_state():
    asm = "\n".join(["s_mov_b32 m0, s4", "buffer_load_dwordx4 v1, s[8:11], s2 offen lds",
                     "v_readfirstlane_b32 s9, v3", "s_nop 2", "buffer_load_dword v1, s[8:11], s2 offen lds",
                     "v_readfirstlane_b32 s12, v3", "s_nop 4", "buffer_load_dword v1, s[12:15], s2 offen lds"])
    got = violations(asm)
    assert [r for r, _ in got] == ["M0 written by s_mov_b32 0 wait states before",
                                   "SGPR written by v_readfirstlane_b32 3 wait states before"]


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not installed")
@pytest.mark.parametrize("sched", ["default", "max-ilp"])
def test_every_lds_transfer_keeps_its_wait_states(sched):
    extra = [] if sched == "default" else ["-mllvm", f"-amdgpu-sched-strategy={sched}"]
    with ThreadPoolExecutor(max_workers=len(SOURCES)) as ex:
        asms = list(ex.map(lambda s: _compile(s, extra), SOURCES))
    total = 0
    for src, asm in zip(SOURCES, asms):
        n = sum(1 for s in _instructions(asm) if s.split()[0].startswith("buffer_load") and s.endswith(" lds"))
        total += n
        bad = violations(asm)
        assert not bad, f"{src}: {len(bad)} transfers miss wait states, e.g. {bad[:3]}"
    assert total > 300
