"""The LDS-DMA protocol of the compiled kernels, checked on their gfx950
assembly (CPU only: the sources are compiled with the library's flags to
assembly, nothing runs).

The attention core, the contraction GEMM and the split-bf16 attention copy
their stage buffers with ``global_load_lds_dwordx4`` issued from inline asm,
which the compiler cannot see into.  What makes that safe is written down in
the sources and checked here on every DMA of the compiled code:

* the DMA takes its LDS address from M0; M0 is written by a scalar (SALU)
  instruction, never by a vector one, with at least one wait state before
  the DMA (the asm's leading ``s_nop``);
* a DMA that reads its base address from SGPRs (the saddr form) has five
  wait states after any vector write of those SGPRs (``v_readfirstlane``);
  the shipped kernels use only the VGPR-address form.
The remaining rules of the protocol (an explicit ``s_waitcnt vmcnt`` by every
wave before the barrier that publishes a stage; a buffer is overwritten only
after a barrier that every wave reached with its reads of it complete) are
stated next to each kernel's stage loop.
"""

import os
import re
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
CSRC = ROOT / "boltz_lumi_amd" / "csrc"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

pytestmark = pytest.mark.skipif(not Path(HIPCC).exists(), reason="hipcc not available")


def _flags(stem):
    from boltz_lumi_amd import build

    flags = [f for f in build.FLAGS if f not in ("-fPIC",)]
    return flags + build.FILE_FLAGS.get(stem, [])


def _asm(stem, tmp_path):
    out = tmp_path / f"{stem}.s"
    cmd = [HIPCC, *_flags(stem), "--cuda-device-only", "-S", str(CSRC / f"{stem}.hip"), "-o", str(out)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    assert proc.returncode == 0, proc.stderr[-2000:]
    return out.read_text()


def _instructions(text):
    """(instruction, is_label) in program order, comments and directives dropped."""
    out = []
    for line in text.splitlines():
        s = line.split(";")[0].strip()
        if not s or s.startswith("."):
            if re.match(r"^\.LBB\S*:", line.strip()):
                out.append((line.strip(), True))
            continue
        if s.endswith(":"):
            out.append((s, True))
            continue
        out.append((s, False))
    return out


def _wait_states(ins):
    m = re.fullmatch(r"s_nop (\d+)", ins)
    return int(m.group(1)) + 1 if m else 1


def _writes(ins, reg):
    parts = ins.replace(",", " ").split()
    return len(parts) > 1 and parts[1] == reg


def _sgprs(op):
    m = re.fullmatch(r"s\[(\d+):(\d+)\]", op)
    return [f"s{i}" for i in range(int(m.group(1)), int(m.group(2)) + 1)] if m else []


@pytest.mark.parametrize("stem", ["triattn", "trimul", "pair_bias"])
def test_compiled_lds_dmas_follow_the_protocol(stem, tmp_path):
    ins = _instructions(_asm(stem, tmp_path))
    dmas = [i for i, (s, lab) in enumerate(ins) if not lab and s.startswith("global_load_lds")]
    assert dmas, f"{stem}: no LDS DMA found"
    for i in dmas:
        s = ins[i][0]
        # M0: the last writer in this block is scalar and at least one wait state back
        states, found = 0, False
        for j in range(i - 1, -1, -1):
            prev, lab = ins[j]
            if lab:
                break
            if _writes(prev, "m0"):
                assert prev.startswith("s_"), f"{stem}: M0 written by a vector instruction before {s}: {prev}"
                assert states >= 1, f"{stem}: no wait state between the M0 write and {s}"
                found = True
                break
            states += _wait_states(prev)
        assert found, f"{stem}: no M0 write in the block before {s}"
        # saddr form: no vector write of the base SGPRs within 5 wait states
        ops = s.replace(",", " ").split()
        base = _sgprs(ops[2]) if len(ops) > 2 else []
        states = 0
        for j in range(i - 1, -1, -1):
            prev, lab = ins[j]
            if lab or states >= 5:
                break
            if prev.startswith("v_") and any(_writes(prev, r) for r in base):
                pytest.fail(f"{stem}: {prev} writes the base of {s} {states} wait states before it")
            states += _wait_states(prev)
