"""Every LDS DMA issued from inline asm reads its LDS address from M0, which
the compiler writes with an SALU instruction right before the asm statement;
gfx9 needs one wait state between the two, which the compiler inserts for its
own global_load_lds but cannot see inside an asm string.  Each asm DMA in the
HIP sources must therefore start with ``s_nop 0``."""

import re
from pathlib import Path

CSRC = Path(__file__).resolve().parents[1] / "boltz_lumi_amd" / "csrc"


def _asm_dmas():
    for src in sorted(CSRC.glob("*.hip")):
        for asm in re.findall(r'asm\s+volatile\s*\(\s*"([^"]*)"', src.read_text()):
            if "_lds" not in asm or "load" not in asm:
                continue
            lines = [s.strip() for s in asm.split("\\n") if s.strip()]
            dma = next(i for i, s in enumerate(lines) if "load" in s and "lds" in s)
            yield src.name, asm, lines, dma


def _nop_states(line):
    m = re.fullmatch(r"s_nop (\d+)", line)
    return int(m.group(1)) + 1 if m else 0


def test_every_asm_lds_dma_waits_one_state_after_m0():
    found = 0
    for name, asm, lines, dma in _asm_dmas():
        found += 1
        assert dma > 0 and _nop_states(lines[dma - 1]) >= 1, f"{name}: {asm!r}"
    assert found >= 3  # attention core, contraction, split-bf16 attention


def test_asm_lds_dma_with_sgpr_base_waits_five_states():
    """A DMA whose base address is an SGPR operand (the saddr form,
    ``global_load_lds_dwordx4 %0, %1`` with an "s" constraint) may read SGPRs
    that a VALU instruction (v_readfirstlane) wrote just before the asm; VMEM
    reads of VALU-written SGPRs need 5 wait states on gfx9, which only the asm
    itself can provide."""
    found = 0
    for src in sorted(CSRC.glob("*.hip")):
        text = src.read_text()
        for m in re.finditer(r'asm\s+volatile\s*\(\s*"([^"]*)"([^;]*);', text):
            asm, operands = m.group(1), m.group(2)
            if "_lds" not in asm or "load" not in asm or not re.search(r'"s"\s*\(', operands):
                continue
            found += 1
            lines = [s.strip() for s in asm.split("\\n") if s.strip()]
            dma = next(i for i, s in enumerate(lines) if "load" in s and "lds" in s)
            assert dma > 0 and _nop_states(lines[dma - 1]) >= 5, f"{src.name}: {asm!r}"
    assert found >= 0
