"""Every LDS DMA issued from inline asm reads its LDS address from M0, which
the compiler writes with an SALU instruction right before the asm statement;
gfx9 needs one wait state between the two, which the compiler inserts for its
own global_load_lds but cannot see inside an asm string.  Each asm DMA in the
HIP sources must therefore start with ``s_nop 0``."""

import re
from pathlib import Path

CSRC = Path(__file__).resolve().parents[1] / "boltz_lumi_amd" / "csrc"


def test_every_asm_lds_dma_waits_one_state_after_m0():
    found = 0
    for src in sorted(CSRC.glob("*.hip")):
        for asm in re.findall(r'asm\s+volatile\s*\(\s*"([^"]*)"', src.read_text()):
            if "_lds" not in asm or "load" not in asm:
                continue
            found += 1
            lines = [s.strip() for s in asm.split("\\n") if s.strip()]
            dma = next(i for i, s in enumerate(lines) if "load" in s and "lds" in s)
            assert dma > 0 and lines[dma - 1] == "s_nop 0", f"{src.name}: {asm!r}"
    assert found >= 3  # attention core, contraction, split-bf16 attention
