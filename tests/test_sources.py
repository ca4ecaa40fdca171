"""Comments and docstrings of the product, the oracle and the tests stand on
their own: they name none of the build's notes files and no build round (the
notes files map the sources to the survey instead)."""

import re
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
NOTES = ("DESIGN", "SURVEY", "VERDICT", "ADVICE", "BASELINE", "INTEGRATION")
# built from parts so that this file does not match itself
NOTE_FILE = re.compile(r"\b(?:" + "|".join(NOTES) + r")\." + "md")
ROUND = re.compile(r"\b[Rr]ound[ -]?\d|\br0\d\b")


def sources():
    for d in ("boltz_lumi_amd", "include", "oracle", "tests"):
        for p in sorted((ROOT / d).rglob("*")):
            if p.suffix in (".py", ".hip", ".h") and "_build" not in p.parts and p.name != Path(__file__).name:
                yield p
    yield ROOT / "bench.py"
    yield ROOT / "__graft_entry__.py"


def comments(text, suffix):
    """Comment and docstring text of a source file."""
    if suffix == ".py":
        yield from re.findall(r"#[^\n]*", text)
        yield from re.findall(r'"""(.*?)"""', text, re.S)
    else:
        yield from re.findall(r"//[^\n]*", text)
        yield from re.findall(r"/\*(.*?)\*/", text, re.S)


def test_comments_name_no_notes_file_or_round():
    found = []
    for p in sources():
        for c in comments(p.read_text(errors="ignore"), p.suffix):
            for pat in (NOTE_FILE, ROUND):
                m = pat.search(c)
                if m:
                    found.append(f"{p.relative_to(ROOT)}: {m.group(0)!r} in {c.strip()[:80]!r}")
    assert not found, "\n".join(found)
