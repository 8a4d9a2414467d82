"""Rules on the library sources, checked on the CPU.

No inline assembly in the device library: an inline-asm store is invisible to
the compiler's hazard tracking (a VALU write of its data registers right after
it changed the stored bytes, which showed up as intermittently wrong rows of
the fused decode kernel).  Device code uses compiler builtins only."""

import os
import re

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(REPO, "bitnet-tt_amd", "csrc")

_ASM = re.compile(r"\b(__asm__|__asm|asm)\b\s*(volatile|__volatile__)?\s*(goto\s*)?\(")


def _strip_comments(text: str) -> str:
    text = re.sub(r"/\*.*?\*/", " ", text, flags=re.S)
    return re.sub(r"//[^\n]*", " ", text)


def test_no_inline_asm_in_library_sources():
    files = sorted(f for f in os.listdir(CSRC) if f.endswith((".hip", ".h", ".cpp", ".hpp")))
    assert files, "no sources found"
    offenders = []
    for f in files:
        with open(os.path.join(CSRC, f)) as fh:
            code = _strip_comments(fh.read())
        for m in _ASM.finditer(code):
            line = code[: m.start()].count("\n") + 1
            offenders.append(f"{f}:{line}")
    assert not offenders, f"inline assembly in the library sources: {offenders}"


def test_rule_catches_inline_asm():
    """The pattern itself: it must flag the usual spellings and ignore prose."""
    for s in ('asm volatile("s_nop 0");', '__asm__("v_mov_b32 v0, v1");', "asm (\"x\");"):
        assert _ASM.search(_strip_comments(s)), s
    for s in ("// an inline asm store", "/* asm */ int x;", "int plasma(int);"):
        assert not _ASM.search(_strip_comments(s)), s
