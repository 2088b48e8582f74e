"""Source checks of the HIP kernels (no GPU).

A cross-lane read (__shfl*, ds_bpermute) reads the source lane's register
only when that lane is active.  Written as one arm of a conditional
expression, or behind && / ||, C++ evaluates it only in the lanes where the
condition holds, so the compiled ds_bpermute runs with the other lanes off
and every lane reading from one of them gets 0.  One such read in the
hierarchical pack kernel turned every position into a hit at slot 0: wrong
outputs in the repair and a read through a null pointer (a GPU fault) in
the exact path.  The rule since: every cross-lane read runs in all lanes and
the condition is applied to its result.  This test rejects the forms that
break the rule, wherever they appear in csrc/.
"""
import re
from pathlib import Path

CSRC = Path(__file__).resolve().parents[1] / "strict-topk-overlap_amd" / "csrc"
XLANE = r"(?:__shfl(?:_xor|_up|_down)?|__builtin_amdgcn_ds_bpermute|__builtin_amdgcn_ds_permute)\s*\("
CONDITIONAL = [
    re.compile(r"\?\s*\(*\s*" + XLANE),          # cond ? shfl(...) : x
    re.compile(r"[^:]:\s*\(*\s*" + XLANE),      # cond ? x : shfl(...)   (not '::')
    re.compile(r"(?:&&|\|\|)\s*\(*\s*" + XLANE),  # a && shfl(...)
    # if (cond) x = shfl(...);   (a one-statement branch)
    re.compile(r"\bif\s*\((?:[^()]|\([^()]*\))*\)\s*[^;{}]*" + XLANE),
]


def _code(text):
    """The text with comments and string literals blanked (lines kept)."""
    text = re.sub(r"/\*.*?\*/", lambda m: re.sub(r"[^\n]", " ", m.group(0)), text, flags=re.S)
    text = re.sub(r"//[^\n]*", "", text)
    return re.sub(r'"(?:\\.|[^"\\])*"', '""', text)


def test_sources_are_present():
    files = sorted(CSRC.glob("*.hip")) + sorted(CSRC.glob("*.hpp"))
    assert len(files) > 20
    assert any(re.search(XLANE, _code(f.read_text())) for f in files)


def test_no_cross_lane_read_under_a_lane_condition():
    bad = []
    for f in sorted(CSRC.glob("*.hip")) + sorted(CSRC.glob("*.hpp")):
        code = _code(f.read_text())
        # join continued expressions: a conditional's arm may start a line
        flat = re.sub(r"\s*\n\s*", " ", code)
        for pat in CONDITIONAL:
            for m in pat.finditer(flat):
                bad.append(f"{f.name}: ...{flat[max(0, m.start() - 60):m.end() + 20]}...")
    assert not bad, "cross-lane reads evaluated only in some lanes:\n" + "\n".join(bad)


def test_the_check_catches_the_faulting_form():
    """The form that faulted is caught (a planted copy, checked in memory)."""
    planted = "const int slot = inr ? __shfl(sl, i * PB + j) : -1;\n" \
              "x = ok && __shfl_xor(v, 1) > 0;\n" \
              "y = c ? 0 : __builtin_amdgcn_ds_bpermute(a, b);\n" \
              "if (lane < 16) z = __shfl(z, 3);\n"
    flat = re.sub(r"\s*\n\s*", " ", _code(planted))
    hits = sum(len(list(p.finditer(flat))) for p in CONDITIONAL)
    assert hits == 4
    ok = "const int s0 = __shfl(sl, i * PB + j);\nconst int slot = inr ? s0 : -1;\n"
    assert not any(p.search(re.sub(r"\s*\n\s*", " ", _code(ok))) for p in CONDITIONAL)
