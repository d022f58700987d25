"""Source check for a miscompile of this toolchain (CPU only).

hipcc of ROCm 7.2 (AMD clang 22.0) compiles ``__builtin_bit_cast(T, w[p])``, with ``w`` an
ext_vector_type such as u32x4_t, as a cast of ``w[0]`` for every ``p``: a loop over the four
words of a 16-byte chunk then reads one word four times (one ``global_load_dword`` and four
``v_dot2`` on the same register, where ``global_load_dwordx4`` and four registers were meant).
Going through a scalar (``const unsigned u = w[p]; __builtin_bit_cast(T, u)``) compiles right.
No product source may use the subscripted form.
"""
import os
import re

import pytest

from tests.test_purity import _sources, _strip

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

# __builtin_bit_cast(<type>, <name>[...] ...) with the subscript directly in the operand
_SUBSCRIPT_CAST = re.compile(r"__builtin_bit_cast\s*\(\s*[\w:<> ]+?\s*,\s*[\w.]+\s*\[")


def lint(src: str):
    code, _ = _strip(src)
    return [m.group(0) for m in _SUBSCRIPT_CAST.finditer(code)]


def test_lint_rejects_the_subscripted_form():
    assert lint("const bf16x2_t v = __builtin_bit_cast(bf16x2_t, w[p]);") != []
    assert lint("x = __builtin_bit_cast(afa::f16x2_t, r.w [i]);") != []
    assert lint("const unsigned u = w[p]; const bf16x2_t v = __builtin_bit_cast(bf16x2_t, u);") == []
    assert lint("y = __builtin_bit_cast(float, w << 16); // __builtin_bit_cast(T, w[p])") == []
    assert lint("y = __builtin_bit_cast(bf16x8_t, a);") == []


@pytest.mark.parametrize("path", _sources(), ids=os.path.basename)
def test_no_bit_cast_of_a_subscript(path):
    hits = lint(open(path).read())
    assert hits == [], f"{os.path.relpath(path, ROOT)}: {hits}"
