"""Zero-transcendental audit of the product sources (CPU only).

The reference enforces its "no exp or any other transcendental" property by test
(tests/test_pallas_afa.py:48-71: AST and token audit of pallas_afa.py; tests/test_attention.py:77-88:
purity and exactly three squarings in the octic kernel; scripts/audit_primitives.py:17-51: the
forbidden set).  The same checks over this build's HIP sources and Python host layer:

* no call, in any C/C++ form (plain, std::, __builtin_, __builtin_amdgcn_, __ocml_, __ prefixed,
  f / l / _f32 suffixed), of a function of the reference's forbidden set or its relatives, and no
  transcendental VALU mnemonic (v_exp_*, v_log_*, v_sin_*, v_cos_*) in inline assembly;
* the device rho^8 helpers form rho^8 by exactly three squarings, rho -> rho^2 -> rho^4 -> rho^8,
  and call no builtin other than rsqrt, reciprocal, fma, fabs and bit casts (no sqrt);
* no forbidden name in the Python package (AST audit, as the reference's);
* the audit itself rejects a planted expf, exp2 builtin and v_exp_f32.
"""
import ast
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "algebraic_intelligence_amd")
CSRC = os.path.join(PKG, "csrc")

# scripts/audit_primitives.py:17-18 and tests/test_pallas_afa.py:41-44, with the inverse and
# hyperbolic relatives and the other exponential/logarithm spellings of the C libraries
FORBIDDEN = {
    "exp", "expm1", "exp2", "exp10", "log", "log1p", "log2", "log10", "logb", "sin", "cos", "tan",
    "tanh", "sinh", "cosh", "asin", "acos", "atan", "atan2", "asinh", "acosh", "atanh", "sincos",
    "sinpi", "cospi", "sigmoid", "logistic", "erf", "erfc", "erfinv", "erfcinv", "pow", "pown",
    "powr", "rootn", "lgamma", "tgamma", "softmax",
}
_PREFIX = r"(?:std::|::)?(?:__builtin_amdgcn_|__builtin_|__ocml_native_|__ocml_|__nv_|__|native_)?"
_SUFFIX = r"(?:f|l|_f16|_f32|_f64|_fast)?"
_CALL = re.compile(_PREFIX + r"(" + "|".join(sorted(FORBIDDEN, key=len, reverse=True)) + r")" + _SUFFIX
                   + r"\s*\(")
_ASM = re.compile(r"\bv_(?:exp|log|sin|cos)(?:_legacy)?_f(?:16|32|64)\b")


def _strip(src: str):
    """(code without comments and string literals, the string literals)."""
    code, strings = [], []
    i, n = 0, len(src)
    while i < n:
        if src.startswith("//", i):
            j = src.find("\n", i)
            i = n if j < 0 else j
        elif src.startswith("/*", i):
            j = src.find("*/", i + 2)
            i = n if j < 0 else j + 2
        elif src[i] == '"':
            j = i + 1
            while j < n and src[j] != '"':
                j += 2 if src[j] == "\\" else 1
            strings.append(src[i + 1:j])
            code.append('""')
            i = j + 1
        elif src[i] == "'":
            j = i + 1
            while j < n and src[j] != "'":
                j += 2 if src[j] == "\\" else 1
            code.append("' '")
            i = j + 1
        else:
            code.append(src[i])
            i += 1
    return "".join(code), strings


def audit_cxx(src: str):
    """Forbidden calls (identifier followed by '(') and transcendental mnemonics in asm strings."""
    code, strings = _strip(src)
    hits = []
    for m in re.finditer(r"(?<![\w.])([A-Za-z_][\w:]*)\s*\(", code):
        ident = m.group(1)
        if _CALL.fullmatch(ident + "("):
            hits.append(ident)
    for s in strings:
        hits.extend(_ASM.findall(s))
    return hits


def _sources():
    files = [os.path.join(CSRC, f) for f in sorted(os.listdir(CSRC)) if f.endswith((".hip", ".h", ".cpp"))]
    files.append(os.path.join(ROOT, "include", "afa.h"))
    return files


def test_audit_rejects_planted_transcendentals():
    assert audit_cxx("float f(float x) { return expf(x); }") == ["expf"]
    assert audit_cxx("y = __builtin_amdgcn_exp2f(t);") == ["__builtin_amdgcn_exp2f"]
    assert audit_cxx("y = std::log(t) + __ocml_sin_f32(u) + powf(a, b);") == ["std::log", "__ocml_sin_f32", "powf"]
    assert audit_cxx('asm volatile("v_exp_f32 %0, %1" : "=v"(y) : "v"(x));') == ["v_exp_f32"]
    assert audit_cxx("// exp(x) is never formed\nconstexpr int expo = 3; float explain(float);") == []
    assert audit_cxx('const char* s = "log(x)"; int logical = 1;') == []


@pytest.mark.parametrize("path", _sources(), ids=os.path.basename)
def test_hip_sources_have_no_transcendentals(path):
    hits = audit_cxx(open(path).read())
    assert hits == [], f"{os.path.relpath(path, ROOT)}: {hits}"


def _function_body(src: str, name: str) -> str:
    code, _ = _strip(src)
    m = re.search(r"\b" + re.escape(name) + r"\s*\([^)]*\)\s*\{", code)
    assert m, name
    depth, i = 1, m.end()
    while depth:
        depth += {"{": 1, "}": -1}.get(code[i], 0)
        i += 1
    return code[m.end():i - 1]


@pytest.mark.parametrize("path,name", [
    ("afa_common.h", "rho8_fast"), ("afa_common.h", "rho8_fast_half"), ("afa_common.h", "rho8_exact"),
    ("afa_common.h", "rho8_exact_half"), ("afa_bwd_mfma.hip", "rho8r"),
])
def test_rho8_helpers_use_three_squarings(path, name):
    """The hot rho^8 helpers: rho^2, rho^4, rho^8 by exactly three self-multiplications in a
    chain from rho, and no builtin besides rsqrt, reciprocal, fma, fabs and bit casts."""
    body = _function_body(open(os.path.join(CSRC, path)).read(), name)
    # "x = y * y;" or "return y * y;"
    squares = re.findall(r"(?:\b(\w+)\s*=|\breturn)\s*(\w+)\s*\*\s*(\w+)\s*;", body)
    squares = [(dst, a) for dst, a, b in squares if a == b]
    assert len(squares) == 3, squares
    assert [a for _, a in squares] == ["rho", squares[0][0], squares[1][0]], squares
    calls = set(re.findall(r"(__builtin_\w+)\s*\(", body))
    assert calls <= {"__builtin_amdgcn_rsqf", "__builtin_amdgcn_rcpf", "__builtin_fmaf", "__builtin_fabsf",
                     "__builtin_bit_cast"}, calls
    assert "__builtin_amdgcn_rsqf" in calls
    assert not re.search(r"\bsqrtf?\s*\(", body)


def test_python_host_layer_has_no_transcendentals():
    """AST audit of the package's Python modules (tests/test_pallas_afa.py:48-71): no attribute
    or name of the forbidden set (math.exp, torch.exp, np.log, ...)."""
    bad = []
    for f in sorted(os.listdir(PKG)):
        if not f.endswith(".py"):
            continue
        tree = ast.parse(open(os.path.join(PKG, f)).read())
        for node in ast.walk(tree):
            name = node.attr if isinstance(node, ast.Attribute) else node.id if isinstance(node, ast.Name) else None
            if name in FORBIDDEN:
                bad.append((f, node.lineno, name))
            if isinstance(node, ast.BinOp) and isinstance(node.op, ast.Pow):
                if not (isinstance(node.right, ast.Constant) and isinstance(node.right.value, int)):
                    bad.append((f, node.lineno, "non-integer power"))
    assert bad == []
