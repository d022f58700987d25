"""The C ABI of libafa_hip.so (include/afa.h) without a GPU: the library loads, exports every
function the header declares with the ctypes signature the binding uses, and rejects invalid
arguments with the documented status codes before any device work (no compute calls here)."""
import ctypes
import math
import os
import re

import pytest

from algebraic_intelligence_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "afa.h")
DUMMY = 0x1000  # never dereferenced: every call below fails validation first


def _declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    text = re.sub(r"//[^\n]*", "", text)
    return re.findall(r"^\s*(?:const\s+)?[A-Za-z_][\w]*\s*\*?\s*([a-z_][\w]*)\s*\(", text, flags=re.M)


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(_lib.LIB_PATH):
        from algebraic_intelligence_amd import build
        build.build()
    return _lib.lib()


def test_header_declares_the_boundary():
    names = _declared()
    for n in ("afa_fwd", "afa_fwd_workspace_size", "afa_bwd", "afa_bwd_workspace_size", "asoftmax_fwd", "asoftmax_bwd",
              "octic_fwd", "octic_bwd", "ago_build_tables", "ago_rotate", "afa_status_string",
              "afa_last_hip_error", "afa_version"):
        assert n in names
    assert set(names) == set(_lib.SIGNATURES), set(names) ^ set(_lib.SIGNATURES)


def test_library_exports_every_declared_symbol(lib):
    handle = ctypes.CDLL(_lib.LIB_PATH)
    for name in _declared():
        assert hasattr(handle, name), name
    assert lib.afa_version() == 1
    assert lib.afa_last_hip_error() == 0


def test_kernel_names_unique_across_sources(lib):
    """Two sources defining the same kernel instantiation share one host handle in the library,
    and a launch can run the other source's kernel with its own grid (this is how the MFMA and
    the generic backward once collided).  The build refuses such objects; check the current ones."""
    from algebraic_intelligence_amd import build
    objs = sorted(os.path.join(build.BUILD, "obj", f) for f in os.listdir(os.path.join(build.BUILD, "obj"))
                  if f.endswith(".o"))
    assert objs
    assert build.duplicate_kernels(objs) == {}


def test_status_strings(lib):
    codes = [_lib.OK, _lib.ERR_NULL, _lib.ERR_DTYPE, _lib.ERR_SHAPE, _lib.ERR_HEAD_DIM, _lib.ERR_SINK,
             _lib.ERR_VALID_LEN, _lib.ERR_EPS, _lib.ERR_ROTARY, _lib.ERR_ALIGN, _lib.ERR_WORKSPACE,
             _lib.ERR_UNSUPPORTED, _lib.ERR_GAMMA, _lib.ERR_SCRATCH_LIMIT, _lib.ERR_HIP]
    texts = [lib.afa_status_string(c).decode() for c in codes]
    assert all(texts) and len(set(texts)) == len(texts)
    assert lib.afa_status_string(12345).decode()


def _fwd(lib, dtype=_lib.AFA_BF16, B=1, H=1, L=64, D=64, q=DUMMY, out=DUMMY, rc=None, rs=None,
         rot_len=0, sink=0.5, valid=0, ws=None, ws_bytes=0):
    return lib.afa_fwd(dtype, B, H, L, D, q, DUMMY, DUMMY, None, out, None, rc, rs, rot_len, sink, 1,
                       valid, 0, ws, ws_bytes, None)


@pytest.mark.parametrize("kw,code", [
    (dict(dtype=7), _lib.ERR_DTYPE),
    (dict(dtype=-1), _lib.ERR_DTYPE),
    (dict(q=None), _lib.ERR_NULL),
    (dict(out=None), _lib.ERR_NULL),
    (dict(B=0), _lib.ERR_SHAPE),
    (dict(L=-3), _lib.ERR_SHAPE),
    (dict(D=0), _lib.ERR_SHAPE),
    (dict(D=192), _lib.ERR_HEAD_DIM),
    (dict(sink=-0.5), _lib.ERR_SINK),
    (dict(sink=math.nan), _lib.ERR_SINK),
    (dict(sink=math.inf), _lib.ERR_SINK),
    (dict(valid=65), _lib.ERR_VALID_LEN),
    (dict(valid=-1), _lib.ERR_VALID_LEN),
    (dict(rc=DUMMY), _lib.ERR_ROTARY),
    (dict(rc=DUMMY, rs=DUMMY, rot_len=63), _lib.ERR_ROTARY),
    (dict(rc=DUMMY, rs=DUMMY, rot_len=64, D=63), _lib.ERR_ROTARY),
])
def test_afa_fwd_rejects_invalid_arguments(lib, kw, code):
    assert _fwd(lib, **kw) == code


def test_afa_fwd_accumulate_arguments(lib):
    """AFA_FLAG_PARTIAL / AFA_FLAG_ACCUMULATE (one hop of src/kernels/pallas_afa.py:618-662) need
    the row-sum array and a zero sink (the sink enters only the final division) and exclude each
    other; afa_ring_finish checks its arguments as afa_fwd does.  Every case is refused before
    any device work."""
    call = lambda den, sink, fl: lib.afa_fwd(_lib.AFA_BF16, 1, 1, 64, 64, DUMMY, DUMMY, DUMMY, None, DUMMY, den,
                                             None, None, 0, sink, 0, 0, fl, None, 0, None)
    for fl in (_lib.FLAG_ACCUMULATE, _lib.FLAG_PARTIAL):
        assert call(None, 0.0, fl) == _lib.ERR_NULL
        assert call(DUMMY, 0.5, fl) == _lib.ERR_SINK
    assert call(DUMMY, 0.0, _lib.FLAG_ACCUMULATE | _lib.FLAG_PARTIAL) == _lib.ERR_UNSUPPORTED
    fin = lambda **kw: lib.afa_ring_finish(kw.get("dt", _lib.AFA_BF16), 1, 1, kw.get("L", 64), kw.get("D", 64),
                                           kw.get("acc", DUMMY), kw.get("den", DUMMY), None,
                                           kw.get("sink", 0.5), kw.get("out", DUMMY), None, None)
    assert fin(dt=9) == _lib.ERR_DTYPE
    assert fin(acc=None) == _lib.ERR_NULL
    assert fin(den=None) == _lib.ERR_NULL
    assert fin(out=None) == _lib.ERR_NULL
    assert fin(L=0) == _lib.ERR_SHAPE
    assert fin(D=192) == _lib.ERR_HEAD_DIM
    assert fin(sink=-1.0) == _lib.ERR_SINK
    # the key-shard plan never takes the fully fused kernel; its pipelined kernels' workspace is covered
    for shape in ((1, 8, 4096, 64), (16, 8, 512, 64), (3, 5, 1000, 128)):
        assert lib.afa_fwd_workspace_size(_lib.AFA_BF16, *shape, 0) > 0


def test_afa_fwd_workspace_contract(lib):
    """afa_fwd_workspace_size covers the call's largest path; a smaller caller workspace and a
    misaligned one are refused before any device work."""
    bf16 = lib.afa_fwd_workspace_size(_lib.AFA_BF16, 8, 12, 4096, 64, 0)
    bf16_rot = lib.afa_fwd_workspace_size(_lib.AFA_BF16, 8, 12, 4096, 64, 1)
    # key-norm bounds: B H ceil(L / 64) floats; the rotated k: B H L D bf16 elements more
    assert bf16 >= 8 * 12 * 64 * 4
    assert bf16_rot >= bf16 + 8 * 12 * 4096 * 64 * 2
    assert lib.afa_fwd_workspace_size(_lib.AFA_F64, 8, 12, 4096, 64, 1) == 0
    assert lib.afa_fwd_workspace_size(_lib.AFA_BF16, 0, 12, 4096, 64, 1) == 0
    assert lib.afa_fwd_workspace_size(_lib.AFA_BF16, 1, 1, 64, 192, 0) == 0
    need = lib.afa_fwd_workspace_size(_lib.AFA_BF16, 1, 1, 64, 64, 0)
    assert need > 0
    assert _fwd(lib, ws=DUMMY, ws_bytes=need - 1) == _lib.ERR_WORKSPACE
    assert _fwd(lib, ws=DUMMY + 4, ws_bytes=need) == _lib.ERR_ALIGN
    # the generic path (fp64) needs no workspace, so a zero-byte one passes validation; that call
    # would launch, so only its size is checked here
    assert lib.afa_fwd_workspace_size(_lib.AFA_F64, 1, 1, 64, 64, 0) == 0


def test_key_split_plan(lib):
    """The 128-query kernel splits a query block's keys over several workgroups only when its
    longest block exceeds the balanced load per workgroup slot by more than half (planned for a
    256-CU MI355X, the CU count the library assumes without a device): B=4 H=8 L=2048 (longest
    block 2.67 parts) splits, B=32 H=4 L=1024 (1.33 parts, faster unsplit) does not, so its
    workspace holds only the key bounds and the rotated k."""
    def base(B, H, L, D, rot):
        n = -(-B * H * -(-L // 64) * 4 // 256) * 256
        return n + (-(-B * H * L * D * 2 // 256) * 256 if rot else 0)

    assert lib.afa_fwd_workspace_size(_lib.AFA_BF16, 32, 4, 1024, 64, 1) == base(32, 4, 1024, 64, True)
    assert lib.afa_fwd_workspace_size(_lib.AFA_BF16, 4, 8, 2048, 64, 0) > base(4, 8, 2048, 64, False)


def test_afa_bwd_workspace_contract(lib):
    plain = lib.afa_bwd_workspace_size(_lib.AFA_BF16, 2, 16, 8192, 128, 0)
    rot = lib.afa_bwd_workspace_size(_lib.AFA_BF16, 2, 16, 8192, 128, 1)
    # E and 1/d per row, the fast-rho bounds of q and k; with tables the rotated q and k
    assert plain >= 2 * 16 * 8192 * 4 * 2 + 2 * 2 * 16 * 128 * 4
    assert rot >= plain + 2 * 2 * 16 * 8192 * 128 * 2
    f32 = lib.afa_bwd_workspace_size(_lib.AFA_F32, 2, 16, 8192, 128, 1)
    assert f32 == lib.afa_bwd_workspace_size(_lib.AFA_F32, 2, 16, 8192, 128, 0) >= 2 * 16 * 8192 * 4 * 2
    assert lib.afa_bwd(_lib.AFA_BF16, 1, 1, 64, 64, DUMMY, DUMMY, DUMMY, DUMMY, DUMMY, DUMMY, DUMMY, DUMMY, DUMMY,
                       None, None, 0, 0.5, 0, 0, 0, DUMMY, 16, None) == _lib.ERR_WORKSPACE


def test_afa_bwd_rejects_invalid_arguments(lib):
    def bwd(dtype=_lib.AFA_BF16, D=64, g=DUMMY, sink=0.5, valid=0):
        return lib.afa_bwd(dtype, 1, 1, 64, D, DUMMY, DUMMY, DUMMY, DUMMY, DUMMY, g, DUMMY, DUMMY, DUMMY,
                           None, None, 0, sink, 0, valid, 0, None, 0, None)
    assert bwd(dtype=9) == _lib.ERR_DTYPE
    assert bwd(g=None) == _lib.ERR_NULL
    assert bwd(D=384) == _lib.ERR_UNSUPPORTED
    assert bwd(D=200) == _lib.ERR_HEAD_DIM
    assert bwd(sink=-1.0) == _lib.ERR_SINK
    assert bwd(valid=99) == _lib.ERR_VALID_LEN
    assert lib.afa_bwd_workspace_size(_lib.AFA_BF16, 2, 16, 8192, 128, 0) > 0


def test_asoftmax_octic_ago_reject_invalid_arguments(lib):
    assert lib.asoftmax_fwd(_lib.AFA_F32, 4, 8, DUMMY, DUMMY, 0.5, 0.0, None) == _lib.ERR_EPS
    assert lib.asoftmax_fwd(_lib.AFA_F32, 4, 8, DUMMY, DUMMY, 0.5, math.inf, None) == _lib.ERR_EPS
    assert lib.asoftmax_fwd(_lib.AFA_F32, 4, 0, DUMMY, DUMMY, 0.5, 1e-5, None) == _lib.ERR_SHAPE
    assert lib.asoftmax_fwd(_lib.AFA_F32, 4, 8, DUMMY, DUMMY, math.nan, 1e-5, None) == _lib.ERR_SINK
    assert lib.asoftmax_bwd(_lib.AFA_F32, 4, 8, DUMMY, None, DUMMY, 0.5, 1e-5, None) == _lib.ERR_NULL
    assert lib.octic_fwd(11, 4, DUMMY, DUMMY, None) == _lib.ERR_DTYPE
    assert lib.octic_bwd(_lib.AFA_F32, -1, DUMMY, DUMMY, DUMMY, None) == _lib.ERR_SHAPE
    assert lib.octic_fwd_r(11, 4, DUMMY, DUMMY, DUMMY, None) == _lib.ERR_DTYPE
    assert lib.octic_fwd_r(_lib.AFA_F32, 4, DUMMY, DUMMY, None, None) == _lib.ERR_NULL
    assert lib.octic_fwd_r(_lib.AFA_F32, -1, DUMMY, DUMMY, DUMMY, None) == _lib.ERR_SHAPE
    assert lib.octic_fwd_r(_lib.AFA_F32, 0, DUMMY, DUMMY, DUMMY, None) == _lib.OK
    assert lib.ago_build_tables(_lib.AFA_BF16, 8, 16, None, 1e4, DUMMY, DUMMY, None) == _lib.ERR_DTYPE
    assert lib.ago_build_tables(_lib.AFA_F32, 7, 16, None, 1e4, DUMMY, DUMMY, None) == _lib.ERR_SHAPE
    assert lib.ago_rotate(_lib.AFA_F32, 1, 16, 1, 8, DUMMY, DUMMY, _lib.AFA_F32, DUMMY, DUMMY, 15,
                          None) == _lib.ERR_ROTARY


def test_oace_rejects_invalid_arguments(lib):
    def fwd(dtype=_lib.AFA_BF16, N=4, d=64, V=100, h=DUMMY, ldh=64, layout=0, ldw=100, t=DUMMY, eps=100.0,
            gamma=2.0, loss=DUMMY):
        return lib.oace_linear_fwd(dtype, N, d, V, h, ldh, DUMMY, layout, ldw, t, eps, gamma, loss, None, 0,
                                   None, 0, None)
    assert fwd(dtype=5) == _lib.ERR_DTYPE
    assert fwd(h=None) == _lib.ERR_NULL
    assert fwd(t=None) == _lib.ERR_NULL
    assert fwd(loss=None) == _lib.ERR_NULL
    assert fwd(N=0) == _lib.ERR_SHAPE
    assert fwd(V=-1) == _lib.ERR_SHAPE
    assert fwd(layout=2) == _lib.ERR_SHAPE
    assert fwd(ldh=63) == _lib.ERR_SHAPE
    assert fwd(ldw=99) == _lib.ERR_SHAPE
    assert fwd(layout=1, ldw=63) == _lib.ERR_SHAPE
    assert fwd(eps=-1.0) == _lib.ERR_EPS
    assert fwd(eps=math.nan) == _lib.ERR_EPS
    assert fwd(gamma=0.0) == _lib.ERR_GAMMA
    assert fwd(gamma=math.inf) == _lib.ERR_GAMMA
    # an explicit workspace smaller than required is refused before any device work
    assert lib.oace_linear_fwd(_lib.AFA_BF16, 4, 64, 100, DUMMY, 64, DUMMY, 0, 100, DUMMY, 100.0, 2.0, DUMMY,
                               None, 0, DUMMY, 16, None) == _lib.ERR_WORKSPACE
    assert lib.oace_linear_bwd(_lib.AFA_BF16, 4, 64, 100, DUMMY, 64, DUMMY, 0, 100, DUMMY, 2.0, None, None,
                               DUMMY, DUMMY, 0, None, 0, None) == _lib.ERR_NULL
    assert lib.oace_workspace_size(_lib.AFA_BF16, 512, 768, 50257, 0, 0) > 512 * 50257 * 2
    assert lib.oace_workspace_size(_lib.AFA_BF16, 0, 768, 50257, 0, 0) == 0
    assert lib.oace_softmax_loss_fwd(_lib.AFA_F32, 4, 9, DUMMY, DUMMY, 100.0, -2.0, DUMMY, None,
                                     None) == _lib.ERR_GAMMA
    assert lib.oace_softmax_loss_bwd(_lib.AFA_F32, 4, 9, DUMMY, DUMMY, 2.0, None, None, DUMMY,
                                     None) == _lib.ERR_NULL


def test_python_constants_match_the_header():
    """Every #define and enum value the Python layer copies (dtype codes, AFA and OACE flags,
    weight layouts, row record width) equals the header's."""
    from algebraic_intelligence_amd import oace
    text = open(HEADER).read()
    defs = {m.group(1): int(m.group(2), 0) for m in re.finditer(r"#define\s+(\w+)\s+(0x[0-9a-fA-F]+|\d+)u?\b", text)}
    enum = {m.group(1): int(m.group(2)) for m in re.finditer(r"\b(AFA_(?:F32|BF16|F16|F64))\s*=\s*(\d+)", text)}
    assert enum == {"AFA_F32": _lib.AFA_F32, "AFA_BF16": _lib.AFA_BF16, "AFA_F16": _lib.AFA_F16, "AFA_F64": _lib.AFA_F64}
    pairs = {
        "AFA_FLAG_EXACT_TAIL": _lib.FLAG_EXACT_TAIL, "AFA_FLAG_GENERIC": _lib.FLAG_GENERIC,
        "AFA_FLAG_EXACT_REF": _lib.FLAG_EXACT_REF, "AFA_FLAG_SIMPLE_SCHEDULE": _lib.FLAG_SIMPLE_SCHEDULE,
        "AFA_FLAG_ACCUMULATE": _lib.FLAG_ACCUMULATE, "AFA_FLAG_PARTIAL": _lib.FLAG_PARTIAL,
        "OACE_W_DV": oace.OACE_W_DV, "OACE_W_VD": oace.OACE_W_VD, "OACE_ROW_FIELDS": oace.ROW_FIELDS,
        "OACE_FLAG_WT_READY": oace.FLAG_WT_READY, "OACE_FLAG_Z_READY": oace.FLAG_Z_READY,
        "OACE_FLAG_RECOMPUTE_Z": oace.FLAG_RECOMPUTE_Z,
    }
    for name, value in pairs.items():
        assert defs[name] == value, name
    flags = [v for k, v in defs.items() if "_FLAG_" in k]
    assert len(set(flags)) == len(flags)  # every flag its own bit
