"""The C ABI of libgdn2_hip.so (include/gdn2.h) -- CPU only: the library loads,
exports every declared entry point, and its host-side checks reject bad input
before any launch (the calls below never reach the GPU)."""
import ctypes
import re
from pathlib import Path

import pytest

from gdn2_package import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "gdn2.h"


def declared():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(gdn2_\w+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    names = declared()
    assert "gdn2_fwd" in names and "gdn2_bwd" in names
    L = _lib.lib()
    for n in names:
        assert hasattr(L, n), n
    assert set(names) == set(_lib.SIGNATURES), "ctypes table out of sync with gdn2.h"


def test_version_and_strerror():
    import gdn2_package
    L = _lib.lib()
    assert L.gdn2_version().decode() == gdn2_package.__version__
    for code in range(0, -12, -1):
        assert L.gdn2_strerror(code) and L.gdn2_strerror(code) != b"unknown error"
    assert L.gdn2_strerror(-1234) == b"unknown error"


F32, BF16, BF16F32 = _lib.GDN2_F32, _lib.GDN2_BF16, _lib.GDN2_BF16_F32


@pytest.mark.parametrize("args,code", [
    ((1, 512, 2, 64, 64, F32, F32), _lib.OK),
    ((8, 8192, 6, 128, 128, BF16, F32), _lib.OK),
    ((8, 8192, 6, 128, 128, BF16, BF16), _lib.OK),
    ((1, 0, 2, 64, 64, F32, F32), _lib.OK),                 # empty sequence
    ((1, 512, 2, 96, 64, F32, F32), _lib.ERR_HEAD_DIM),     # ref: D==128 assert, gdn2_fwd.py:145
    ((1, 512, 2, 256, 64, F32, F32), _lib.OK),              # D = 256 (forward), chunk 64
    ((1, 512, 2, 256, 64, BF16, BF16), _lib.OK),
    ((1, 512, 2, 256, 128, BF16, F32), _lib.ERR_CHUNK),     # D = 256 needs BT = 64
    ((1, 512, 2, 512, 64, F32, F32), _lib.ERR_HEAD_DIM),
    ((1, 500, 2, 64, 64, F32, F32), _lib.ERR_SEQ_LEN),      # ref: L%BT assert, gdn2_fwd.py:146
    ((1, 512, 2, 64, 256, BF16, F32), _lib.ERR_CHUNK),
    ((1, 512, 2, 64, 128, F32, F32), _lib.ERR_CHUNK),       # fp32 needs BT=64
    ((1, 512, 2, 64, 64, 7, F32), _lib.ERR_DTYPE),
    ((1, 512, 2, 64, 64, F32, BF16), _lib.ERR_DTYPE),
    ((8, 8192, 6, 128, 64, BF16F32, F32), _lib.OK),       # bf16 data, float32 arithmetic
    ((1, 512, 2, 256, 64, BF16F32, BF16), _lib.OK),
    ((1, 512, 2, 128, 128, BF16F32, F32), _lib.ERR_CHUNK), # float32 tiles need BT=64
    ((0, 512, 2, 64, 64, F32, F32), _lib.ERR_SHAPE),
    ((1, 512, 0, 64, 64, F32, F32), _lib.ERR_SHAPE),
    ((1, -64, 2, 64, 64, F32, F32), _lib.ERR_SHAPE),
])
def test_validate(args, code):
    assert _lib.lib().gdn2_validate(*args) == code


def test_workspace_bytes():
    L = _lib.lib()
    # layout: 9 per-chunk tensors W, UT, KgT, Qg, Aqk, GL, HT, VnT, A (float32), each
    # region 256-byte aligned; the residual-keeping forward (GDN2_FWD_SAVE_A) takes all
    B, T, H, D, BT = 1, 512, 2, 64, 64
    nc = B * H * (T // BT)
    al = lambda x: (x + 255) // 256 * 256
    s = 4
    head = [nc * BT * D * s, nc * D * BT * s, nc * D * BT * s, nc * BT * D * s,
            nc * BT * BT * s, nc * D * 4]
    states = [nc * D * D * s, nc * D * BT * s]
    a_tiles = [nc * BT * BT * 4]
    exp = sum(al(x) for x in head + states + a_tiles)
    assert L.gdn2_fwd_workspace_bytes_ex(B, T, H, D, BT, F32, _lib.FWD_SAVE_A) == exp
    # float32 at D = 64: the inference scan forms the outputs itself and writes no
    # h^T / v_new^T tiles, which then take no space
    assert L.gdn2_fwd_workspace_bytes(B, T, H, D, BT, F32) == \
        sum(al(x) for x in head + a_tiles)
    # float32 at D = 128 has a separate output pass, which reads those tiles
    nc2, D2 = nc, 128
    assert L.gdn2_fwd_workspace_bytes(B, T, H, D2, BT, F32) == sum(al(x) for x in [
        nc2 * BT * D2 * s, nc2 * D2 * BT * s, nc2 * D2 * BT * s, nc2 * BT * D2 * s,
        nc2 * BT * BT * s, nc2 * D2 * 4, nc2 * D2 * D2 * s, nc2 * D2 * BT * s, nc2 * BT * BT * 4])
    # bfloat16 data with float32 arithmetic keeps float32 tiles
    assert L.gdn2_fwd_workspace_bytes_ex(B, T, H, D, BT, BF16F32, _lib.FWD_SAVE_A) == exp
    assert L.gdn2_bwd_workspace_bytes(B, T, H, D, BT, BF16F32) == \
        L.gdn2_bwd_workspace_bytes(B, T, H, D, BT, F32)
    assert L.gdn2_fwd_workspace_bytes_ex(B, T, H, D, BT, BF16, _lib.FWD_SAVE_A) < exp
    assert L.gdn2_fwd_workspace_bytes(1, 1024, 2, 64, 64, F32) > \
        L.gdn2_fwd_workspace_bytes(B, T, H, D, BT, F32)
    assert L.gdn2_fwd_workspace_bytes(1, 512, 2, 96, 64, F32) == 0
    assert L.gdn2_fwd_workspace_bytes(1, 0, 2, 64, 64, F32) == 0


def _fwd(L, dims, ptrs, h0=None, out=None, hf=None, ws=None, wsb=0, flags=0):
    return L.gdn2_fwd(None, *dims, *ptrs, h0, 0.125, out, hf, ws, wsb, flags)


def test_fwd_rejects_before_launch():
    L = _lib.lib()
    good = (1, 512, 2, 64, 64, F32, F32)
    fake = [0x100000 * (i + 1) for i in range(6)]          # never dereferenced
    ws_need = L.gdn2_fwd_workspace_bytes(*good[:6])
    # shape errors come first
    assert _fwd(L, (1, 512, 2, 96, 64, F32, F32), fake, None, 0x1000, 0x2000) == _lib.ERR_HEAD_DIM
    assert _fwd(L, (1, 500, 2, 64, 64, F32, F32), fake, None, 0x1000, 0x2000) == _lib.ERR_SEQ_LEN
    # then pointers
    assert _fwd(L, good, [None] + fake[1:], None, 0x1000, 0x2000, 0x3000, ws_need) == _lib.ERR_NULL
    assert _fwd(L, good, fake, None, 0x1000, None, 0x3000, ws_need) == _lib.ERR_NULL
    assert _fwd(L, good, [0x100008] + fake[1:], None, 0x1000, 0x2000, 0x3000, ws_need) \
        == _lib.ERR_ALIGN
    assert _fwd(L, good, fake, 0x1004, 0x1000, 0x2000, 0x3000, ws_need) == _lib.ERR_ALIGN
    # raw inputs are inference-only
    assert _fwd(L, good, fake, None, 0x1000, 0x2000, 0x3000, ws_need,
                _lib.FWD_RAW_INPUTS | _lib.FWD_SAVE_A) == _lib.ERR_FLAGS
    # a short last chunk only with GDN2_FWD_PARTIAL_CHUNK; sized as the rounded-up T
    part = (1, 500, 2, 64, 64, F32, F32)
    ws_part = L.gdn2_fwd_workspace_bytes_ex(*part[:6], _lib.FWD_PARTIAL_CHUNK)
    assert L.gdn2_fwd_workspace_bytes(*part[:6]) == 0
    assert ws_part == L.gdn2_fwd_workspace_bytes(1, 512, 2, 64, 64, F32)
    assert _fwd(L, part, fake, None, 0x1000, 0x2000, 0x3000, ws_part - 1,
                _lib.FWD_PARTIAL_CHUNK) == _lib.ERR_WORKSPACE
    assert _fwd(L, (1, 500, 2, 96, 64, F32, F32), fake, None, 0x1000, 0x2000, 0x3000,
                ws_part, _lib.FWD_PARTIAL_CHUNK) == _lib.ERR_HEAD_DIM
    # then workspace size
    assert _fwd(L, good, fake, None, 0x1000, 0x2000, 0x3000, ws_need - 1) == _lib.ERR_WORKSPACE
    assert _fwd(L, good, fake, None, 0x1000, 0x2000, None, ws_need) == _lib.ERR_NULL


def test_bwd_rejects_before_launch():
    L = _lib.lib()
    dims = (1, 512, 2, 64, 64, F32, F32)
    fake = [0x100000 * (i + 1) for i in range(6)]
    grads = [0x900000 * (i + 1) for i in range(6)]
    fws = L.gdn2_fwd_workspace_bytes(*dims[:6])
    bws = L.gdn2_bwd_workspace_bytes(*dims[:6])
    call = lambda d, dout, fwsb: L.gdn2_bwd(None, *d, *fake, None, 0.125, dout, None, *grads,
                                            0x5000, 0x6000, fwsb, 0x7000, bws)
    assert call((1, 512, 2, 96, 64, F32, F32), 0x4000, fws) == _lib.ERR_HEAD_DIM
    # D = 256: a larger backward workspace, checked before anything is launched
    assert L.gdn2_bwd_workspace_bytes(1, 512, 2, 256, 64, F32) > bws
    assert call((1, 512, 2, 256, 64, F32, F32), 0x4000, 1 << 30) == _lib.ERR_WORKSPACE
    assert call(dims, None, fws) == _lib.ERR_NULL
    assert call(dims, 0x4000, fws - 1) == _lib.ERR_WORKSPACE


def test_bwd_rejects_bf16_residuals():
    """The backward runs on float32 residuals only (GDN2_F32, GDN2_BF16_F32), as
    the reference upcasts before any arithmetic (ref gdn2_bwd.py:130-142,
    gdn2_pipeline.py:129-135): GDN2_BF16 is refused by the sizing function and
    by both backward entry points, before any pointer is looked at."""
    L = _lib.lib()
    fake = [0x100000 * (i + 1) for i in range(6)]
    grads = [0x900000 * (i + 1) for i in range(6)]
    assert L.gdn2_bwd_workspace_bytes(1, 512, 2, 64, 64, BF16) == 0
    assert L.gdn2_bwd_varlen_workspace_bytes(4, 2, 64, 64, BF16) == 0
    assert L.gdn2_bwd_workspace_bytes(1, 512, 2, 64, 64, BF16F32) > 0
    for gdt in (F32, BF16):
        assert L.gdn2_bwd(None, 1, 512, 2, 64, 64, BF16, gdt, *fake, None, 0.125, 0x4000, None,
                          *grads, 0x5000, 0x6000, 1 << 40, 0x7000, 1 << 40) == _lib.ERR_DTYPE
        assert L.gdn2_bwd_varlen(None, 2, 0x7000, 4, 2, 64, 64, BF16, gdt, *fake, None, 0.125,
                                 0x4000, None, *grads, 0x6000, 0x5000, 1 << 40, 0x7100,
                                 1 << 40) == _lib.ERR_DTYPE


def test_launch_events_hook_is_host_only():
    L = _lib.lib()
    arr = (ctypes.c_void_p * 4)()
    assert L.gdn2_set_launch_events(arr, 4) == 0
    # a rejected call consumes the request without touching the events
    assert _fwd(L, (1, 512, 2, 96, 64, F32, F32), [0] * 6) == _lib.ERR_HEAD_DIM
    assert L.gdn2_set_launch_events(None, 0) == 0


def test_segment_workspace():
    """Forward workspace with a segmented state scan: S segments add
    B*H*S*3*D*D floats (end states, transitions, entry states) and a 256-byte
    slot for the saturation flag after the per-chunk tensors.  The automatic
    choice fills 256 workgroups in the final pass: for config 5 (1 x 131072 x 8
    heads, D = 128) with bfloat16 tiles S = 8 for inference (the final pass is
    the 32-column scan with output waves) and S = 16 when the residuals are kept
    (64-column final pass), S = 8 with float32 tiles (32 columns per
    workgroup), and none for the headline shape."""
    L = _lib.lib()
    al = lambda x: (x + 255) // 256 * 256
    seg = lambda units, D: al(units * 3 * D * D * 4 + 256)
    plain = L.gdn2_fwd_workspace_bytes_ex(1, 131072, 8, 128, 128, BF16, _lib.FWD_SEGMENTS(1))
    assert L.gdn2_fwd_workspace_bytes(1, 131072, 8, 128, 128, BF16) == plain + seg(8 * 8, 128)
    saved = L.gdn2_fwd_workspace_bytes_ex(1, 131072, 8, 128, 128, BF16,
                                          _lib.FWD_SEGMENTS(1) | _lib.FWD_SAVE_A)
    assert L.gdn2_fwd_workspace_bytes_ex(1, 131072, 8, 128, 128, BF16, _lib.FWD_SAVE_A) == \
        saved + seg(8 * 16, 128)
    plain32 = L.gdn2_fwd_workspace_bytes_ex(1, 131072, 8, 128, 64, F32, _lib.FWD_SEGMENTS(1))
    assert L.gdn2_fwd_workspace_bytes(1, 131072, 8, 128, 64, F32) == plain32 + seg(8 * 8, 128)
    assert L.gdn2_fwd_workspace_bytes_ex(1, 131072, 8, 128, 128, BF16, _lib.FWD_SEGMENTS(3)) == \
        plain + seg(8 * 3, 128)
    head = L.gdn2_fwd_workspace_bytes(8, 8192, 6, 128, 128, BF16)
    assert head == L.gdn2_fwd_workspace_bytes_ex(8, 8192, 6, 128, 128, BF16, _lib.FWD_SEGMENTS(1))
    # a count above the chunk count is clamped; uneven splits leave no empty segment
    assert L.gdn2_fwd_workspace_bytes_ex(1, 640, 1, 64, 64, F32, _lib.FWD_SEGMENTS(200)) == \
        L.gdn2_fwd_workspace_bytes_ex(1, 640, 1, 64, 64, F32, _lib.FWD_SEGMENTS(10))
    base = L.gdn2_fwd_workspace_bytes_ex(1, 640, 1, 64, 64, F32, _lib.FWD_SEGMENTS(1))
    # N = 10, asked for 4: segments of 3 -> 4 segments (3, 3, 3, 1)
    assert L.gdn2_fwd_workspace_bytes_ex(1, 640, 1, 64, 64, F32, _lib.FWD_SEGMENTS(4)) == \
        base + seg(4, 64)
    # N = 10, asked for 6: segments of 2 -> 5 segments
    assert L.gdn2_fwd_workspace_bytes_ex(1, 640, 1, 64, 64, F32, _lib.FWD_SEGMENTS(6)) == \
        base + seg(5, 64)


def test_decode_rejects_before_launch():
    L = _lib.lib()
    fake = [0x100000 * (i + 1) for i in range(6)]
    call = lambda D, dt, gdt, ptrs, hin, hout, out: L.gdn2_decode(
        None, 2, 3, D, dt, gdt, *ptrs, 0.125, hin, hout, out)
    assert call(96, F32, F32, fake, None, 0x2000, 0x3000) == _lib.ERR_HEAD_DIM
    assert call(64, 7, F32, fake, None, 0x2000, 0x3000) == _lib.ERR_DTYPE
    assert call(64, F32, BF16, fake, None, 0x2000, 0x3000) == _lib.ERR_DTYPE
    assert call(64, F32, F32, [None] + fake[1:], None, 0x2000, 0x3000) == _lib.ERR_NULL
    assert call(64, F32, F32, fake, None, None, 0x3000) == _lib.ERR_NULL
    assert call(64, F32, F32, fake, 0x1004, 0x2000, 0x3000) == _lib.ERR_ALIGN
    assert L.gdn2_decode(None, 0, 3, 64, F32, F32, *fake, 0.125, None, 0x2000, 0x3000) == \
        _lib.ERR_SHAPE


def test_varlen_rejects_before_launch():
    L = _lib.lib()
    fake = [0x100000 * (i + 1) for i in range(6)]
    call = lambda nseq, total, T, flags=0, cu=0x7000, cs=0x8000, hf=0x2000: L.gdn2_fwd_varlen(
        None, nseq, cu, cs, total, T, 2, 64, 64, F32, F32, *fake, None, 0.125, 0x1000, hf,
        0x3000, 1 << 30, flags)
    assert call(0, 1, 10) == _lib.ERR_SHAPE                 # no sequences
    assert call(2, 2, 200) == _lib.ERR_SHAPE                # more tokens than chunks can hold
    assert call(2, 3, 2) == _lib.ERR_SEQ_LEN                # a chunk without tokens
    assert call(2, 2, 100, _lib.FWD_SAVE_A | _lib.FWD_RAW_INPUTS) == _lib.ERR_FLAGS
    assert call(2, 2, 100, cu=None) == _lib.ERR_NULL
    assert call(2, 2, 100, hf=None) == _lib.ERR_NULL
    # sized for either use (inference, or the residuals of GDN2_FWD_SAVE_A)
    assert L.gdn2_fwd_varlen_workspace_bytes(5, 2, 64, 64, F32) == \
        L.gdn2_fwd_workspace_bytes_ex(1, 5 * 64, 2, 64, 64, F32, _lib.FWD_SAVE_A)


def test_bwd_varlen_rejects_before_launch():
    L = _lib.lib()
    fake = [0x100000 * (i + 1) for i in range(6)]
    grads = [0x900000 * (i + 1) for i in range(6)]
    need_f = L.gdn2_fwd_varlen_workspace_bytes(4, 2, 64, 64, F32)
    need_b = L.gdn2_bwd_varlen_workspace_bytes(4, 2, 64, 64, F32)
    assert need_b == L.gdn2_bwd_workspace_bytes(1, 4 * 64, 2, 64, 64, F32) > 0
    call = lambda nseq, total, D=64, BT=64, cu=0x7000, fws=need_f, bws=need_b, dh0=0x6000: \
        L.gdn2_bwd_varlen(None, nseq, cu, total, 2, D, BT, F32, F32, *fake, None, 0.125, 0x4000,
                          None, *grads, dh0, 0x5000, fws, 0x7100, bws)
    assert call(0, 4) == _lib.ERR_SHAPE                     # no sequences
    assert call(2, -1) == _lib.ERR_SHAPE
    assert call(2, 4, D=96) == _lib.ERR_HEAD_DIM
    assert call(2, 4, D=256) == _lib.ERR_WORKSPACE          # D = 256 needs a larger one
    assert call(2, 4, BT=128) == _lib.ERR_CHUNK             # float32 needs chunk 64
    assert call(2, 4, cu=None) == _lib.ERR_NULL
    assert call(2, 4, dh0=None) == _lib.ERR_NULL
    assert call(2, 4, fws=need_f - 1) == _lib.ERR_WORKSPACE
    assert call(2, 4, bws=need_b - 1) == _lib.ERR_WORKSPACE


def test_stage_entry_points_reject_before_launch():
    """gdn2_chunk_scores / gdn2_wy_solve / gdn2_recompute_wy / gdn2_chunk_combine
    (the reference's kernels A-D one at a time): chunk 64 only, the forward's
    shape and dtype rules, then pointers and workspace, all before a launch."""
    L = _lib.lib()
    fake = [0x100000 * (i + 1) for i in range(6)]
    outs = [0x900000 * (i + 1) for i in range(5)]
    sc = lambda d, p=fake, o=outs: L.gdn2_chunk_scores(None, *d, p[0], p[1], p[4], p[5], 0.125,
                                                       o[0], o[1])
    assert sc((1, 512, 2, 64, 128, BF16, F32)) == _lib.ERR_CHUNK     # chunk 64 only
    assert sc((1, 512, 2, 96, 64, F32, F32)) == _lib.ERR_HEAD_DIM
    assert sc((1, 500, 2, 64, 64, F32, F32)) == _lib.ERR_SEQ_LEN
    assert sc((1, 512, 2, 64, 64, F32, BF16)) == _lib.ERR_DTYPE
    assert sc((1, 512, 2, 64, 64, F32, F32), o=[None] + outs[1:]) == _lib.ERR_NULL
    assert sc((1, 512, 2, 64, 64, BF16, F32), p=[0x100002] + fake[1:]) == _lib.ERR_ALIGN
    assert sc((1, 0, 2, 64, 64, F32, F32), p=[None] * 6, o=[None] * 5) == _lib.OK  # nothing to do
    assert L.gdn2_wy_solve(None, 4, 128, 0x1000, 0x2000) == _lib.ERR_CHUNK
    assert L.gdn2_wy_solve(None, -1, 64, 0x1000, 0x2000) == _lib.ERR_SHAPE
    assert L.gdn2_wy_solve(None, 1 << 31, 64, 0x1000, 0x2000) == _lib.ERR_SHAPE
    assert L.gdn2_wy_solve(None, 4, 64, None, 0x2000) == _lib.ERR_NULL
    assert L.gdn2_wy_solve(None, 0, 64, None, None) == _lib.OK
    wy = lambda d, a=0x3000: L.gdn2_recompute_wy(None, *d, *fake, a, *outs)
    assert wy((1, 512, 2, 64, 128, BF16, F32)) == _lib.ERR_CHUNK
    assert wy((1, 512, 2, 64, 64, F32, F32), a=None) == _lib.ERR_NULL
    # combine: N chunks of 64; workspace = u^T, kg^T, W (split pair layout), h^T,
    # v_new^T float32 tiles
    nc, D = 2 * 2 * 8, 64
    need = L.gdn2_chunk_combine_workspace_bytes(2, 8, 2, D, 64)
    assert need == 4 * nc * D * 64 * 4 + nc * D * D * 4
    assert L.gdn2_chunk_combine_workspace_bytes(2, 8, 2, D, 128) == 0
    assert L.gdn2_chunk_combine_workspace_bytes(2, -1, 2, D, 64) == 0
    tiles = [0x100000 * (i + 1) for i in range(6)]
    cb = lambda dims, t=tiles, hf=0x8000, wsb=need, ws=0x9000: L.gdn2_chunk_combine(
        None, *dims, *t, None, 0.125, 0x7000, hf, None, None, ws, wsb)
    assert cb((2, 8, 2, 96, 64)) == _lib.ERR_HEAD_DIM
    assert cb((2, 8, 2, D, 128)) == _lib.ERR_CHUNK
    assert cb((2, 1 << 26, 2, D, 64)) == _lib.ERR_SHAPE              # N * 64 past 31 bits
    assert cb((2, 8, 2, D, 64), t=[None] + tiles[1:]) == _lib.ERR_NULL
    assert cb((2, 8, 2, D, 64), hf=None) == _lib.ERR_NULL
    assert cb((2, 8, 2, D, 64), wsb=need - 1) == _lib.ERR_WORKSPACE
    assert cb((2, 8, 2, D, 64), ws=None) == _lib.ERR_NULL


def test_backward_stage_entry_points_reject_before_launch():
    """gdn2_bwd_dhu / _dav / _wy_dqkg / _intra / _reverse_cumsum (the reference's
    kernels B1-B5 one at a time): chunk 64, D in {64, 128, 256}, then pointers and
    the workspace (its size: the layout copies each stage makes), all before a
    launch; zero chunks return at once, except B1 whose dh0 = sanitize(dht)."""
    L = _lib.lib()
    B, N, H, D = 2, 8, 2, 64
    nc = B * H * N
    rows, sq = nc * 64 * D * 4, nc * D * D * 4
    ws = L.gdn2_bwd_stage_workspace_bytes
    assert ws(_lib.STAGE_DAV, B, N, H, D, 64) == 3 * rows
    assert ws(_lib.STAGE_DHU, B, N, H, D, 64) == 5 * rows + 2 * sq   # + W, split pair layout
    assert ws(_lib.STAGE_WY, B, N, H, D, 64) == 18 * rows + 2 * sq + nc * D * 4
    assert ws(_lib.STAGE_INTRA, B, N, H, D, 64) == 4 * rows
    assert ws(9, B, N, H, D, 64) == 0 and ws(_lib.STAGE_DAV, B, N, H, D, 128) == 0
    assert ws(_lib.STAGE_DAV, B, N, H, 96, 64) == 0
    p = [0x100000 * (i + 1) for i in range(12)]
    o = [0x900000 * (i + 1) for i in range(7)]
    need = ws(_lib.STAGE_DAV, B, N, H, D, 64)
    dav = lambda dims, a=p[0], w=0x7000000, wb=need: L.gdn2_bwd_dav(None, *dims, a, p[1], p[2],
                                                                 o[0], o[1], w, wb)
    assert dav((B, N, H, D, 128)) == _lib.ERR_CHUNK
    assert dav((B, N, H, 96, 64)) == _lib.ERR_HEAD_DIM
    assert dav((B, 1 << 26, H, D, 64)) == _lib.ERR_SHAPE
    assert dav((B, N, H, D, 64), a=None) == _lib.ERR_NULL
    assert dav((B, N, H, D, 64), wb=need - 1) == _lib.ERR_WORKSPACE
    assert dav((B, N, H, D, 64), w=None) == _lib.ERR_NULL
    assert dav((B, N, H, D, 64), w=0x7000008) == _lib.ERR_ALIGN
    assert L.gdn2_bwd_dav(None, B, 0, H, D, 64, *[None] * 6, 0) == _lib.OK
    need = ws(_lib.STAGE_DHU, B, N, H, D, 64)
    dhu = lambda dims, d0=o[1], wb=need: L.gdn2_bwd_dhu(None, *dims, *p[:6], 0.125, None, o[0],
                                                       d0, o[2], 0x7000000, wb)
    assert dhu((B, N, H, D, 128)) == _lib.ERR_CHUNK
    assert dhu((B, N, H, D, 64), d0=None) == _lib.ERR_NULL
    assert dhu((B, N, H, D, 64), wb=0) == _lib.ERR_WORKSPACE
    need = ws(_lib.STAGE_WY, B, N, H, D, 64)
    wy = lambda dims, x=p, wb=need: L.gdn2_bwd_wy_dqkg(None, *dims, *x, 0.125, *o, 0x7000000,
                                                       wb)
    assert wy((B, N, H, 128, 128)) == _lib.ERR_CHUNK
    assert wy((B, N, H, D, 64), x=p[:11] + [None]) == _lib.ERR_NULL
    assert wy((B, N, H, D, 64), wb=need - 256) == _lib.ERR_WORKSPACE
    assert L.gdn2_bwd_wy_dqkg(None, B, 0, H, D, 64, *[None] * 12, 0.1, *[None] * 8, 0) == _lib.OK
    need = ws(_lib.STAGE_INTRA, B, N, H, D, 64)
    intra = lambda T, wb=need: L.gdn2_bwd_intra(None, B, T, H, D, 64, *p[:6], 0.125, *o[:4],
                                               0x7000000, wb)
    assert intra(N * 64 - 1) == _lib.ERR_SEQ_LEN
    assert intra(-64) == _lib.ERR_SHAPE
    assert intra(N * 64, wb=need - 1) == _lib.ERR_WORKSPACE
    assert L.gdn2_bwd_intra(None, B, 0, H, D, 64, *[None] * 6, 0.1, *[None] * 5, 0) == _lib.OK
    rc = L.gdn2_bwd_reverse_cumsum
    assert rc(None, -1, 64, 128, 0x1000, 0x2000) == _lib.ERR_SHAPE
    assert rc(None, 4, 0, 128, 0x1000, 0x2000) == _lib.ERR_SHAPE
    assert rc(None, 4, 64, 128, None, 0x2000) == _lib.ERR_NULL
    assert rc(None, 4, 64, 128, 0x1002, 0x2000) == _lib.ERR_ALIGN
    assert rc(None, 0, 64, 128, None, None) == _lib.OK
