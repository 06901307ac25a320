"""Package surface and host-side behaviour of the Python drop-in -- CPU only.

Mirrors the reference's tests/test_imports.py:3-12 (exports and __version__)
and its trace-time shape assertions (gdn2_fwd.py:145-146)."""
import pytest
import torch


def test_imports():
    from gdn2_package import gdn2_pallas_forward, gdn2_pallas_forward_trainable
    assert gdn2_pallas_forward_trainable is not None
    assert gdn2_pallas_forward is not None


def test_version():
    import gdn2_package
    assert hasattr(gdn2_package, "__version__")


def test_reference_constants_exist():
    from gdn2_package import gdn2_fwd
    assert gdn2_fwd.CLIP == 1e4 and gdn2_fwd.MB == 16


def _inputs(shape, dtype=torch.float32):
    return [torch.zeros(shape, dtype=dtype) for _ in range(6)]


@pytest.mark.parametrize("shape", [(1, 512, 2, 96), (1, 512, 2, 32)])
def test_shape_errors_are_assertion_errors(shape):
    import gdn2_package as gp
    with pytest.raises(AssertionError):
        gp.gdn2_pallas_forward(*_inputs(shape), 0.1)
    with pytest.raises(gp.GDN2ShapeError):
        gp.gdn2_pallas_forward(*_inputs(shape), 0.1)


@pytest.mark.parametrize("bad", [0.0, -1e3, float("nan"), float("inf"), "x"])
def test_clip_override_must_be_finite_and_positive(monkeypatch, bad):
    """CLIP (gdn2_fwd.py:33) is read at call time and may be overridden (the
    reference README's fwd.CLIP = 1e3); a bound that is not a finite positive
    number raises before anything runs, and the C ABI refuses it as well."""
    import gdn2_package as gp
    from gdn2_package import _lib, gdn2_fwd
    monkeypatch.setattr(gdn2_fwd, "CLIP", bad)
    with pytest.raises(gp.GDN2Error, match="CLIP"):
        gp.gdn2_pallas_forward(*_inputs((1, 128, 2, 64)), 0.1)
    with pytest.raises(gp.GDN2Error, match="CLIP"):
        gp.gdn2_pallas_forward_trainable(*_inputs((1, 128, 2, 64)), 0.1)
    if not isinstance(bad, str):
        assert _lib.lib().gdn2_set_clip(bad) == _lib.ERR_SHAPE


def test_chunk_256_runs_at_the_automatic_chunk(monkeypatch):
    """The reference's default BT = 256 (gdn2_fwd.py:29), passed as chunk_size
    or set as the module constant (the reference README's fwd.BT = ...), runs
    at the automatic chunk (a 256 x 256 float32 inverse does not fit a gfx950
    workgroup; results do not depend on the chunk size beyond rounding); other
    sizes reach the library's shape check."""
    import gdn2_package as gp
    from gdn2_package import gdn2_fwd
    for dt, D in ((torch.bfloat16, 64), (torch.bfloat16, 128), (torch.float32, 128)):
        assert gdn2_fwd.chunk_size_for(dt, 256, D) == gdn2_fwd.chunk_size_for(dt, None, D)
    monkeypatch.setattr(gdn2_fwd, "BT", 256)
    assert gdn2_fwd.chunk_size_for(torch.bfloat16, None, 64) == 128
    with pytest.raises(AssertionError):
        gp.gdn2_pallas_forward(*_inputs((1, 512, 2, 64)), 0.1, chunk_size=32)


def test_chunk_size_choice():
    """None picks 128 for bfloat16 inputs at D = 64 and 64 otherwise; the
    module constant BT, when set, wins over that choice (64 and 128 accepted)."""
    from gdn2_package import gdn2_fwd
    assert gdn2_fwd.chunk_size_for(torch.bfloat16, None, 64) == 128
    assert gdn2_fwd.chunk_size_for(torch.bfloat16, None, 128) == 64
    assert gdn2_fwd.chunk_size_for(torch.bfloat16, None, 256) == 64
    assert gdn2_fwd.chunk_size_for(torch.float32, None, 64) == 64
    assert gdn2_fwd.chunk_size_for(torch.bfloat16, 128, 128) == 128
    old = gdn2_fwd.BT
    try:
        gdn2_fwd.BT = 128
        assert gdn2_fwd.chunk_size_for(torch.bfloat16, None, 128) == 128
    finally:
        gdn2_fwd.BT = old


def test_mismatched_input_shapes_rejected():
    import gdn2_package as gp
    xs = _inputs((1, 128, 2, 64))
    xs[3] = torch.zeros((1, 128, 2, 32))
    with pytest.raises(gp.GDN2ShapeError):
        gp.gdn2_pallas_forward(*xs, 0.1)


def test_partial_last_chunk_passes_validation():
    """T % BT != 0 is accepted (short last chunk); the reference asserts
    (gdn2_fwd.py:146).  On host tensors the device check is what refuses."""
    import gdn2_package as gp
    with pytest.raises(gp.GDN2Error) as e:
        gp.gdn2_pallas_forward(*_inputs((1, 500, 2, 64)), 0.1)
    assert not isinstance(e.value, gp.GDN2ShapeError)


def test_bwd_workspace_d256():
    """D = 256 trains with the layout of D <= 128 (B3 is fused at every width):
    ten per-chunk float32 regions, each 256-byte aligned."""
    from gdn2_package import _lib
    al = lambda x: (x + 255) // 256 * 256
    nc, BT, D = 1 * 2 * (128 // 64), 64, 256
    tt, td, dd = BT * BT, BT * D, D * D
    per = [tt, td, dd, dd, td, td, td, td, tt, D]
    assert _lib.lib().gdn2_bwd_workspace_bytes(1, 128, 2, 256, 64, _lib.GDN2_F32) == \
        sum(al(nc * p * 4) for p in per)


def test_no_cpu_fallback():
    """Host tensors are refused: the only compute path is the gfx950 library."""
    import gdn2_package as gp
    with pytest.raises(gp.GDN2Error):
        gp.gdn2_pallas_forward(*_inputs((1, 128, 2, 64)), 0.1)


def test_chunk_size_resolution():
    from gdn2_package import gdn2_fwd
    assert gdn2_fwd.chunk_size_for(torch.bfloat16) == 64
    assert gdn2_fwd.chunk_size_for(torch.bfloat16, D=64) == 128
    assert gdn2_fwd.chunk_size_for(torch.float32) == 64
    assert gdn2_fwd.chunk_size_for(torch.bfloat16, D=256) == 64
    old = gdn2_fwd.BT
    try:
        gdn2_fwd.BT = 128             # README.md:87-92 style override, read at call time
        assert gdn2_fwd.chunk_size_for(torch.bfloat16) == 128
    finally:
        gdn2_fwd.BT = old
    import gdn2_package as gp
    with pytest.raises(gp.GDN2ShapeError):   # fp32 with a 128-token chunk is not supported
        gp.gdn2_pallas_forward(*_inputs((1, 256, 2, 64)), 0.1, chunk_size=128)


@pytest.mark.parametrize("n", [64, 128])
def test_chained_column_order(n):
    """The bfloat16 state tiles' column order (gdn2_common.h kpos): inside each
    32-block, column 16*half + 4*lg + r is stored at 8*lg + 4*half + r.  Built
    here by enumerating (half, lg, r) and compared with the view helper."""
    from gdn2_package.gdn2_fwd import _kpos_index
    expect = [0] * n
    for blk in range(0, n, 32):
        for half in range(2):
            for lg in range(4):
                for r in range(4):
                    expect[blk + 16 * half + 4 * lg + r] = blk + 8 * lg + 4 * half + r
    got = _kpos_index(n, "cpu").tolist()
    assert got == expect
    assert sorted(got) == list(range(n))
    # a lane-group's operand k positions {4lg..4lg+3} U {16+4lg..} become one 8-wide run
    for lg in range(4):
        ks = [4 * lg + r for r in range(4)] + [16 + 4 * lg + r for r in range(4)]
        assert sorted(got[k] for k in ks) == list(range(8 * lg, 8 * lg + 8))


@pytest.mark.parametrize("L", [64, 128, 256])
def test_split_pair_layout_decode(L):
    """The float32 scans' split pair layout (gdn2_common.h: per 32-element run of a
    row, bytes 16j .. 16j+15 hold bf16 hi parts of elements 4j..4j+3 and
    16+4j..16+4j+3, the lo parts 64 bytes further; lo = bf16(x - hi)).  Encoded
    here element by element from that description (round to nearest even done on
    the float32 bits) and decoded by the residual views' helper: the value is
    hi + lo, within 2^-17 of x, and a planted swap of two slots is caught."""
    import numpy as np
    from gdn2_package.gdn2_fwd import _split_decode

    def bf16_bits(x):
        u = np.asarray(x, np.float32).view(np.uint32).astype(np.uint64)
        return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)

    def bf16_val(b):
        return (b.astype(np.uint32) << 16).view(np.float32)

    rng = np.random.default_rng(7)
    x = (rng.standard_normal((3, L)) * np.exp(rng.uniform(-8, 8, (3, L)))).astype(np.float32)
    enc = np.zeros((3, L * 2), np.uint16)     # bf16 slots, L floats = 2 L halves
    for r in range(3):
        for e in range(L):
            run, i = divmod(e, 32)
            j, half, slot = (i % 16) // 4, i // 16, i % 4
            pos = run * 64 + j * 8 + half * 4 + slot          # in bf16 units
            hi = bf16_bits(x[r, e])
            lo = bf16_bits(np.float32(x[r, e] - bf16_val(hi)))
            enc[r, pos], enc[r, pos + 32] = hi, lo
    got = _split_decode(torch.from_numpy(enc.view(np.float32).copy())).numpy()
    assert np.all(np.abs(got - x) <= 2.0 ** -17 * np.abs(x))
    assert np.abs(got - x).max() > 0            # hi + lo is not float32-exact
    bad = enc.copy()
    bad[:, [1, 5]] = bad[:, [5, 1]]             # element 1 and element 17 exchanged
    wrong = _split_decode(torch.from_numpy(bad.view(np.float32).copy())).numpy()
    assert not np.all(np.abs(wrong - x) <= 2.0 ** -17 * np.abs(x))


def test_stage_diag_reports(monkeypatch, capsys):
    """GDN2_FWD_DIAG stage checks (gdn2_fwd.py:47-76): non-finite entries are
    counted with the largest finite magnitude; finite values above 1e6 are
    flagged; anything else, or the switch off, prints nothing.  The tensor
    always comes back unchanged."""
    from gdn2_package import gdn2_fwd as F
    bad = torch.tensor([1.0, float("nan"), -3.0, float("inf")])
    big = torch.tensor([[2e6, -1.0]])
    ok = torch.tensor([1.0, -5e5])
    monkeypatch.setattr(F, "_GDN2_FWD_DIAG", False)
    assert F._stage_diag("t:off", bad) is bad
    assert capsys.readouterr().out == ""
    monkeypatch.setattr(F, "_GDN2_FWD_DIAG", True)
    assert F._stage_diag("t:kernel_A_Aqk", bad) is bad
    out = capsys.readouterr().out
    assert "[GDN2-FWD-DIAG]" in out and "t:kernel_A_Aqk" in out
    assert "n_nonfinite=2" in out and "3.000e+00" in out
    F._stage_diag("t:kernel_C_u", big)
    out = capsys.readouterr().out
    assert "t:kernel_C_u" in out and "2.000e+06" in out and "non-finite" not in out
    F._stage_diag("t:kernel_C_qg", ok)
    assert capsys.readouterr().out == ""


def test_stage_functions_exist_and_refuse_other_chunks(monkeypatch):
    """The reference's per-kernel forward functions (gdn2_fwd.py:142-397) are in
    gdn2_package.gdn2_fwd; they run at chunk 64, and a module BT override to
    128 or a wrongly shaped Akk raises the shape error before anything runs."""
    import torch
    from gdn2_package import gdn2_fwd as F
    for n in ("build_chunk_scores_pallas", "wy_solve_pallas", "recompute_wy_pallas",
              "gdn2_inter_chunk_combine", "gdn2_inter_chunk_combine_with_state"):
        assert callable(getattr(F, n)), n
    with pytest.raises(AssertionError, match="ends? in|end in"):
        F.wy_solve_pallas(torch.zeros(2, 32, 32))
    monkeypatch.setattr(F, "BT", 128)
    q = _inputs((1, 128, 2, 64))
    with pytest.raises(AssertionError, match="chunk 64"):
        F.build_chunk_scores_pallas(q[0], q[1], q[4], q[5], 0.1)
    with pytest.raises(AssertionError, match="chunk 64"):
        F.wy_solve_pallas(torch.zeros(2, 64, 64))


def test_backward_stage_functions_exist_and_check_shapes(monkeypatch):
    """The reference's backward module functions (gdn2_bwd.py:32-375) are in
    gdn2_package.gdn2_bwd; wrongly shaped tiles, a module BT override and tensors
    off the ROCm device are refused before anything runs."""
    import torch
    from gdn2_package import gdn2_bwd as G, gdn2_fwd as F
    for n in ("reverse_cumsum_bwd", "gdn2_dhu_backward", "dav_backward_pallas",
              "wy_dqkg_backward_pallas", "intra_backward_pallas"):
        assert callable(getattr(G, n)), n
    t = torch.zeros(1, 2, 3, 64, 64)
    with pytest.raises(AssertionError, match="end in"):
        G.reverse_cumsum_bwd(torch.zeros(2, 32, 8), 64)
    with pytest.raises(AssertionError, match="shape"):
        G.dav_backward_pallas(torch.zeros(1, 2, 3, 64, 32), t, t)
    with pytest.raises(AssertionError, match="divisible"):
        G.intra_backward_pallas(t, t, *[torch.zeros(1, 100, 2, 64)] * 4, 0.1)
    with pytest.raises(G.GDN2Error, match="ROCm"):
        G.dav_backward_pallas(torch.zeros(1, 2, 3, 64, 64), t, t)
    monkeypatch.setattr(F, "BT", 128)
    with pytest.raises(AssertionError, match="chunk 64"):
        G.gdn2_dhu_backward(t, t, t, t, t, torch.zeros(1, 2, 3, 64), 0.1)
