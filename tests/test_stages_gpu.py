"""The reference's per-kernel forward functions (gdn2_fwd.py:142-397), each
run alone on the GPU, against the oracle's restatement of the same kernel in
float64 (oracle.chunk_scores / wy_solve / recompute_wy / inter_chunk_combine,
each pinned in tests/test_oracle.py): build_chunk_scores_pallas (kernel A),
wy_solve_pallas (B), recompute_wy_pallas (C), gdn2_inter_chunk_combine and
_with_state (D).  Float32 arithmetic at chunk 64; tolerance 1e-4 (rtol = atol)
for float32 and for bfloat16 inputs (computed in float32, as the reference
upcasts; the oracle runs on the bf16-rounded inputs).  Each stage is fed the
oracle's own upstream tensors, so a stage is checked on its own, and the four
stages composed are checked against gdn2_pallas_forward."""
import numpy as np
import pytest
import torch

from oracle import gdn2_oracle as O

pytestmark = pytest.mark.gpu
BT = 64


def close(got, ref, tol=1e-4):
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    err = np.abs(got - ref) - (tol + tol * np.abs(ref))
    return float(err.max()) <= 0.0, float(np.abs(got - ref).max())


def F():
    from gdn2_package import gdn2_fwd
    return gdn2_fwd


def inputs(dev, B, T, H, D, dtype, seed, g_scale=1.0):
    xs = O.make_inputs(B, T, H, D, seed=seed, g_scale=g_scale)
    xt = [torch.tensor(x, device=dev).to(dtype) for x in xs[:5]] + \
        [torch.tensor(xs[5], device=dev)]
    xh = [x.double().cpu().numpy() for x in xt]   # what the kernels see
    return xt, xh


def chunked(xh):
    qs, ks, vs, ws, bs, gs = (O.to_chunks(x, BT) for x in xh)
    return qs, ks, vs, ws, bs, np.cumsum(gs, axis=-2)


@pytest.mark.parametrize("D,dtype,g_scale", [
    (64, torch.float32, 1.0), (128, torch.float32, 1.0), (256, torch.float32, 1.0),
    (128, torch.bfloat16, 1.0),
    (64, torch.float32, 30.0),    # strong decay: the exact diagonal-block path
])
def test_chunk_scores_match_oracle(dev, D, dtype, g_scale):
    B, T, H = 1, 256, 2
    xt, xh = inputs(dev, B, T, H, D, dtype, seed=D + 7, g_scale=g_scale)
    scale = D ** -0.5
    aqk, akk = F().build_chunk_scores_pallas(xt[0], xt[1], xt[4], xt[5], scale)
    qs, ks, _, _, bs, gc = chunked(xh)
    raqk, rakk = O.chunk_scores(qs, ks, bs, gc, scale)
    assert aqk.shape == (B, H, T // BT, BT, BT) and aqk.dtype == torch.float32
    ok_q, e_q = close(aqk.cpu().numpy(), raqk)
    ok_k, e_k = close(akk.cpu().numpy(), rakk)
    assert ok_q and ok_k, (e_q, e_k)
    # exact zeros above the diagonal (Aqk) and on and above it (Akk)
    iu = np.triu_indices(BT, 1)
    assert not aqk.cpu().numpy()[..., iu[0], iu[1]].any()
    assert not akk.cpu().numpy()[..., np.triu_indices(BT)[0], np.triu_indices(BT)[1]].any()


def test_wy_solve_matches_oracle(dev):
    """A = (I + Akk)^{-1} against the oracle's blocked substitution (pinned to
    scipy's triangular solve); entries on and above Akk's diagonal are ignored."""
    xt, xh = inputs(dev, 2, 192, 3, 128, torch.float32, seed=11)
    qs, ks, _, _, bs, gc = chunked(xh)
    _, rakk = O.chunk_scores(qs, ks, bs, gc, 128 ** -0.5)
    ref = O.wy_solve(rakk)
    akk = torch.tensor(rakk, device=dev, dtype=torch.float32)
    a = F().wy_solve_pallas(akk)
    ok, e = close(a.cpu().numpy(), ref)
    assert ok, e
    junk = akk + torch.triu(torch.randn_like(akk), 0)
    assert torch.equal(F().wy_solve_pallas(junk), a)
    # any leading shape; an identity check on a random strictly lower matrix
    L = 0.1 * torch.tril(torch.randn(5, BT, BT, device=dev, dtype=torch.float64), -1)
    inv = F().wy_solve_pallas(L.float()).double()
    eye = torch.eye(BT, device=dev, dtype=torch.float64)
    assert float((inv @ (eye + L) - eye).abs().max()) < 1e-5


@pytest.mark.parametrize("D,dtype", [(64, torch.float32), (128, torch.bfloat16),
                                     (256, torch.float32)])
def test_recompute_wy_matches_oracle(dev, D, dtype):
    """Kernel C from the oracle's A, and from a perturbed A: the given A is the
    one used (all of it, as the reference's A @ (b k e^gc))."""
    B, T, H = 1, 192, 2
    xt, xh = inputs(dev, B, T, H, D, dtype, seed=D + 3)
    qs, ks, vs, ws, bs, gc = chunked(xh)
    _, rakk = O.chunk_scores(qs, ks, bs, gc, D ** -0.5)
    A = O.wy_solve(rakk)
    A2 = A + 0.05 * np.random.default_rng(1).standard_normal(A.shape)
    for a in (A, A2):
        got = F().recompute_wy_pallas(*xt, torch.tensor(a, device=dev, dtype=torch.float32))
        ref = O.recompute_wy(qs, ks, vs, ws, bs, gc, a.astype(np.float32).astype(np.float64))
        for name, x, r in zip(("w_pseudo", "u", "kg", "qg", "gc_last"), got, ref):
            assert x.shape == r.shape and x.dtype == torch.float32, name
            ok, e = close(x.cpu().numpy(), r)
            assert ok, (name, e)


@pytest.mark.parametrize("D,h0", [(64, True), (128, False), (256, True)])
def test_combine_matches_oracle(dev, D, h0):
    """Kernel D on the oracle's tiles: o, h_final, and the per-chunk states and
    v_new of the _with_state variant."""
    B, T, H = 2, 256, 2
    xt, xh = inputs(dev, B, T, H, D, torch.float32, seed=D + 5)
    scale = D ** -0.5
    h0n = 0.2 * np.random.default_rng(2).standard_normal((B, H, D, D)) if h0 else \
        np.zeros((B, H, D, D))
    _, _, res = O.chunked_fwd(*xh, scale, h0=h0n, BT=BT, return_residuals=True)
    names = ("Aqk", "w_pseudo", "u", "kg", "qg", "gc_last")
    tiles = [torch.tensor(res[n], device=dev, dtype=torch.float32) for n in names]
    ro, rh, rhp, rvn = O.inter_chunk_combine(*(res[n] for n in names), scale, h0n)
    h0t = torch.tensor(h0n, device=dev, dtype=torch.float32) if h0 else None
    o, hf = F().gdn2_inter_chunk_combine(*tiles, scale, h0=h0t)
    o2, hf2, hp, vn = F().gdn2_inter_chunk_combine_with_state(*tiles, scale, h0=h0t)
    assert o.shape == (B, H, T // BT, BT, D) and hp.shape == (B, H, T // BT, D, D)
    for name, x, r in (("o", o, ro), ("h_final", hf, rh), ("h_pre_all", hp, rhp),
                       ("v_new_all", vn, rvn)):
        ok, e = close(x.cpu().numpy(), r)
        assert ok, (name, e)
    assert torch.equal(o, o2) and torch.equal(hf, hf2)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_stages_compose_to_the_forward(dev, dtype):
    """A -> B -> C -> D through the stage functions (gdn2_fwd.py:400-424)
    equals gdn2_pallas_forward at chunk 64 and the token recurrence."""
    B, T, H, D = 1, 320, 3, 128
    xt, xh = inputs(dev, B, T, H, D, dtype, seed=21)
    scale = D ** -0.5
    f = F()
    aqk, akk = f.build_chunk_scores_pallas(xt[0], xt[1], xt[4], xt[5], scale)
    a = f.wy_solve_pallas(akk)
    wp, u, kg, qg, gl = f.recompute_wy_pallas(*xt, a)
    o, hf = f.gdn2_inter_chunk_combine(aqk, wp, u, kg, qg, gl, scale)
    out = o.permute(0, 2, 3, 1, 4).reshape(B, T, H, D)
    ro, rh = O.recurrent_fwd(*xh, scale)
    ok_o, e_o = close(out.cpu().numpy(), ro)
    ok_h, e_h = close(hf.cpu().numpy(), rh)
    assert ok_o and ok_h, (e_o, e_h)
    xf = [x.float() for x in xt]
    fo, fh = f.gdn2_pallas_forward(*xf, scale, chunk_size=BT)
    assert float((fo - out).abs().max()) < 1e-5 and float((fh - hf).abs().max()) < 1e-5


def test_stage_errors(dev):
    f = F()
    xt, _ = inputs(dev, 1, 100, 2, 64, torch.float32, seed=1)     # T % 64 != 0
    with pytest.raises(AssertionError):
        f.build_chunk_scores_pallas(xt[0], xt[1], xt[4], xt[5], 0.125)
    with pytest.raises(AssertionError):
        f.wy_solve_pallas(torch.zeros(2, 32, 32, device=dev))
    xt, _ = inputs(dev, 1, 128, 2, 64, torch.float32, seed=1)
    with pytest.raises(AssertionError):                            # A of the wrong shape
        f.recompute_wy_pallas(*xt, torch.zeros(1, 2, 2, 64, 32, device=dev))
