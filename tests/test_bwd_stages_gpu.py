"""The reference's per-kernel backward functions (gdn2_bwd.py:32-375), each run
alone on the GPU, against the oracle's restatement of the same kernel in float64
(oracle._reverse_cumsum / _dhu_backward / _dav_backward / _wy_dqkg_backward /
_intra_backward, pinned in tests/test_oracle.py through chunked_bwd against
torch.autograd of the token recurrence): reverse_cumsum_bwd (B5),
gdn2_dhu_backward (B1), dav_backward_pallas (B2), wy_dqkg_backward_pallas (B3)
and intra_backward_pallas (B4).  Each stage is fed the oracle's own upstream
tensors rounded to float32 (the oracle runs on the rounded values), so a stage
is checked on its own; the five composed after the forward stages are checked
against oracle.chunked_bwd and the fused trainable path.  Float32 arithmetic at
chunk 64; tolerance |got - ref| <= tol + tol * |ref|, tol = 1e-4, and on the
1e4 clip scale where outputs saturate."""
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


def G():
    from gdn2_package import gdn2_bwd
    return gdn2_bwd


def r32(a):
    """The float32 rounding of a float64 array, in float64."""
    return np.asarray(a, dtype=np.float32).astype(np.float64)


def dev_t(a, dev):
    return torch.tensor(np.asarray(a, dtype=np.float32), device=dev)


def case(B, T, H, D, seed, g_scale=1.0, h0=False):
    """The forward's residuals and the upstream gradients of every backward
    stage, from the oracle in float64 on float32 inputs (gdn2_pipeline.py:70-137
    order: B2, B1, B3, B4, B5)."""
    xs = O.make_inputs(B, T, H, D, seed=seed, g_scale=g_scale)
    xh = [x.astype(np.float64) for x in xs]
    rng = np.random.default_rng(seed + 1)
    h0n = 0.2 * rng.standard_normal((B, H, D, D)) if h0 else None
    scale = D ** -0.5
    _, _, res = O.chunked_fwd(*xh, scale, h0=h0n, BT=BT, return_residuals=True)
    res = {n: r32(x) for n, x in res.items()}
    qs, ks, vs, ws, bs, _, _ = O._prep(*xh, BT, np.float64)
    do = r32(rng.standard_normal((B, T, H, D)))
    dht = r32(rng.standard_normal((B, H, D, D)))
    c = dict(xs=xs, q=qs, k=ks, v=vs, w=ws, b=bs, do=O.to_chunks(do, BT), dht=dht,
             scale=scale, **res)   # res["gc"]: the in-chunk cumsum of g
    daqk, dvp = O._dav_backward(c["Aqk"], c["v_new_all"], c["do"])
    c["daqk"], c["dv_partial"] = r32(daqk), r32(dvp)
    dh_all, _, dv_all = O._dhu_backward(c["do"], c["dv_partial"], c["w_pseudo"], c["qg"],
                                        c["kg"], c["gc_last"], scale, dht)
    c["dv_all"] = r32(dv_all)
    c["dh_next"] = r32(np.concatenate([dh_all[:, :, 1:], dht[:, :, None]], axis=2))
    b3 = O._wy_dqkg_backward(qs, ks, bs, ws, vs, c["gc"], c["A"], c["h_pre_all"],
                             c["v_new_all"], c["do"], c["dv_all"], c["dh_next"], scale)
    c["dakk"] = r32(b3["dAkk"])
    return c


# ----------------------------------------------------------------------------- B5
@pytest.mark.parametrize("shape,mag", [((2, 3, 4, BT, 128), 1.0), ((3, 16, 5), 1.0),
                                       ((2, 2, 3, BT, 64), 3e3)])
def test_reverse_cumsum_matches_oracle(dev, shape, mag):
    """Any chunk length and width; with entries of 3e3 the suffix sums pass the
    1e4 clip, and a few non-finite entries map as nan_to_num does (nan -> 0,
    +-inf -> +-1e4, and everything above them in the column the same)."""
    rng = np.random.default_rng(len(shape))
    x = (rng.standard_normal(shape) * mag).astype(np.float32)
    if mag > 1:
        x[0, 0, 0, 40, 3], x[1, 1, 2, 10, 7], x[0, 1, 1, 5, 9] = np.nan, np.inf, -np.inf
    got = G().reverse_cumsum_bwd(torch.tensor(x, device=dev), shape[-2]).cpu().numpy()
    with np.errstate(invalid="ignore"):
        ref = O._reverse_cumsum(x.astype(np.float64))
    assert np.isfinite(got).all()
    if mag > 1:
        assert 0.05 < np.mean(np.abs(ref) == 1e4) < 0.9
        assert got[0, 0, 0, 0, 3] == 0.0 and got[1, 1, 2, 0, 7] == 1e4
        ok, e = close(got * 1e-4, ref * 1e-4)
    else:
        ok, e = close(got, ref)
    assert ok, e


# ----------------------------------------------------------------------------- B2
@pytest.mark.parametrize("D", [64, 128, 256])
def test_dav_matches_oracle(dev, D):
    c = case(1, 256, 2, D, seed=D + 1)
    daqk, dvn = G().dav_backward_pallas(dev_t(c["Aqk"], dev), dev_t(c["v_new_all"], dev),
                                        dev_t(c["do"], dev))
    ref_q, ref_v = O._dav_backward(c["Aqk"], c["v_new_all"], c["do"])
    assert daqk.shape == ref_q.shape and dvn.shape == ref_v.shape
    for name, x, r in (("dAqk", daqk, ref_q), ("dv_new", dvn, ref_v)):
        ok, e = close(x.cpu().numpy(), r)
        assert ok, (name, e)
    iu = np.triu_indices(BT, 1)
    assert not daqk.cpu().numpy()[..., iu[0], iu[1]].any()    # causal: exact zeros


# ----------------------------------------------------------------------------- B1
@pytest.mark.parametrize("D,with_dht,g_scale", [(64, True, 1.0), (128, False, 1.0),
                                                (128, True, 0.05), (256, True, 1.0)])
def test_dhu_matches_oracle(dev, D, with_dht, g_scale):
    """The reverse state scan: dh_all[c] the gradient of the state entering chunk c
    (dh_all[0] = dh0), dv_all; slow decay (g_scale 0.05) keeps every chunk's
    state terms in play."""
    c = case(2, 320, 2, D, seed=D + 2, g_scale=g_scale)
    dht = c["dht"] if with_dht else np.zeros_like(c["dht"])
    names = ("do", "dv_partial", "w_pseudo", "qg", "kg", "gc_last")
    got = G().gdn2_dhu_backward(*(dev_t(c[n], dev) for n in names), c["scale"],
                                dht=dev_t(dht, dev) if with_dht else None)
    ref = O._dhu_backward(*(c[n] for n in names), c["scale"], dht)
    for name, x, r in zip(("dh_all", "dh0", "dv_all"), got, ref):
        assert x.shape == r.shape, name
        ok, e = close(x.cpu().numpy(), r)
        assert ok, (name, e)
    assert torch.equal(got[0][:, :, 0], got[1])


def test_dhu_zero_chunks_and_saturated_dht(dev):
    """No chunk: dh0 = sanitize(dht), the scan's initial carry (gdn2_bwd.py:53);
    without dht, zeros."""
    B, H, D = 2, 3, 128
    dht = np.random.default_rng(5).standard_normal((B, H, D, D)).astype(np.float32) * 2e4
    z = torch.zeros((B, H, 0, BT, D), device=dev)
    gl = torch.zeros((B, H, 0, D), device=dev)
    dh_all, dh0, dv_all = G().gdn2_dhu_backward(z, z, z, z, z, gl, 0.1,
                                                dht=torch.tensor(dht, device=dev))
    assert dh_all.shape == (B, H, 0, D, D) and dv_all.shape == z.shape
    assert np.array_equal(dh0.cpu().numpy(), O.sanitize(dht).astype(np.float32))
    _, dh0, _ = G().gdn2_dhu_backward(z, z, z, z, z, gl, 0.1)
    assert not dh0.any()


# ----------------------------------------------------------------------------- B3
@pytest.mark.parametrize("D,g_scale", [(64, 1.0), (128, 1.0), (128, 0.05), (256, 1.0),
                                     (128, 30.0)])
def test_wy_dqkg_matches_oracle(dev, D, g_scale):
    """The kernels take g per token and form gc by their own in-chunk cumsum, so
    the given gc is turned into g by differences first; strong decay (g_scale
    30, |gc| up to ~1e3) checks that this round trip keeps the tolerance."""
    c = case(1, 256, 2, D, seed=D + 3, g_scale=g_scale)
    ins = [c[n] for n in ("q", "k", "b", "w", "v", "gc", "A", "Akk", "h_pre_all",
                          "v_new_all", "do", "dv_all", "dh_next")]
    got = G().wy_dqkg_backward_pallas(*(dev_t(x, dev) for x in ins), c["scale"])
    ref = O._wy_dqkg_backward(*(r32(x) for x in ins[:7]), *ins[8:], c["scale"])
    assert set(got) == set(ref)
    for name, r in ref.items():
        assert got[name].shape == r.shape, name
        ok, e = close(got[name].cpu().numpy(), r)
        assert ok, (name, e, float(np.abs(r).max()))
    il = np.triu_indices(BT)
    assert not got["dAkk"].cpu().numpy()[..., il[0], il[1]].any()   # strictly lower


# ----------------------------------------------------------------------------- B4
@pytest.mark.parametrize("D,g_scale", [(64, 1.0), (128, 1.0), (128, 30.0), (256, 1.0)])
def test_intra_matches_oracle(dev, D, g_scale):
    """q, k, b, g in the reference's (B,L,H,D) layout; strong decay (g_scale 30)
    puts most in-chunk decays past e^-20."""
    c = case(1, 256, 2, D, seed=D + 4, g_scale=g_scale)
    q, k, _, _, b, g = c["xs"]
    got = G().intra_backward_pallas(dev_t(c["daqk"], dev), dev_t(c["dakk"], dev),
                                    *(torch.tensor(x, device=dev) for x in (q, k, b, g)),
                                    c["scale"])
    ref = O._intra_backward(c["daqk"], c["dakk"], c["q"], c["k"], c["b"], c["gc"],
                            c["scale"])
    for name, x, r in zip(("dq", "dk", "db", "dgc"), got, ref):
        assert x.shape == r.shape, name
        ok, e = close(x.cpu().numpy(), r)
        assert ok, (name, e, float(np.abs(r).max()))


def test_intra_saturation_follows_the_pair_order(dev):
    """Score gradients x 1e5: B4's accumulators clip after each sub-block pair
    (gdn2_bwd.py:287-328), and that order changes the result here (checked on
    the oracle first: one clip per output differs), so the kernel must follow it."""
    D = 64
    c = case(1, 128, 2, D, seed=9, g_scale=0.05)
    daqk, dakk = r32(c["daqk"] * 1e5), r32(c["dakk"] * 1e5)
    q, k, _, _, b, g = c["xs"]
    got = G().intra_backward_pallas(dev_t(daqk, dev), dev_t(dakk, dev),
                                    *(torch.tensor(x, device=dev) for x in (q, k, b, g)),
                                    c["scale"])
    args = (daqk, dakk, c["q"], c["k"], c["b"], c["gc"], c["scale"])
    ref = O._intra_backward(*args)
    whole = O._intra_backward(*args, n_sub=None)
    assert max(np.abs(ref[i] - whole[i]).max() for i in range(4)) > 100.0
    for name, x, r in zip(("dq", "dk", "db", "dgc"), got, ref):
        x = x.cpu().numpy()
        assert np.isfinite(x).all() and np.abs(x).max() <= 1e4, name
        ok, e = close(x * 1e-4, r * 1e-4)
        assert ok, (name, e * 1e4)


# ----------------------------------------------------------------------------- B1-B5
@pytest.mark.parametrize("D,h0", [(128, True), (64, False)])
def test_backward_stages_compose_to_the_gradients(dev, D, h0):
    """Forward stages A-D, then B2 -> B1 -> B3 -> B4 -> B5 through the stage
    functions and the sums of gdn2_pipeline.py:100-135, give the gradients of
    oracle.chunked_bwd and of the fused trainable path (gdn2_bwd) at chunk 64."""
    from gdn2_package import gdn2_fwd as F
    import gdn2_package as gp
    B, T, H = 1, 320, 2
    scale = D ** -0.5
    xs = O.make_inputs(B, T, H, D, seed=D + 17)
    rng = np.random.default_rng(4)
    h0n = (0.2 * rng.standard_normal((B, H, D, D))).astype(np.float32) if h0 else None
    do = rng.standard_normal((B, T, H, D)).astype(np.float32)
    dht = rng.standard_normal((B, H, D, D)).astype(np.float32)
    xt = [torch.tensor(x, device=dev) for x in xs]
    q, k, v, w, b, g = xt
    h0t = None if h0n is None else torch.tensor(h0n, device=dev)
    aqk, akk = F.build_chunk_scores_pallas(q, k, b, g, scale)
    A = F.wy_solve_pallas(akk)
    wp, u, kg, qg, gl = F.recompute_wy_pallas(q, k, v, w, b, g, A)
    _, _, h_pre, v_new = F.gdn2_inter_chunk_combine_with_state(aqk, wp, u, kg, qg, gl, scale,
                                                               h0=h0t)
    ch = lambda x: x.view(B, T // BT, BT, H, D).permute(0, 3, 1, 2, 4).contiguous()
    dos, dhtt = ch(torch.tensor(do, device=dev)), torch.tensor(dht, device=dev)
    daqk, dvp = G().dav_backward_pallas(aqk, v_new, dos)
    dh_all, dh0, dv_all = G().gdn2_dhu_backward(dos, dvp, wp, qg, kg, gl, scale, dht=dhtt)
    dh_next = torch.cat([dh_all[:, :, 1:], dhtt[:, :, None]], dim=2)
    gc = ch(g).cumsum(dim=-2)
    b3 = G().wy_dqkg_backward_pallas(ch(q), ch(k), ch(b), ch(w), ch(v), gc, A, akk, h_pre,
                                     v_new, dos, dv_all, dh_next, scale)
    dq4, dk4, db4, dgc4 = G().intra_backward_pallas(daqk, b3["dAkk"], q, k, b, g, scale)
    dg = G().reverse_cumsum_bwd(b3["dgc"] + dgc4, BT)
    tok = lambda x: x.permute(0, 2, 3, 1, 4).reshape(B, T, H, D)
    sat = lambda x: torch.nan_to_num(x.clamp(-1e4, 1e4), nan=0.0)
    grads = [sat(tok(x)) for x in (b3["dq"] + dq4, b3["dk"] + dk4, b3["dv_raw"], b3["dw"],
                                   b3["db"] + db4, dg)] + [sat(dh0)]
    ref = O.chunked_bwd(*xs, scale, do, dht, h0=h0n, BT=BT)
    for name, x, r in zip(("dq", "dk", "dv", "dw", "db", "dg", "dh0"), grads, ref):
        ok, e = close(x.cpu().numpy(), r)
        assert ok, (name, e, float(np.abs(r).max()))
    xr = [x.clone().requires_grad_(True) for x in xt]
    h0r = None if h0t is None else h0t.clone().requires_grad_(True)
    out, hf = gp.gdn2_pallas_forward_trainable(*xr, scale, h0=h0r, chunk_size=BT)
    ((out * torch.tensor(do, device=dev)).sum() + (hf * dhtt).sum()).backward()
    for name, x, r in zip(("dq", "dk", "dv", "dw", "db", "dg"), grads, xr):
        assert float((x - r.grad).abs().max()) <= 1e-4 * (1 + float(r.grad.abs().max())), name
