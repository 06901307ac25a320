"""The clip bound CLIP (gdn2_fwd.py:33) overridden after import, as the
reference README does (fwd.CLIP = 1e3, README.md:87-92): every stage sanitize
of the library then saturates at the new bound.  Each kernel unit holds its own
copy of the bound (gdn2_set_clip sets them all), so each is checked here through
a path that runs it: the forward (fwd_prep / fwd_state / fwd_out), the training
backward (bwd_b2 / bwd_state / bwd_wy / gram_bwd), the decode step and a stage
function (reverse cumsum).  Against the oracle with the same CLIP (its sanitize
reads the module constant at call time), on the saturation scale: |got - ref| <=
1e-4 * CLIP + 1e-4 * |ref|.  Restoring 1e4 gives the default results bit for bit."""
import numpy as np
import pytest
import torch

from oracle import gdn2_oracle as O

pytestmark = pytest.mark.gpu


def close(got, ref, tol):
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    return float((np.abs(got - ref) - (tol + tol * np.abs(ref))).max()) <= 0.0, \
        float(np.abs(got - ref).max())


def gp():
    import gdn2_package
    return gdn2_package


@pytest.fixture
def clip(monkeypatch):
    """Set CLIP in the package and the oracle alike (both restored afterwards)."""
    from gdn2_package import gdn2_fwd

    def set_(c):
        monkeypatch.setattr(gdn2_fwd, "CLIP", c)
        monkeypatch.setattr(O, "CLIP", c)
    return set_


def dev_inputs(dev, xs):
    return [torch.tensor(x, device=dev) for x in xs]


def test_forward_saturates_at_the_override(dev, clip):
    """CLIP = 1e3, v x 1e4, scale 20, slow decay: u, the outputs and the states
    saturate at +-1e3 (unclipped they pass 1e4); float32 forward at chunk 64
    against oracle.chunked_fwd(clip=True) under the same CLIP."""
    B, T, H, D, scale = 1, 256, 2, 64, 20.0
    xs = list(O.make_inputs(B, T, H, D, seed=41, g_scale=0.05))
    xs[2] = xs[2] * 1e4
    xt = dev_inputs(dev, xs)
    base = [y.clone() for y in gp().gdn2_pallas_forward(*xt, scale, chunk_size=64)]
    clip(1e3)
    out, hf = gp().gdn2_pallas_forward(*xt, scale, chunk_size=64)
    ro, rh, res = O.chunked_fwd(*xs, scale, BT=64, clip=True, return_residuals=True)
    assert np.abs(res["u"]).max() == 1e3 and np.abs(ro).max() == 1e3
    assert np.abs(base[0].cpu().numpy()).max() > 2e3          # the default bound is not hit
    ok_o, e_o = close(out.cpu().numpy() * 1e-3, ro * 1e-3, 1e-4)
    ok_h, e_h = close(hf.cpu().numpy() * 1e-3, rh * 1e-3, 1e-4)
    assert ok_o and ok_h, (e_o, e_h)
    assert float(out.abs().max()) <= 1e3 and float(hf.abs().max()) <= 1e3
    clip(1e4)                                   # back to the default: bit for bit
    out2, hf2 = gp().gdn2_pallas_forward(*xt, scale, chunk_size=64)
    assert torch.equal(out2, base[0]) and torch.equal(hf2, base[1])


def test_training_saturates_at_the_override(dev, clip):
    """CLIP = 1e3 with cotangents past it (do x 1e3, dh_final x 3e3; slow decay,
    unit v and scale): the float32 trainable path's gradients against
    oracle.chunked_bwd(clip=True) under the same CLIP, several percent of them
    saturated."""
    B, T, H, D, scale = 1, 256, 2, 64, 1.0
    xs = O.make_inputs(B, T, H, D, seed=42, g_scale=0.05)
    rng = np.random.default_rng(5)
    do = (rng.standard_normal((B, T, H, D)) * 1e3).astype(np.float32)
    dh = (rng.standard_normal((B, H, D, D)) * 3e3).astype(np.float32)
    h0 = rng.standard_normal((B, H, D, D)).astype(np.float32)
    clip(1e3)
    xt = [x.requires_grad_(True) for x in dev_inputs(dev, xs)]
    h0t = torch.tensor(h0, device=dev, requires_grad=True)
    out, hf = gp().gdn2_pallas_forward_trainable(*xt, scale, h0=h0t)
    ((out * torch.tensor(do, device=dev)).sum() + (hf * torch.tensor(dh, device=dev)).sum()).backward()
    ref = O.chunked_bwd(*xs, scale, do, dh, h0=h0, BT=64, clip=True)
    assert 0.01 < np.mean(np.abs(ref[0]) == 1e3) < 0.5
    grads = [x.grad.cpu().numpy() for x in xt] + [h0t.grad.cpu().numpy()]
    for n, g, r in zip(["dq", "dk", "dv", "dw", "db", "dg", "dh0"], grads, ref):
        assert np.isfinite(g).all() and np.abs(g).max() <= 1e3, n
        ok, e = close(g * 1e-3, r * 1e-3, 1e-4)
        assert ok, (n, e * 1e3)


def test_decode_and_stage_function_saturate_at_the_override(dev, clip):
    """CLIP = 100 in the decode step (its entry state, new state and output are
    sanitized, gdn2_fwd.py:334-335,355-356, with a chunk of one token) and in the
    reverse cumsum of the backward stage functions (gdn2_bwd.py:41)."""
    B, H, D = 2, 3, 64
    xs = O.make_inputs(B, 1, H, D, seed=43)
    xt = dev_inputs(dev, xs)
    state = (np.random.default_rng(6).standard_normal((B, H, D, D)) * 300.0).astype(np.float32)
    clip(100.0)
    o, h = gp().gdn2_decode_step(*xt, D ** -0.5, state=torch.tensor(state, device=dev))
    s0 = O.sanitize(state.astype(np.float64))
    assert np.abs(s0).max() == 100.0
    _, s_new = O.recurrent_fwd(*[x.astype(np.float64) for x in xs], D ** -0.5, h0=s0)
    s2 = O.sanitize(s_new)
    o_ref = O.sanitize(D ** -0.5 * np.einsum("bhd,bhde->bhe", xs[0][:, 0].astype(np.float64), s2))
    assert close(h.cpu().numpy() * 1e-2, s2 * 1e-2, 1e-4)[0]
    assert close(o[:, 0].cpu().numpy() * 1e-2, o_ref * 1e-2, 1e-4)[0]
    from gdn2_package import gdn2_bwd
    dgc = torch.tensor(np.random.default_rng(7).standard_normal((2, 3, 4, 64, 64)) * 40.0,
                       device=dev, dtype=torch.float32)
    dg = gdn2_bwd.reverse_cumsum_bwd(dgc, 64).cpu().numpy()
    ref = O._reverse_cumsum(dgc.double().cpu().numpy())
    assert np.abs(ref).max() == 100.0 and np.mean(np.abs(ref) == 100.0) > 0.05
    assert close(dg * 1e-2, ref * 1e-2, 1e-4)[0]
