"""Backward parity on the GPU: gradients of gdn2_pallas_forward_trainable
(torch.autograd through the gfx950 library) against the oracle's restatement
of B1-B5 (float64), which tests/test_oracle.py pins to torch.autograd of the
token recurrence.  Tolerance |got - ref| <= tol + tol*|ref|, tol = 1e-4 for
float32 inputs and 2e-2 for bfloat16 inputs.
"""
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import gdn2_oracle as O

pytestmark = pytest.mark.gpu
GOLD = Path(__file__).resolve().parent / "golden"
NAMES = ["dq", "dk", "dv", "dw", "db", "dg", "dh0"]


def close(got, ref, tol):
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    return float((np.abs(got - ref) - (tol + tol * np.abs(ref))).max()) <= 0.0, \
        float(np.abs(got - ref).max())


def gp():
    import gdn2_package
    return gdn2_package


def run_grads(xs, scale, do, dh=None, h0=None, dtype=torch.float32, dev="cuda:0", **kw):
    xt = [torch.tensor(np.asarray(x), device=dev).to(dtype if i < 5 else torch.float32)
          .requires_grad_(True) for i, x in enumerate(xs)]
    h0t = None if h0 is None else torch.tensor(h0, device=dev, requires_grad=True)
    out, hf = gp().gdn2_pallas_forward_trainable(*xt, scale, h0=h0t, **kw)
    loss = (out * torch.tensor(do, device=dev)).sum()
    if dh is not None:
        loss = loss + (hf * torch.tensor(dh, device=dev)).sum()
    loss.backward()
    grads = [x.grad.float().cpu().numpy() for x in xt]
    grads.append(None if h0t is None else h0t.grad.cpu().numpy())
    return (out, hf), grads, xt


def check(grads, ref, tol, names=NAMES):
    for n, g, r in zip(names, grads, ref):
        if g is None:
            continue
        ok, e = close(g, r, tol)
        assert ok, (n, e, float(np.abs(r).max()))


def test_bwd_golden_fixture(dev):
    with np.load(GOLD / "bwd_small.npz", allow_pickle=False) as z:
        xs = [z[n] for n in "qkvwbg"]
        (out, hf), grads, _ = run_grads(xs, float(z["scale"]), z["do"], z["dh"], h0=z["h0"],
                                        dev=dev)
        assert close(out.detach().cpu().numpy(), z["out"], 1e-4)[0]
        assert close(hf.detach().cpu().numpy(), z["h_final"], 1e-4)[0]
        check(grads, [z[n] for n in NAMES], 1e-4)


@pytest.mark.parametrize("B,T,H,D,h0,dh,gs", [
    (1, 256, 2, 64, False, False, 1.0),
    (2, 256, 3, 128, True, True, 1.0),
    (1, 512, 2, 128, True, True, 0.05),     # slow decay: state terms of dgc_last matter
    (1, 128, 1, 64, False, True, 4.0),      # strong decay
])
def test_bwd_matches_oracle_fp32(dev, B, T, H, D, h0, dh, gs):
    xs = O.make_inputs(B, T, H, D, seed=T + D + H, g_scale=gs)
    rng = np.random.default_rng(11)
    h0n = (0.2 * rng.standard_normal((B, H, D, D))).astype(np.float32) if h0 else None
    do = rng.standard_normal((B, T, H, D)).astype(np.float32)
    dhn = rng.standard_normal((B, H, D, D)).astype(np.float32) if dh else None
    _, grads, _ = run_grads(xs, D ** -0.5, do, dhn, h0=h0n, dev=dev)
    ref = O.chunked_bwd(*xs, D ** -0.5, do, dhn, h0=h0n, BT=64, clip=False)
    check(grads, ref, 1e-4)


@pytest.mark.parametrize("D,dtype", [(64, torch.float32), (128, torch.float32),
                                     (128, torch.bfloat16), (256, torch.float32),
                                     (256, torch.bfloat16)])
def test_bwd_strong_decay_diagonal_blocks(dev, D, dtype):
    """Channels 0..7 at about -20 of log-decay per token (past the single-center
    factorisation of the diagonal score blocks, which take the exact
    hierarchical sums in the forward and in gram_bwd): all gradients against
    torch.autograd of the float64 recurrence (oracle.recurrent_grads)."""
    B, T, H = 1, 128, 2
    xs = O.make_inputs(B, T, H, D, seed=D + 3)
    g = np.array(xs[5])
    g[..., :8] *= 30.0
    xs = list(xs[:5]) + [g]
    rng = np.random.default_rng(13)
    h0n = (0.2 * rng.standard_normal((B, H, D, D))).astype(np.float32)
    do = rng.standard_normal((B, T, H, D)).astype(np.float32)
    dhn = rng.standard_normal((B, H, D, D)).astype(np.float32)
    _, grads, xt = run_grads(xs, D ** -0.5, do, dhn, h0=h0n, dtype=dtype, dev=dev)
    xin = [x.detach().float().cpu().numpy() for x in xt]
    ref = O.recurrent_grads(*xin, D ** -0.5, do, dhn, h0=h0n)
    check(grads, ref, 1e-4 if dtype == torch.float32 else 2e-2)


@pytest.mark.parametrize("T,h0", [(200, True), (37, False)])
def test_bwd_partial_last_chunk(dev, T, h0):
    """T % 64 != 0 in the trainable path (zero tokens pad the inputs to whole
    chunks): gradients of the real tokens against the oracle's."""
    B, H, D = 1, 2, 64
    xs = O.make_inputs(B, T, H, D, seed=T + 3)
    rng = np.random.default_rng(12)
    h0n = (0.2 * rng.standard_normal((B, H, D, D))).astype(np.float32) if h0 else None
    do = rng.standard_normal((B, T, H, D)).astype(np.float32)
    dhn = rng.standard_normal((B, H, D, D)).astype(np.float32)
    (out, _), grads, _ = run_grads(xs, D ** -0.5, do, dhn, h0=h0n, dev=dev)
    assert out.shape == (B, T, H, D)
    ref = O.recurrent_grads(*xs, D ** -0.5, do, dhn, h0=h0n)
    check(grads, ref, 1e-4)


def test_bwd_bf16_inputs(dev):
    """bfloat16 inputs with a unit-scale h0 and dh_final: the trainable path
    computes in float32 (the reference upcasts, gdn2_fwd.py:100-103) and
    returns bfloat16 gradients, within 2e-2 of the oracle on the same
    bf16-rounded inputs."""
    B, T, H, D = 1, 256, 2, 128
    xs = O.make_inputs(B, T, H, D, seed=21)
    rng = np.random.default_rng(3)
    do = rng.standard_normal(xs[0].shape).astype(np.float32)
    dhn = rng.standard_normal((B, H, D, D)).astype(np.float32)
    h0n = rng.standard_normal((B, H, D, D)).astype(np.float32)
    _, grads, xt = run_grads(xs, D ** -0.5, do, dhn, h0=h0n, dtype=torch.bfloat16, dev=dev)
    for x in xt[:5]:
        assert x.grad.dtype == torch.bfloat16
    xin = [x.detach().float().cpu().numpy() for x in xt]
    ref = O.chunked_bwd(*xin, D ** -0.5, do, dhn, h0=h0n, BT=64, clip=False)
    check(grads, ref, 2e-2)


@pytest.mark.parametrize("D", [64, 128, 256])
def test_bf16_storage_float32_arithmetic_equals_widened(dev, D):
    """GDN2_BF16_F32 (bfloat16 q,k,v,w,b read as they are, float32 arithmetic and
    residuals, bfloat16 gradients) against the same float32 kernels on the
    inputs widened to float32 first, the gradients rounded to bfloat16
    afterwards: the arithmetic is the same, so out, h_final and every gradient
    agree bit for bit; g in float32 and in bfloat16."""
    from gdn2_package import _lib
    from gdn2_package.gdn2_fwd import _Prepared, _run_forward
    from gdn2_package.gdn2_pipeline import _run_backward
    B, T, H = 1, 256, 2
    xs = O.make_inputs(B, T, H, D, seed=31)
    rng = np.random.default_rng(5)
    do = torch.tensor(rng.standard_normal(xs[0].shape).astype(np.float32), device=dev)
    dh = torch.tensor(rng.standard_normal((B, H, D, D)).astype(np.float32), device=dev)
    h0 = torch.tensor(rng.standard_normal((B, H, D, D)).astype(np.float32), device=dev)
    for g_dt in (torch.float32, torch.bfloat16):
        xb = [torch.tensor(x, device=dev).to(torch.bfloat16) for x in xs[:5]] + \
            [torch.tensor(xs[5], device=dev).to(g_dt)]
        pm = _Prepared(*xb, D ** -0.5, h0, 64, compute_dtype=torch.float32)
        assert pm.code == _lib.GDN2_BF16_F32 and pm.q.dtype == torch.bfloat16
        pw = _Prepared(*[x.float() for x in xb], D ** -0.5, h0, 64, compute_dtype=torch.float32)
        assert pw.code == _lib.GDN2_F32
        om, hm, wsm, _ = _run_forward(pm, flags=_lib.FWD_SAVE_A)
        ow, hw, wsw, _ = _run_forward(pw, flags=_lib.FWD_SAVE_A)
        assert torch.equal(om, ow) and torch.equal(hm, hw)
        gm = _run_backward(pm, wsm, do, dh)
        gw = _run_backward(pw, wsw, do, dh)
        for i, (a, b) in enumerate(zip(gm, gw)):
            want = b if i == 6 else b.to(xb[i].dtype)
            assert a.dtype == want.dtype, (NAMES[i], a.dtype, want.dtype)
            assert torch.equal(a, want), (NAMES[i], float((a.float() - want.float()).abs().max()))


def test_config4_training_path_bf16(dev):
    """The training path at BASELINE configs[3]'s shape (8,8192,6,128) with
    bfloat16 q,k,v,w,b, float32 g, an N(0,1) cotangent on out and a unit N(0,1)
    cotangent on h_final.  Two sampled (batch, head) pairs are checked against
    the oracle's B1-B5 on the bf16-rounded inputs at 2e-2."""
    B, T, H, D = 8, 8192, 6, 128
    gen = torch.Generator(device=dev).manual_seed(4)
    r = lambda *s: torch.randn(s or (B, T, H, D), generator=gen, device=dev)
    q, k, v, w, b, g = r(), r(), r(), r(), r(), r()
    q, k = q / q.norm(dim=-1, keepdim=True), k / k.norm(dim=-1, keepdim=True)
    w, b, g = torch.sigmoid(w), torch.sigmoid(b), -torch.nn.functional.softplus(g)
    xt = [x.to(torch.bfloat16).detach().requires_grad_(True) for x in (q, k, v, w, b)] + \
        [g.detach().requires_grad_(True)]
    do, dh = r(), r(B, H, D, D)
    out, hf = gp().gdn2_pallas_forward_trainable(*xt, D ** -0.5)
    torch.autograd.backward([out, hf], [do, dh])
    for x in xt:
        assert torch.isfinite(x.grad.float()).all()
    for bb, hh in [(2, 1), (6, 5)]:
        sl = [x.detach()[bb:bb + 1, :, hh:hh + 1].float().cpu().numpy() for x in xt]
        ref = O.chunked_bwd(*sl, D ** -0.5, do[bb:bb + 1, :, hh:hh + 1].cpu().numpy(),
                            dh[bb:bb + 1, hh:hh + 1].cpu().numpy(), BT=64, clip=False)
        got = [x.grad[bb:bb + 1, :, hh:hh + 1].float().cpu().numpy() for x in xt]
        check(got, ref[:6], 2e-2, NAMES[:6])


def test_bwd_recompute_matches_saved_residuals(dev):
    xs = O.make_inputs(1, 256, 2, 64, seed=5)
    do = np.random.default_rng(2).standard_normal(xs[0].shape).astype(np.float32)
    _, g1, _ = run_grads(xs, 0.125, do, dev=dev)
    _, g2, _ = run_grads(xs, 0.125, do, dev=dev, recompute=True)
    for a, b in zip(g1[:6], g2[:6]):
        assert np.array_equal(a, b)


def test_config4_training_path_fp32(dev):
    """(8,8192,6,128) fp32 forward + custom backward with an
    N(0,1) cotangent on out and zero cotangent on h_final.  Two sampled
    (batch, head) pairs are checked against the oracle (pairs are independent)."""
    B, T, H, D = 8, 8192, 6, 128
    gen = torch.Generator(device=dev).manual_seed(0)
    r = lambda: torch.randn((B, T, H, D), generator=gen, device=dev)
    q, k, v, w, b, g = r(), r(), r(), r(), r(), r()
    q, k = q / q.norm(dim=-1, keepdim=True), k / k.norm(dim=-1, keepdim=True)
    w, b, g = torch.sigmoid(w), torch.sigmoid(b), -torch.nn.functional.softplus(g)
    xt = [x.detach().requires_grad_(True) for x in (q, k, v, w, b, g)]
    do = torch.randn((B, T, H, D), generator=gen, device=dev)
    out, hf = gp().gdn2_pallas_forward_trainable(*xt, D ** -0.5)
    torch.autograd.backward([out], [do])
    for x in xt:
        assert torch.isfinite(x.grad).all()
    for bb, hh in [(0, 0), (5, 4)]:
        sl = [x.detach()[bb:bb + 1, :, hh:hh + 1].cpu().numpy() for x in xt]
        ref = O.chunked_bwd(*sl, D ** -0.5, do[bb:bb + 1, :, hh:hh + 1].cpu().numpy(), BT=64,
                            clip=False)
        got = [x.grad[bb:bb + 1, :, hh:hh + 1].cpu().numpy() for x in xt]
        check(got, ref[:6], 1e-4, NAMES[:6])


def test_reference_all_ones_forward_backward(dev):
    """tests/test_pallas.py:27-39: all-ones (2,512,4,128), scale 0.1, through the
    trainable path; shapes and finiteness (values are saturation artefacts)."""
    shape = (2, 512, 4, 128)
    xs = [torch.ones(shape, device=dev, requires_grad=True) for _ in range(6)]
    out, hf = gp().gdn2_pallas_forward_trainable(*xs, 0.1)
    assert out.shape == shape and hf.shape == (2, 4, 128, 128)
    (out.sum() + hf.sum()).backward()
    for x in xs:
        assert x.grad.shape == shape and torch.isfinite(x.grad).all()
        assert x.grad.abs().max().item() <= 1e4


def test_grad_of_h0_only_when_given(dev):
    xs = O.make_inputs(1, 128, 2, 64, seed=1)
    do = np.ones(xs[0].shape, dtype=np.float32)
    _, grads, _ = run_grads(xs, 0.125, do, dev=dev)
    assert grads[6] is None


@pytest.mark.parametrize("T,H,h0,dh,dtype", [
    (128, 2, True, 1.0, torch.float32),
    (192, 1, False, 0.0, torch.float32),
    (128, 1, True, 1.0, torch.bfloat16),
])
def test_bwd_d256_matches_oracle(dev, T, H, h0, dh, dtype):
    """D = 256 (beyond the reference, which asserts D == 128): the backward of
    per-chunk products, against the oracle's B1-B5 in float64, with unit-scale
    h0 and dh_final also for bfloat16 inputs (computed in float32)."""
    B, D = 1, 256
    xs = O.make_inputs(B, T, H, D, seed=T + H)
    rng = np.random.default_rng(13)
    h0n = (0.2 * rng.standard_normal((B, H, D, D))).astype(np.float32) if h0 else None
    do = rng.standard_normal((B, T, H, D)).astype(np.float32)
    dhn = (dh * rng.standard_normal((B, H, D, D))).astype(np.float32) if dh else None
    _, grads, xt = run_grads(xs, D ** -0.5, do, dhn, h0=h0n, dtype=dtype, dev=dev)
    xin = [x.detach().float().cpu().numpy() for x in xt]
    ref = O.chunked_bwd(*xin, D ** -0.5, do, dhn, h0=h0n, BT=64, clip=False)
    check(grads, ref, 1e-4 if dtype == torch.float32 else 2e-2)


# ----------------------------------------------------------------------------- saturation
@pytest.mark.parametrize("D,dos,dhs", [(64, 1e4, 0.0), (64, 3e3, 3e4), (128, 3e3, 3e4),
                                       (256, 3e3, 3e4)])
def test_bwd_saturation_matches_reference_clipping(dev, D, dos, dhs):
    """Cotangents past the reference's clip (do x 1e4, or do x 3e3 with dh_final x
    3e4, D = 64, 128 and 256; slow decay, unit v and scale): B2's dAqk / dv_partial, B1's dv_new and
    dh carry (and its sanitized dh_final), B3's dA, dA A^T and outputs, B4's
    accumulators in the sub-block pair order and B5 all clip somewhere, and
    4-20 % of the gradients saturate.  The float32 trainable path matches the
    oracle's restatement with the same clip points (oracle.chunked_bwd,
    clip=True: B4's pair loop with _clip_acc, gdn2_bwd.py:287-339, and the raw
    dh_final as B3's last dh', gdn2_pipeline.py:52-56).  The test first checks
    on the oracle that both of those change the result here, so a kernel that
    clipped B4 once per output or fed B3 the sanitized dh_final would fail.
    Tolerance on the saturation scale: |got - ref| <= 1e-4 * 1e4 + 1e-4 * |ref|."""
    B, T, H, scale = 1, 256, 2, 1.0
    xs = O.make_inputs(B, T, H, D, seed=40, g_scale=0.05)
    rng = np.random.default_rng(3)
    do = (rng.standard_normal((B, T, H, D)) * dos).astype(np.float32)
    dhn = (rng.standard_normal((B, H, D, D)) * dhs).astype(np.float32)
    h0n = rng.standard_normal((B, H, D, D)).astype(np.float32)
    _, grads, _ = run_grads(xs, scale, do, dhn, h0=h0n, dev=dev)
    ref = O.chunked_bwd(*xs, scale, do, dhn, h0=h0n, BT=64, clip=True)
    whole = O.chunked_bwd(*xs, scale, do, dhn, h0=h0n, BT=64, clip=True, n_sub=None)
    # B4's pair order matters here (in dq, dk or db).  Not at D = 256, whose sums over
    # twice the channels make it matter only from do x 1e5, where the float32 scans'
    # split products (operands rounded to 2^-17) amplified 1e5-fold put dq past this
    # bound (1.6-1.75, at D = 128 as at 256): this case pins bwd_wy_wide's and the
    # D = 256 scans' clip points and the raw dh_final, the pair order is pinned above
    pair = max(np.abs(ref[i] - whole[i]).max() for i in (0, 1, 4))
    assert pair > 100.0 if D <= 128 else pair < 1e-6
    if dhs:
        san = O.chunked_bwd(*xs, scale, do, O.sanitize(dhn), h0=h0n, BT=64, clip=True)
        assert np.abs(ref[1] - san[1]).max() > 100.0        # and so does the raw dh_final
    assert 0.01 < np.mean(np.abs(ref[0]) == 1e4) < 0.5
    for n, g, r in zip(NAMES, grads, ref):
        assert np.isfinite(g).all() and np.abs(g).max() <= 1e4, n
        ok, e = close(g * 1e-4, r * 1e-4, 1e-4)
        assert ok, (n, e * 1e4)


# ----------------------------------------------------------------------------- empty
@pytest.mark.parametrize("dtype,D", [(torch.float32, 64), (torch.float32, 128),
                                     (torch.bfloat16, 128), (torch.float32, 256)])
def test_empty_sequence_training(dev, dtype, D):
    """T = 0 through the trainable path: h_final = h0, every input gradient is
    empty, and dh0 is the cotangent on h_final (the state passes through no chunk;
    B1 starts its carry from the sanitized dh_final, which a value inside the clip
    leaves unchanged)."""
    B, H = 2, 2
    xs = [torch.zeros((B, 0, H, D), device=dev, dtype=dtype if i < 5 else torch.float32)
          .requires_grad_(True) for i in range(6)]
    h0 = torch.randn((B, H, D, D), device=dev, requires_grad=True)
    out, hf = gp().gdn2_pallas_forward_trainable(*xs, D ** -0.5, h0=h0)
    assert out.shape == (B, 0, H, D) and torch.equal(hf.detach(), h0.detach())
    dhf = torch.randn_like(hf)
    grads = torch.autograd.grad((hf * dhf).sum() + out.sum(), xs + [h0])
    torch.cuda.synchronize()
    for x, g in zip(xs, grads[:6]):
        assert g.shape == x.shape and g.dtype == x.dtype
    assert torch.equal(grads[6], dhf)


@pytest.mark.parametrize("D", [128, 256])
def test_bwd_split_products_headroom_under_saturation(dev, D):
    """The float32 scans' split products (operands as bfloat16 hi + lo, 2^-17)
    under a cotangent ten times past the test above (do x 3e4; 32 % of dq at the
    clip at D = 256): the forward state's rounding, amplified 3e4-fold into dq, must still
    sit inside the saturation-scale bound |got - ref| <= 1 + 1e-4 |ref| (measured
    about half of it; from do x 1e5 it does not, see the clip-point test)."""
    B, T, H, scale = 1, 256, 2, 1.0
    xs = O.make_inputs(B, T, H, D, seed=40, g_scale=0.05)
    rng = np.random.default_rng(3)
    do = (rng.standard_normal((B, T, H, D)) * 3e4).astype(np.float32)
    dhn = (rng.standard_normal((B, H, D, D)) * 0.0).astype(np.float32)   # zero dh_final
    h0n = rng.standard_normal((B, H, D, D)).astype(np.float32)
    _, grads, _ = run_grads(xs, scale, do, dhn, h0=h0n, dev=dev)
    ref = O.chunked_bwd(*xs, scale, do, dhn, h0=h0n, BT=64, clip=True)
    assert 0.01 < np.mean(np.abs(ref[0]) == 1e4) < 0.5
    for n, g, r in zip(NAMES, grads, ref):
        assert np.isfinite(g).all() and np.abs(g).max() <= 1e4, n
        ok, e = close(g * 1e-4, r * 1e-4, 1e-4)
        assert ok, (n, e * 1e4)
