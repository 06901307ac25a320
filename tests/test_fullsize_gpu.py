"""Full-size parity over every (batch, head) pair.

The gfx950 forward at the BASELINE configs[2] and configs[4] shapes, the training
path's gradients at configs[3], and the D = 256 forward and training path (B8 T8192
H3), are compared with the token recurrence
(gdn2_fwd.py:342-360, restated by oracle.recurrent_fwd) and its adjoint, evaluated in
float64 with torch on the same GPU: the CPU oracle cannot finish these sizes in
seconds, so test_fwd_gpu.py / test_bwd_gpu.py check sampled pairs there; this file
checks all of them.  The torch recurrence and adjoint are pinned against
oracle.recurrent_fwd and oracle.recurrent_grads (torch.autograd) on small cases first.
Tolerances as in the other parity tests: |got - ref| <= tol (1 + |ref|), tol = 2e-2
for bfloat16 inputs (the reference running on the bf16-rounded inputs), 1e-4 for
float32.
"""
import numpy as np
import pytest
import torch

from oracle import gdn2_oracle as O

pytestmark = pytest.mark.gpu


def gp():
    import gdn2_package
    return gdn2_package


def recurrence_fp64(q, k, v, w, b, g, scale, h0=None):
    """out (B,T,H,D) and h_final (B,H,D,D), float64, one token at a time on the
    device: S <- e^{g_t} S;  S <- S + k_t (w_t v_t - (b_t k_t)^T S);  o_t = scale q_t^T S.
    Element-wise products and sums only (no batched matrix products)."""
    q, k, v, w, b, g = (x.double() for x in (q, k, v, w, b, g))
    B, T, H, D = q.shape
    S = torch.zeros((B, H, D, D), dtype=torch.float64, device=q.device) if h0 is None \
        else h0.double().clone()
    out = torch.empty((B, T, H, D), dtype=torch.float64, device=q.device)
    eg, bk, wv = g.exp(), b * k, w * v
    for t in range(T):
        S.mul_(eg[:, t, :, :, None])
        pred = (bk[:, t, :, :, None] * S).sum(2)
        S.add_(k[:, t, :, :, None] * (wv[:, t] - pred)[:, :, None, :])
        out[:, t] = scale * (q[:, t, :, :, None] * S).sum(2)
    return out, S


def recurrence_grads_fp64(q, k, v, w, b, g, scale, do, dh_final=None, h0=None, seg=64):
    """Gradients (dq, dk, dv, dw, db, dg, dh0) of sum(out * do) + sum(h_final *
    dh_final) for recurrence_fp64, float64 on the device: the adjoint of each token
    step, run backwards; the states are recomputed per segment of `seg` tokens from
    checkpoints taken in a first forward sweep."""
    q, k, v, w, b, g, do = (x.double() for x in (q, k, v, w, b, g, do))
    B, T, H, D = q.shape
    eg, bk, wv = g.exp(), b * k, w * v

    def step(S, t):
        Sp = eg[:, t, :, :, None] * S
        pred = (bk[:, t, :, :, None] * Sp).sum(2)
        return Sp + k[:, t, :, :, None] * (wv[:, t] - pred)[:, :, None, :]

    S = torch.zeros((B, H, D, D), dtype=torch.float64, device=q.device) if h0 is None \
        else h0.double().clone()
    ckpt = []
    for t0 in range(0, T, seg):
        ckpt.append(S)
        for t in range(t0, min(T, t0 + seg)):
            S = step(S, t)
    dS = torch.zeros_like(S) if dh_final is None else dh_final.double().clone()
    dq, dk, dv, dw, db, dg = (torch.empty_like(q) for _ in range(6))
    for si in reversed(range(len(ckpt))):
        t0, t1 = si * seg, min(T, si * seg + seg)
        prev, S = [], ckpt[si]
        for t in range(t0, t1):
            prev.append(S)
            S = step(S, t)
        for t in reversed(range(t0, t1)):
            Sp = eg[:, t, :, :, None] * prev[t - t0]                 # e^{g_t} S_{t-1}
            delta = wv[:, t] - (bk[:, t, :, :, None] * Sp).sum(2)
            St = Sp + k[:, t, :, :, None] * delta[:, :, None, :]
            dS = dS + scale * q[:, t, :, :, None] * do[:, t, :, None, :]   # o_t = scale q_t^T S_t
            dq[:, t] = scale * (St * do[:, t, :, None, :]).sum(3)
            ddelta = (dS * k[:, t, :, :, None]).sum(2)               # S_t = Sp + k delta^T
            dkt = (dS * delta[:, :, None, :]).sum(3)
            dw[:, t], dv[:, t] = ddelta * v[:, t], ddelta * w[:, t]  # delta = w v - pred
            dbk = -(Sp * ddelta[:, :, None, :]).sum(3)               # pred = Sp^T (b k)
            dSp = dS - bk[:, t, :, :, None] * ddelta[:, :, None, :]
            db[:, t], dk[:, t] = dbk * k[:, t], dkt + dbk * b[:, t]
            dg[:, t] = (dSp * Sp).sum(3)                             # Sp = e^{g_t} S_{t-1}
            dS = eg[:, t, :, :, None] * dSp
    return dq, dk, dv, dw, db, dg, dS


def within(got, ref, tol):
    err = (got.double() - ref).abs() - (tol + tol * ref.abs())
    return float(err.max()) <= 0.0, float((got.double() - ref).abs().max())


def baseline_inputs(B, T, H, D, dev, g_mul=1.0, seed=0):
    """The BASELINE distributions (q, k L2-normalised; w, b sigmoid; g = -softplus),
    q, k, v, w, b rounded to bfloat16, g in float32."""
    gen = torch.Generator(device=dev).manual_seed(seed)
    r = lambda: torch.randn((B, T, H, D), generator=gen, device=dev)
    q, k, v, w, b, g = r(), r(), r(), r(), r(), r()
    q, k = q / q.norm(dim=-1, keepdim=True), k / k.norm(dim=-1, keepdim=True)
    w, b = torch.sigmoid(w), torch.sigmoid(b)
    g = -torch.nn.functional.softplus(g) * g_mul
    return [x.to(torch.bfloat16) for x in (q, k, v, w, b)] + [g]


def test_recurrence_fp64_matches_oracle(dev):
    """The device recurrence equals oracle.recurrent_fwd (float64 numpy) to rounding."""
    xs = O.make_inputs(2, 96, 3, 32, seed=5)
    h0 = (0.3 * np.random.default_rng(2).standard_normal((2, 3, 32, 32)))
    ro, rh = O.recurrent_fwd(*xs, 0.25, h0=h0)
    to, th = recurrence_fp64(*[torch.tensor(x, device=dev) for x in xs], 0.25,
                             h0=torch.tensor(h0, device=dev))
    assert np.abs(to.cpu().numpy() - ro).max() < 1e-12
    assert np.abs(th.cpu().numpy() - rh).max() < 1e-12


def test_recurrence_grads_fp64_matches_oracle(dev):
    """The device adjoint equals oracle.recurrent_grads (torch.autograd, float64 CPU),
    with h0, a cotangent on h_final and a segment length that does not divide T."""
    xs = O.make_inputs(2, 70, 2, 16, seed=9)
    rng = np.random.default_rng(4)
    h0 = 0.3 * rng.standard_normal((2, 2, 16, 16))
    do, dh = rng.standard_normal((2, 70, 2, 16)), rng.standard_normal((2, 2, 16, 16))
    ref = O.recurrent_grads(*xs, 0.25, do, dh, h0=h0)
    t = lambda x: torch.tensor(np.asarray(x, dtype=np.float64), device=dev)
    got = recurrence_grads_fp64(*[t(x) for x in xs], 0.25, t(do), t(dh), h0=t(h0), seg=16)
    for a, r in zip(got, ref):
        assert np.abs(a.cpu().numpy() - np.asarray(r)).max() < 1e-11


def test_config3_headline_all_pairs(dev):
    """(8,8192,6,128) bf16 inputs, fp32 g; all 48 pairs, at
    BT=128 (the configuration's chunk) and at the library's default chunk 64."""
    B, T, H, D = 8, 8192, 6, 128
    xt = baseline_inputs(B, T, H, D, dev)
    ro, rh = recurrence_fp64(*xt, D ** -0.5)
    for bt in (128, 64):
        out, hf = gp().gdn2_pallas_forward(*xt, D ** -0.5, chunk_size=bt)
        ok_o, e_o = within(out, ro, 2e-2)
        ok_h, e_h = within(hf, rh, 2e-2)
        assert ok_o and ok_h, (bt, e_o, e_h)


def test_config5_long_context_all_heads(dev):
    """(1,131072,8,128) bf16, g = -softplus * 0.1 (the
    segmented scan); all 8 heads over the full 131072-token chain, at BT=128 (the
    configuration's chunk) and at the default chunk 64."""
    B, T, H, D = 1, 131072, 8, 128
    xt = baseline_inputs(B, T, H, D, dev, g_mul=0.1)
    ro, rh = recurrence_fp64(*xt, D ** -0.5)
    for bt in (128, 64):
        out, hf = gp().gdn2_pallas_forward(*xt, D ** -0.5, chunk_size=bt)
        ok_o, e_o = within(out, ro, 2e-2)
        ok_h, e_h = within(hf, rh, 2e-2)
        assert ok_o and ok_h, (bt, e_o, e_h)


def test_config4_training_all_pairs(dev):
    """(8,8192,6,128) float32 training path with an N(0,1)
    cotangent on out and zero cotangent on h_final; the six input gradients of all
    48 pairs against the float64 adjoint at 1e-4."""
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
    ref = recurrence_grads_fp64(*[x.detach() for x in xt], D ** -0.5, do)
    for n, x, rg in zip(["dq", "dk", "dv", "dw", "db", "dg"], xt, ref):
        ok, e = within(x.grad, rg, 1e-4)
        assert ok, (n, e, float(rg.abs().max()))


def test_config4_training_bf16_all_pairs(dev):
    """The training path at configs[3]'s shape with bfloat16 q, k, v, w, b, float32 g,
    an N(0,1) cotangent on out and a unit N(0,1) cotangent on h_final; the six input
    gradients of all 48 pairs against the float64 adjoint on the bf16-rounded inputs
    at 2e-2."""
    B, T, H, D = 8, 8192, 6, 128
    xt = [x.detach().requires_grad_(True) for x in baseline_inputs(B, T, H, D, dev, seed=4)]
    gen = torch.Generator(device=dev).manual_seed(5)
    do = torch.randn((B, T, H, D), generator=gen, device=dev)
    dh = torch.randn((B, H, D, D), generator=gen, device=dev)
    out, hf = gp().gdn2_pallas_forward_trainable(*xt, D ** -0.5)
    torch.autograd.backward([out, hf], [do, dh])
    ref = recurrence_grads_fp64(*[x.detach() for x in xt], D ** -0.5, do, dh)
    for n, x, rg in zip(["dq", "dk", "dv", "dw", "db", "dg"], xt, ref):
        ok, e = within(x.grad, rg, 2e-2)
        assert ok, (n, e, float(rg.abs().max()))


def test_d256_forward_all_pairs(dev):
    """D = 256 (beyond the reference's D = 128 assert) at B8 T8192 H3, bf16 inputs,
    chunk 64: all 24 pairs against the float64 recurrence."""
    B, T, H, D = 8, 8192, 3, 256
    xt = baseline_inputs(B, T, H, D, dev, seed=6)
    out, hf = gp().gdn2_pallas_forward(*xt, D ** -0.5)
    ro, rh = recurrence_fp64(*xt, D ** -0.5)
    ok_o, e_o = within(out, ro, 2e-2)
    ok_h, e_h = within(hf, rh, 2e-2)
    assert ok_o and ok_h, (e_o, e_h)


def test_d256_training_all_pairs(dev):
    """D = 256 float32 training path at B8 T8192 H3 with an N(0,1) cotangent on out
    and on h_final: the six input gradients of all 24 pairs against the float64
    adjoint at 1e-4."""
    B, T, H, D = 8, 8192, 3, 256
    gen = torch.Generator(device=dev).manual_seed(7)
    r = lambda *s: torch.randn(s or (B, T, H, D), generator=gen, device=dev)
    q, k, v, w, b, g = r(), r(), r(), r(), r(), r()
    q, k = q / q.norm(dim=-1, keepdim=True), k / k.norm(dim=-1, keepdim=True)
    w, b, g = torch.sigmoid(w), torch.sigmoid(b), -torch.nn.functional.softplus(g)
    xt = [x.detach().requires_grad_(True) for x in (q, k, v, w, b, g)]
    do, dh = r(), r(B, H, D, D)
    out, hf = gp().gdn2_pallas_forward_trainable(*xt, D ** -0.5)
    torch.autograd.backward([out, hf], [do, dh])
    ref = recurrence_grads_fp64(*[x.detach() for x in xt], D ** -0.5, do, dh)
    for n, x, rg in zip(["dq", "dk", "dv", "dw", "db", "dg"], xt, ref):
        ok, e = within(x.grad, rg, 1e-4)
        assert ok, (n, e, float(rg.abs().max()))
