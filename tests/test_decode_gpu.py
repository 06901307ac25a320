"""Single-token decode step (gdn2_decode_step / gdn2_decode) on the GPU.

It is the forward with a one-token chunk on the (B,H,D,D) state, so it is
checked against the float64 token recurrence (oracle.recurrent_fwd, T = 1) and
against the chunked forward itself: a prefix through gdn2_pallas_forward, then
the remaining tokens one by one from its h_final, must reproduce the forward
over the whole sequence.  Tolerances as the forward's (1e-4 float32, 2e-2
bfloat16)."""
import numpy as np
import pytest
import torch

from oracle import gdn2_oracle as O

pytestmark = pytest.mark.gpu
TOL = {torch.float32: 1e-4, torch.bfloat16: 2e-2}


def close(got, ref, tol):
    got, ref = np.asarray(got, np.float64), np.asarray(ref, np.float64)
    return float((np.abs(got - ref) - (tol + tol * np.abs(ref))).max()) <= 0.0, \
        float(np.abs(got - ref).max())


def dev_inputs(xs, dev, dtype):
    t = [torch.tensor(np.asarray(x), device=dev) for x in xs]
    return [x.to(dtype) for x in t[:5]] + [t[5]]


@pytest.mark.parametrize("D,dtype,with_state", [(128, torch.float32, True), (64, torch.float32, False),
                                                (128, torch.bfloat16, True), (64, torch.bfloat16, True),
                                                (256, torch.float32, True), (256, torch.bfloat16, False)])
def test_one_token_matches_recurrence(dev, D, dtype, with_state):
    import gdn2_package as gp
    B, H = 2, 3
    xs = O.make_inputs(B, 1, H, D, seed=D)
    h0 = (0.3 * np.random.default_rng(1).standard_normal((B, H, D, D))).astype(np.float32) \
        if with_state else None
    xt = dev_inputs(xs, dev, dtype)
    st = None if h0 is None else torch.tensor(h0, device=dev)
    out, s1 = gp.gdn2_decode_step(*xt, D ** -0.5, state=st)
    ro, rh = O.recurrent_fwd(*[x.float().cpu().numpy() for x in xt], D ** -0.5, h0=h0)
    ok_o, e_o = close(out.cpu().numpy(), ro, TOL[dtype])
    ok_h, e_h = close(s1.cpu().numpy(), rh, TOL[dtype])
    assert out.shape == (B, 1, H, D) and s1.shape == (B, H, D, D)
    assert ok_o and ok_h, (e_o, e_h)
    if st is not None:
        assert torch.equal(st, torch.tensor(h0, device=dev))   # not in place by default


@pytest.mark.parametrize("dtype,BT,D", [(torch.float32, 64, 128), (torch.bfloat16, 128, 128),
                                        (torch.bfloat16, 64, 64), (torch.bfloat16, 64, 256)])
def test_prefix_then_decode_equals_forward(dev, dtype, BT, D):
    """forward(prefix) -> decode 24 tokens == forward(prefix + 24 tokens)."""
    import gdn2_package as gp
    B, H, T0, NT = 2, 2, 2 * BT, 24
    T = T0 + BT            # the full forward needs whole chunks; compare the first NT new tokens
    xs = O.make_inputs(B, T, H, D, seed=7)
    xt = dev_inputs(xs, dev, dtype)
    out_full, _ = gp.gdn2_pallas_forward(*xt, D ** -0.5, chunk_size=BT)
    _, h = gp.gdn2_pallas_forward(*[x[:, :T0] for x in xt], D ** -0.5, chunk_size=BT)
    outs = []
    for t in range(T0, T0 + NT):
        o, h = gp.gdn2_decode_step(*[x[:, t:t + 1] for x in xt], D ** -0.5, state=h)
        outs.append(o)
    got = torch.cat(outs, 1).cpu().numpy()
    ok, err = close(got, out_full[:, T0:T0 + NT].cpu().numpy(), 1e-4 if dtype == torch.float32 else 2e-2)
    assert ok, err
    # and against the recurrence over the whole prefix + decoded span
    ro, _ = O.recurrent_fwd(*[x[:, :T0 + NT].float().cpu().numpy() for x in xt], D ** -0.5)
    ok, err = close(got, ro[:, T0:], TOL[dtype])
    assert ok, err


def test_inplace_state_and_3d_inputs(dev):
    import gdn2_package as gp
    B, H, D = 3, 2, 64
    xs = O.make_inputs(B, 1, H, D, seed=3)
    xt = [x[:, 0] for x in dev_inputs(xs, dev, torch.float32)]      # (B,H,D)
    st = (0.1 * torch.randn((B, H, D, D), device=dev)).contiguous()
    ref_out, ref_state = gp.gdn2_decode_step(*xt, 0.2, state=st.clone())
    out, s = gp.gdn2_decode_step(*xt, 0.2, state=st, inplace=True)
    assert s.data_ptr() == st.data_ptr() and out.shape == (B, H, D)
    assert torch.equal(out, ref_out) and torch.equal(st, ref_state)
