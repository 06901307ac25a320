"""Variable-length batches on the GPU (gdn2_pallas_forward_varlen /
gdn2_fwd_varlen): sequences of any length packed along T, each chunked and
scanned on its own from its own h0.  Every sequence is checked against the
float64 recurrence over its own tokens, and one sequence of whole chunks
against the plain forward.  Tolerances as the forward's."""
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


@pytest.mark.parametrize("dtype,BT,D,lens", [
    (torch.float32, 64, 64, [130, 0, 64, 17, 200]),          # tails, empty, exact, short
    (torch.bfloat16, 128, 128, [300, 128, 5, 257]),
    (torch.bfloat16, 64, 128, [1, 63, 65, 190]),
    (torch.bfloat16, 64, 256, [70, 1, 128]),
    (torch.float32, 64, 256, [100, 64]),
])
def test_varlen_matches_per_sequence_recurrence(dev, dtype, BT, D, lens):
    import gdn2_package as gp
    H, T = 2, sum(lens)
    xs = O.make_inputs(1, T, H, D, seed=len(lens) + BT)
    xt = [torch.tensor(x, device=dev) for x in xs]
    xt = [x.to(dtype) for x in xt[:5]] + [xt[5]]
    S = len(lens)
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    h0 = (0.2 * np.random.default_rng(3).standard_normal((S, H, D, D))).astype(np.float32)
    out, hf = gp.gdn2_pallas_forward_varlen(*xt, D ** -0.5, torch.tensor(cu),
                                            h0=torch.tensor(h0, device=dev), chunk_size=BT)
    assert out.shape == (1, T, H, D) and hf.shape == (S, H, D, D)
    host = [x.float().cpu().numpy() for x in xt]
    for s in range(S):
        a, e = cu[s], cu[s + 1]
        ro, rh = O.recurrent_fwd(*[x[:, a:e] for x in host], D ** -0.5, h0=h0[s:s + 1])
        if e > a:
            ok_o, e_o = close(out[:, a:e].cpu().numpy(), ro, TOL[dtype])
            assert ok_o, (s, "out", e_o)
        ok_h, e_h = close(hf[s:s + 1].cpu().numpy(), rh, TOL[dtype])
        assert ok_h, (s, "h_final", e_h)


def test_varlen_raw_inputs(dev):
    import gdn2_package as gp
    H, D, BT, lens = 2, 64, 64, [70, 40, 130]
    T = sum(lens)
    rng = np.random.default_rng(9)
    raw = [torch.tensor(rng.standard_normal((1, T, H, D)).astype(np.float32), device=dev)
           for _ in range(6)]
    cu = torch.tensor(np.concatenate([[0], np.cumsum(lens)]))
    out_r, hf_r = gp.gdn2_pallas_forward_varlen(*raw, 0.125, cu, chunk_size=BT, raw=True)
    f = torch.nn.functional
    act = [f.normalize(raw[0], dim=-1), f.normalize(raw[1], dim=-1), raw[2],
           torch.sigmoid(raw[3]), torch.sigmoid(raw[4]), -f.softplus(raw[5])]
    out_a, hf_a = gp.gdn2_pallas_forward_varlen(*act, 0.125, cu, chunk_size=BT)
    assert (out_r - out_a).abs().max().item() < 1e-4 and (hf_r - hf_a).abs().max().item() < 1e-4


def test_varlen_single_sequence_equals_forward(dev):
    import gdn2_package as gp
    B, T, H, D = 1, 512, 3, 128
    xs = O.make_inputs(B, T, H, D, seed=2)
    xt = [torch.tensor(x, device=dev) for x in xs]
    xt = [x.to(torch.bfloat16) for x in xt[:5]] + [xt[5]]
    o1, h1 = gp.gdn2_pallas_forward(*xt, D ** -0.5, chunk_size=128)
    o2, h2 = gp.gdn2_pallas_forward_varlen(*xt, D ** -0.5, torch.tensor([0, T]), chunk_size=128)
    assert torch.equal(o1, o2) and torch.equal(h1, h2[0:1])


def test_varlen_bad_tables_stay_in_bounds(dev):
    """The C entry point trusts its device tables only after clamping them:
    a table that points past the data gives garbage results, never an access
    outside the buffers (every output stays finite)."""
    import gdn2_package as gp
    from gdn2_package import _lib
    H, D, BT, T = 1, 64, 64, 128
    xs = [torch.zeros((1, T, H, D), device=dev) for _ in range(6)]
    out = torch.zeros((1, T, H, D), device=dev)
    hf = torch.zeros((2, H, D, D), device=dev)
    L = _lib.lib()
    nb = L.gdn2_fwd_varlen_workspace_bytes(2, H, D, BT, _lib.GDN2_F32)
    ws = torch.zeros(nb, dtype=torch.uint8, device=dev)
    cu = torch.tensor([0, 5, 1 << 30], dtype=torch.int32, device=dev)       # sequence 1 overflows
    cs = torch.tensor([0, 1 << 29, -7], dtype=torch.int32, device=dev)      # nonsense rows
    rc = L.gdn2_fwd_varlen(torch.cuda.current_stream().cuda_stream, 2, cu.data_ptr(), cs.data_ptr(),
                           2, T, H, D, BT, _lib.GDN2_F32, _lib.GDN2_F32,
                           *(x.data_ptr() for x in xs), None, 0.125, out.data_ptr(),
                           hf.data_ptr(), ws.data_ptr(), nb, 0)
    torch.cuda.synchronize()
    assert rc == 0 and torch.isfinite(out).all() and torch.isfinite(hf).all()


# ----------------------------------------------------------------------------- training
@pytest.mark.parametrize("dtype,D,lens,h0", [
    (torch.float32, 64, [70, 1, 128, 33], True),   # tails, one token, whole chunks
    (torch.float32, 128, [200, 64], False),
    (torch.bfloat16, 64, [100, 29], True),
    (torch.float32, 256, [90, 64], True),          # D = 256: the backward of per-chunk products
])
def test_varlen_trainable_matches_per_sequence_oracle(dev, dtype, D, lens, h0):
    """gdn2_pallas_forward_varlen_trainable: out, h_final and every gradient
    (q..g, h0) of each sequence against the float64 recurrence and its autograd
    over that sequence alone (oracle.recurrent_grads), with a unit-scale
    dh_final.  bfloat16 inputs are computed in float32 and return bfloat16
    gradients."""
    import gdn2_package as gp
    H, T, S = 2, sum(lens), len(lens)
    cu = np.concatenate([[0], np.cumsum(lens)])
    xs = O.make_inputs(1, T, H, D, seed=T + D)
    xt = [torch.tensor(np.asarray(x), device=dev).to(dtype if i < 5 else torch.float32)
          .requires_grad_(True) for i, x in enumerate(xs)]
    rng = np.random.default_rng(S + D)
    h0n = (0.2 * rng.standard_normal((S, H, D, D))).astype(np.float32) if h0 else None
    h0t = None if h0n is None else torch.tensor(h0n, device=dev, requires_grad=True)
    do = rng.standard_normal((1, T, H, D)).astype(np.float32)
    dh = rng.standard_normal((S, H, D, D)).astype(np.float32)
    out, hf = gp.gdn2_pallas_forward_varlen_trainable(*xt, D ** -0.5, cu, h0=h0t)
    assert out.shape == (1, T, H, D) and hf.shape == (S, H, D, D)
    ((out * torch.tensor(do, device=dev)).sum() + (hf * torch.tensor(dh, device=dev)).sum()).backward()
    xin = [x.detach().float().cpu().numpy() for x in xt]
    tol = TOL[dtype]
    for s in range(S):
        a, e = int(cu[s]), int(cu[s + 1])
        seg = [x[:, a:e] for x in xin]
        hs = None if h0n is None else h0n[s:s + 1]
        ro, rh = O.recurrent_fwd(*seg, D ** -0.5, h0=hs)
        assert close(out.detach()[:, a:e].cpu().numpy(), ro, tol)[0], ("out", s)
        assert close(hf.detach()[s:s + 1].cpu().numpy(), rh, tol)[0], ("h_final", s)
        ref = O.recurrent_grads(*seg, D ** -0.5, do[:, a:e], dh[s:s + 1], h0=hs)
        for name, x, r in zip("qkvwbg", xt, ref[:6]):
            ok, err = close(x.grad[:, a:e].float().cpu().numpy(), r, tol)
            assert ok, (name, s, err)
        if h0t is not None:
            ok, err = close(h0t.grad[s:s + 1].cpu().numpy(), ref[6], tol)
            assert ok, ("h0", s, err)
