"""Pins for the CPU oracle (oracle/gdn2_oracle.py) -- CPU only.

The reference ships no numeric fixtures and cannot run here (JAX/Pallas-TPU),
so the oracle is pinned by mathematics: closed forms of special cases, a
brute-force kernel A, scipy's triangular solve for kernel B, agreement of three
independent restatements, invariants (chunk size, h0 chaining, linearity),
torch.autograd + finite differences for the backward, and mutation tests that
plant a plausible mistake in a copy and check that a pin catches it.
"""
import numpy as np
import pytest
import scipy.linalg

from oracle import gdn2_oracle as O


def inputs(B=1, T=64, H=2, D=8, seed=0, g_scale=1.0):
    return O.make_inputs(B, T, H, D, seed=seed, g_scale=g_scale, dtype=np.float64)


def maxerr(a, b):
    return float(np.max(np.abs(np.asarray(a) - np.asarray(b))))


# --------------------------------------------------------------------------- sanitize
def test_sanitize_semantics():
    # gdn2_fwd.py:42-44: nan -> 0, +-inf -> +-CLIP, clip to [-CLIP, CLIP]
    x = np.array([np.nan, np.inf, -np.inf, 2e4, -3e4, -3.0, 0.5])
    np.testing.assert_array_equal(O.sanitize(x), [0.0, 1e4, -1e4, 1e4, -1e4, -3.0, 0.5])


# --------------------------------------------------------------------------- closed forms
def test_linear_attention_closed_form():
    """b = 0, g = 0: o = scale * tril(Q K^T) (W * V) per (batch, head)."""
    q, k, v, w, b, g = inputs(T=40)
    b = np.zeros_like(b)
    g = np.zeros_like(g)
    s = 0.3
    out, h = O.recurrent_fwd(q, k, v, w, b, g, s)
    for bb in range(q.shape[0]):
        for hh in range(q.shape[2]):
            Q, K, WV = q[bb, :, hh], k[bb, :, hh], (w * v)[bb, :, hh]
            ref = s * np.tril(Q @ K.T) @ WV
            assert maxerr(out[bb, :, hh], ref) < 1e-12
            assert maxerr(h[bb, hh], K.T @ WV) < 1e-12


def test_gated_linear_attention_closed_form():
    """b = 0: o_t = scale sum_{s<=t} sum_d q_t k_s exp(G_t - G_s) (w v)_s, G = cumsum(g)."""
    q, k, v, w, b, g = inputs(T=24, g_scale=0.3)
    b = np.zeros_like(b)
    s = 0.7
    out, _ = O.recurrent_fwd(q, k, v, w, b, g, s)
    G = np.cumsum(g, axis=1)
    T = q.shape[1]
    ref = np.zeros_like(out)
    for t in range(T):
        for u in range(t + 1):
            coef = np.sum(q[:, t] * k[:, u] * np.exp(G[:, t] - G[:, u]), axis=-1)  # (B,H)
            ref[:, t] += s * coef[..., None] * (w * v)[:, u]
    assert maxerr(out, ref) < 1e-12


def test_deltanet_special_case():
    """g = 0, b = w = beta (constant over D): the textbook delta rule
    M_t = M_{t-1} + beta_t (v_t - M_{t-1} k_t) k_t^T, o_t = scale M_t q_t."""
    q, k, v, w, b, g = inputs(T=32)
    beta = 1.0 / (1.0 + np.exp(-np.random.default_rng(3).standard_normal(q.shape[:3])))
    bw = np.repeat(beta[..., None], q.shape[-1], axis=-1)
    s = 0.5
    out, h = O.recurrent_fwd(q, k, v, bw, bw, np.zeros_like(g), s)
    B, T, H, D = q.shape
    for bb in range(B):
        for hh in range(H):
            M = np.zeros((D, D))  # (Dv, Dk)
            for t in range(T):
                kt, vt, qt = k[bb, t, hh], v[bb, t, hh], q[bb, t, hh]
                M = M + beta[bb, t, hh] * np.outer(vt - M @ kt, kt)
                assert maxerr(out[bb, t, hh], s * M @ qt) < 1e-12
            assert maxerr(h[bb, hh], M.T) < 1e-12


def test_single_token_closed_form():
    """T = 1 with h0: S_1 = (I - k (b*k)^T) Diag(e^g) h0 + k (w*v)^T, o = scale S_1^T q."""
    q, k, v, w, b, g = inputs(T=1, D=6)
    h0 = np.random.default_rng(1).standard_normal((1, 2, 6, 6))
    s = 0.9
    out, h = O.recurrent_fwd(q, k, v, w, b, g, s, h0=h0)
    for hh in range(2):
        kk, bb_, gg = k[0, 0, hh], b[0, 0, hh], g[0, 0, hh]
        S1 = (np.eye(6) - np.outer(kk, bb_ * kk)) @ np.diag(np.exp(gg)) @ h0[0, hh] \
            + np.outer(kk, (w * v)[0, 0, hh])
        assert maxerr(h[0, hh], S1) < 1e-13
        assert maxerr(out[0, 0, hh], s * S1.T @ q[0, 0, hh]) < 1e-13


def test_scalar_state_closed_form():
    """D = 1: s_T = sum_t (prod_{u>t} a_u) c_t with a = (1 - b k^2) e^g, c = k w v."""
    rng = np.random.default_rng(4)
    T = 50
    q, k, v = (rng.standard_normal((1, T, 1, 1)) for _ in range(3))
    w, b = (1 / (1 + np.exp(-rng.standard_normal((1, T, 1, 1)))) for _ in range(2))
    g = -np.logaddexp(0, rng.standard_normal((1, T, 1, 1))) * 0.2
    out, h = O.recurrent_fwd(q, k, v, w, b, g, 1.0)
    a = ((1 - b * k * k) * np.exp(g)).ravel()
    c = (k * w * v).ravel()
    st = np.array([sum(np.prod(a[u + 1:t + 1]) * c[u] for u in range(t + 1)) for t in range(T)])
    assert maxerr(out.ravel(), q.ravel() * st) < 1e-12
    assert maxerr(h.ravel()[0], st[-1]) < 1e-12


def test_full_reset_limit():
    """g -> -inf: the state forgets every step, o_t = scale (q_t . k_t)(w_t * v_t)."""
    q, k, v, w, b, g = inputs(T=16)
    g = np.full_like(g, -1e3)
    out, _ = O.recurrent_fwd(q, k, v, w, b, g, 0.4)
    ref = 0.4 * np.sum(q * k, axis=-1, keepdims=True) * (w * v)
    assert maxerr(out, ref) < 1e-12


# --------------------------------------------------------------------------- kernels A-C
def test_kernel_a_brute_force_with_clip():
    rng = np.random.default_rng(5)
    BT, D = 8, 4
    q, k, b = (rng.standard_normal((1, BT, D)) for _ in range(3))
    g = -np.abs(rng.standard_normal((1, BT, D))) * 8.0   # pairs beyond the +-20 clip
    gc = np.cumsum(g, axis=-2)
    aqk, akk = O.chunk_scores(q, k, b, gc, 0.25, clip=True)
    assert np.any(gc[0, :, None, :] - gc[0, None, :, :] < -20)
    for i in range(BT):
        for j in range(BT):
            e = np.exp(np.clip(gc[0, i] - gc[0, j], -20, 20))
            rq = 0.25 * np.sum(q[0, i] * k[0, j] * e) if j <= i else 0.0
            rk = np.sum(b[0, i] * k[0, i] * k[0, j] * e) if j < i else 0.0
            assert abs(aqk[0, i, j] - rq) < 1e-12
            assert abs(akk[0, i, j] - rk) < 1e-12


@pytest.mark.parametrize("BT,BC", [(32, None), (64, 32), (64, None)])
def test_kernel_b_matches_triangular_solve(BT, BC):
    q, k, v, w, b, g = inputs(T=BT, D=16)
    gc = np.cumsum(O.to_chunks(g, BT), axis=-2)
    _, akk = O.chunk_scores(O.to_chunks(q, BT), O.to_chunks(k, BT), O.to_chunks(b, BT), gc, 1.0)
    A = O.wy_solve(akk, BC)
    for idx in np.ndindex(akk.shape[:-2]):
        ref = scipy.linalg.solve_triangular(np.eye(BT) + akk[idx], np.eye(BT), lower=True,
                                            unit_diagonal=True)
        assert maxerr(A[idx], ref) < 1e-12


def test_kernel_c_solves_wy_system():
    """w_pseudo and u solve (I + Akk) X = (b k e^gc), (w v) -- checked by scipy."""
    BT = 32
    q, k, v, w, b, g = (O.to_chunks(x, BT) for x in inputs(T=BT, D=8))
    gc = np.cumsum(g, axis=-2)
    _, akk = O.chunk_scores(q, k, b, gc, 1.0)
    A = O.wy_solve(akk)
    wp, u, kg, qg, gl = O.recompute_wy(q, k, v, w, b, gc, A)
    for idx in np.ndindex(akk.shape[:-2]):
        L = np.eye(BT) + akk[idx]
        assert maxerr(L @ wp[idx], (b * k * np.exp(gc))[idx]) < 1e-12
        assert maxerr(L @ u[idx], (w * v)[idx]) < 1e-12
    assert maxerr(gl, gc[..., -1, :]) == 0.0
    assert maxerr(kg * np.exp(gc - gl[..., None, :]), k) < 1e-12


# --------------------------------------------------------------------------- restatements agree
@pytest.mark.parametrize("BT", [16, 32, 64])
def test_chunked_equals_recurrent(BT):
    q, k, v, w, b, g = inputs(B=2, T=128, H=2, D=16)
    h0 = np.random.default_rng(2).standard_normal((2, 2, 16, 16)) * 0.2
    ro, rh = O.recurrent_fwd(q, k, v, w, b, g, 0.25, h0=h0)
    co, ch = O.chunked_fwd(q, k, v, w, b, g, 0.25, h0=h0, BT=BT, clip=False)
    assert maxerr(co, ro) < 1e-12 and maxerr(ch, rh) < 1e-12
    ao, ah = O.assoc_scan_fwd(q, k, v, w, b, g, 0.25, h0=h0, BT=BT)
    assert maxerr(ao, ro) < 1e-12 and maxerr(ah, rh) < 1e-12


def test_reference_clip_is_tiny_in_domain():
    q, k, v, w, b, g = inputs(B=1, T=128, H=2, D=16)
    ro, rh = O.recurrent_fwd(q, k, v, w, b, g, 0.25)
    co, ch = O.chunked_fwd(q, k, v, w, b, g, 0.25, BT=64, BC=32, clip=True)
    assert maxerr(co, ro) < 1e-6 and maxerr(ch, rh) < 1e-6


def test_h0_chaining():
    q, k, v, w, b, g = inputs(T=128, D=16)
    full_o, full_h = O.chunked_fwd(q, k, v, w, b, g, 0.3, BT=32, clip=False)
    o1, h1 = O.chunked_fwd(*(x[:, :64] for x in (q, k, v, w, b, g)), 0.3, BT=32, clip=False)
    o2, h2 = O.chunked_fwd(*(x[:, 64:] for x in (q, k, v, w, b, g)), 0.3, h0=h1, BT=32,
                           clip=False)
    assert maxerr(np.concatenate([o1, o2], axis=1), full_o) < 1e-12
    assert maxerr(h2, full_h) < 1e-12


def test_linearity_in_v_and_h0():
    q, k, v, w, b, g = inputs(T=64, D=8)
    rng = np.random.default_rng(9)
    v2 = rng.standard_normal(v.shape)
    h01, h02 = rng.standard_normal((2, 1, 2, 8, 8))
    f = lambda vv, hh: O.recurrent_fwd(q, k, vv, w, b, g, 0.5, h0=hh)
    o1, s1 = f(v, h01)
    o2, s2 = f(v2, h02)
    o3, s3 = f(v + 2.5 * v2, h01 + 2.5 * h02)
    assert maxerr(o3, o1 + 2.5 * o2) < 1e-11 and maxerr(s3, s1 + 2.5 * s2) < 1e-11


# --------------------------------------------------------------------------- backward
def _torch_recurrence(q, k, v, w, b, g, scale, h0):
    import torch
    S = h0
    outs = []
    for t in range(q.shape[1]):
        S = torch.exp(g[:, t])[..., None] * S
        pred = torch.einsum("bhd,bhde->bhe", b[:, t] * k[:, t], S)
        S = S + torch.einsum("bhd,bhe->bhde", k[:, t], w[:, t] * v[:, t] - pred)
        outs.append(scale * torch.einsum("bhd,bhde->bhe", q[:, t], S))
    return torch.stack(outs, 1), S


@pytest.mark.parametrize("BT", [16, 32])
def test_backward_matches_autograd(BT):
    import torch
    q, k, v, w, b, g = inputs(B=1, T=64, H=2, D=8, seed=3)
    rng = np.random.default_rng(6)
    h0 = rng.standard_normal((1, 2, 8, 8)) * 0.3
    do = rng.standard_normal(q.shape)
    dh = rng.standard_normal(h0.shape)
    ts = [torch.tensor(x, requires_grad=True) for x in (q, k, v, w, b, g, h0)]
    o, h = _torch_recurrence(*ts[:6], 0.35, ts[6])
    ((o * torch.tensor(do)).sum() + (h * torch.tensor(dh)).sum()).backward()
    got = O.chunked_bwd(q, k, v, w, b, g, 0.35, do, dh, h0=h0, BT=BT, clip=False)
    for name, gv, t in zip("q k v w b g h0".split(), got, ts):
        ref = t.grad.numpy()
        assert maxerr(gv, ref) < 1e-10 * max(1.0, np.abs(ref).max()), name


def test_recurrent_grads_match_chunked_bwd_and_finite_differences():
    """recurrent_grads (autograd of the token recurrence, any T) against
    chunked_bwd at a whole number of chunks and against a central finite
    difference in one coordinate of each input."""
    q, k, v, w, b, g = inputs(B=1, T=64, H=2, D=8, seed=4)
    rng = np.random.default_rng(9)
    h0 = rng.standard_normal((1, 2, 8, 8)) * 0.3
    do = rng.standard_normal(q.shape)
    dh = rng.standard_normal(h0.shape)
    got = O.recurrent_grads(q, k, v, w, b, g, 0.35, do, dh, h0=h0)
    ref = O.chunked_bwd(q, k, v, w, b, g, 0.35, do, dh, h0=h0, BT=32, clip=False)
    for gv, rv in zip(got, ref):
        assert maxerr(gv, rv) < 1e-10 * max(1.0, np.abs(rv).max())
    q2, k2, v2, w2, b2, g2 = inputs(B=1, T=37, H=1, D=4, seed=2)
    h02 = rng.standard_normal((1, 1, 4, 4)) * 0.3
    do2 = rng.standard_normal(q2.shape)
    dh2 = rng.standard_normal(h02.shape)
    got2 = O.recurrent_grads(q2, k2, v2, w2, b2, g2, 0.35, do2, dh2, h0=h02)
    xs2 = [q2, k2, v2, w2, b2, g2, h02]
    def loss2(ys):
        o, h = O.recurrent_fwd(*ys[:6], 0.35, h0=ys[6])
        return float((o * do2).sum() + (h * dh2).sum())
    for i, gv in enumerate(got2):
        idx = (0, 36, 0, 3) if i < 6 else (0, 0, 2, 1)
        eps = 1e-6
        up = [x.copy() for x in xs2]
        dn = [x.copy() for x in xs2]
        up[i][idx] += eps
        dn[i][idx] -= eps
        fd = (loss2(up) - loss2(dn)) / (2 * eps)
        assert abs(gv[idx] - fd) < 1e-6 * max(1.0, abs(fd)), (i, gv[idx], fd)


def test_backward_finite_differences():
    q, k, v, w, b, g = inputs(B=1, T=32, H=1, D=4, seed=8)
    rng = np.random.default_rng(7)
    do = rng.standard_normal(q.shape)
    grads = O.chunked_bwd(q, k, v, w, b, g, 0.6, do, BT=16, clip=False)
    base = [q, k, v, w, b, g]
    loss = lambda xs: float(np.sum(O.recurrent_fwd(*xs, 0.6)[0] * do))
    eps = 1e-6
    for which in range(6):
        for idx in [(0, 3, 0, 1), (0, 17, 0, 2), (0, 31, 0, 0)]:
            xp = [x.copy() for x in base]
            xm = [x.copy() for x in base]
            xp[which][idx] += eps
            xm[which][idx] -= eps
            fd = (loss(xp) - loss(xm)) / (2 * eps)
            assert abs(fd - grads[which][idx]) < 1e-6 * max(1.0, abs(fd)), (which, idx)


# --------------------------------------------------------------------------- mutation tests
def _fwd_close(mod):
    q, k, v, w, b, g = inputs(B=1, T=64, H=1, D=8, seed=11)
    ro, rh = mod.recurrent_fwd(q, k, v, w, b, g, 0.5)
    co, ch = mod.chunked_fwd(q, k, v, w, b, g, 0.5, BT=32, clip=False)
    return maxerr(co, ro) < 1e-9 and maxerr(ch, rh) < 1e-9


def test_mutation_transposed_akk_is_caught(monkeypatch):
    orig = O.chunk_scores
    monkeypatch.setattr(O, "chunk_scores", lambda *a, **kw: (orig(*a, **kw)[0],
                                                               np.swapaxes(orig(*a, **kw)[1],
                                                                           -1, -2)))
    assert not _fwd_close(O)


def test_mutation_wrong_kg_sign_is_caught(monkeypatch):
    orig = O.recompute_wy

    def bad(q, k, v, w, b, gc, A):
        wp, u, kg, qg, gl = orig(q, k, v, w, b, gc, A)
        return wp, u, k * np.exp(gc - gl[..., None, :]), qg, gl
    monkeypatch.setattr(O, "recompute_wy", bad)
    assert not _fwd_close(O)


def test_mutation_dropped_erase_term_is_caught(monkeypatch):
    """A recurrence that forgets the b*k erase term fails the DeltaNet/chunked pins."""
    orig = O.recurrent_fwd
    monkeypatch.setattr(O, "recurrent_fwd",
                        lambda q, k, v, w, b, g, s, h0=None: orig(q, k, v, w, 0 * b, g, s, h0))
    assert not _fwd_close(O)


def test_mutation_missing_last_row_dgl_is_caught(monkeypatch):
    """Dropping the state-decay term of dgc_last (gdn2_bwd.py:196-201) breaks dg."""
    import torch
    orig = O._wy_dqkg_backward

    def bad(*a):
        res = orig(*a)
        q, k, b, w, v, gc, A, h_pre, v_new, do, dv, dh_next, scale = a
        gl = gc[..., -1, :]
        res["dgc"] = res["dgc"].copy()
        res["dgc"][..., -1, :] -= np.exp(gl) * np.sum(dh_next * h_pre, axis=-1)
        return res
    monkeypatch.setattr(O, "_wy_dqkg_backward", bad)
    # >= 3 chunks (the term needs a nonzero incoming state and dh from the right) and
    # slow decay (it carries exp(gc_last), ~e^-25 per 32 tokens at the default scale)
    q, k, v, w, b, g = inputs(B=1, T=128, H=1, D=8, seed=12, g_scale=0.02)
    do = np.random.default_rng(1).standard_normal(q.shape)
    ts = [torch.tensor(x, requires_grad=True) for x in (q, k, v, w, b, g)]
    o, _ = _torch_recurrence(*ts, 0.5, torch.zeros(1, 1, 8, 8, dtype=torch.float64))
    (o * torch.tensor(do)).sum().backward()
    got = O.chunked_bwd(q, k, v, w, b, g, 0.5, do, BT=32, clip=False)
    assert maxerr(got[5], ts[5].grad.numpy()) > 1e-6


# --------------------------------------------------------------------------- saturation order
def test_b4_pair_loop_equals_whole_sums_in_domain():
    """B4's sub-block pair loop (ref gdn2_bwd.py:287-328) sums the same terms as
    the whole-chunk form: with every partial sum inside the clip, 1, 2 and 4
    sub-blocks and the unclipped whole sums agree (the whole sums are pinned to
    torch.autograd through chunked_bwd above)."""
    q, k, v, w, b, g = inputs(B=1, T=64, H=2, D=8, seed=21)
    rng = np.random.default_rng(5)
    qs, ks, bs = (O.to_chunks(x, 32) for x in (q, k, b))
    gc = np.cumsum(O.to_chunks(g, 32), axis=-2)
    daqk = rng.standard_normal(qs.shape[:-1] + (32,))
    dakk = rng.standard_normal(qs.shape[:-1] + (32,))
    ref = O._intra_backward(daqk, dakk, qs, ks, bs, gc, 0.4, clip=False, n_sub=None)
    for ns in (1, 2, 4):
        got = O._intra_backward(daqk, dakk, qs, ks, bs, gc, 0.4, clip=False, n_sub=ns)
        for gv, rv in zip(got, ref):
            assert maxerr(gv, rv) < 1e-12, ns


def test_b4_pair_loop_clip_order_known_answer():
    """Known answer, worked by hand from ref gdn2_bwd.py:287-339 with two
    one-token sub-blocks (BT = 2, D = 1, gc = 0, scale = 1): q = (2, 1),
    k = (1, 2), b = (0.5, 0.5), dAqk = [[1.5e4, .], [-4e3, 7e3]], dAkk[1][0] = 2e3.
      pair (0,0): dq0 = c(1.5e4) = 1e4, dk0 = c(3e4) = 1e4, dgc0 = c(c(3e4) - 3e4) = -1e4
      pair (1,0): dq1 = -4e3, dbk1 = 2e3, dk0 = c(1e4 - 4e3 + 2e3) = 8e3,
                  dgc1 = c(-4e3 + 2e3) = -2e3, dgc0 = c(-1e4 + 4e3 - 2e3) = -8e3
      pair (1,1): dq1 = c(-4e3 + 1.4e4) = 1e4, dk1 = 7e3,
                  dgc1 = c(c(-2e3 + 1.4e4) - 1.4e4) = -4e3
      outputs:    dk = (8e3, 7e3 + 2e3 * 0.5), db = (0, 2e3 * 2)
    Clipping each output once instead (the whole sums) gives dk0 = 1e4,
    dgc = (2e3, -2e3): the known answer catches a dropped accumulator clip."""
    q = np.array([[[2.0], [1.0]]])
    k = np.array([[[1.0], [2.0]]])
    b = np.full((1, 2, 1), 0.5)
    gc = np.zeros((1, 2, 1))
    daqk = np.array([[[1.5e4, 9e9], [-4e3, 7e3]]])     # 9e9: masked (right of the diagonal)
    dakk = np.array([[[9e9, 9e9], [2e3, 9e9]]])
    want = ([1e4, 1e4], [8e3, 8e3], [0.0, 4e3], [-8e3, -4e3])
    got = O._intra_backward(daqk, dakk, q, k, b, gc, 1.0, clip=True, n_sub=2)
    for gv, wv in zip(got, want):
        np.testing.assert_array_equal(gv.ravel(), wv)
    whole = O._intra_backward(daqk, dakk, q, k, b, gc, 1.0, clip=True, n_sub=None)
    assert whole[1].ravel()[0] == 1e4 and list(whole[3].ravel()) == [2e3, -2e3]


def test_raw_dh_final_reaches_b3_known_answer():
    """B1 carries sanitize(dh_final) (ref gdn2_bwd.py:53) but B3 receives the raw
    dh_final as the last chunk's dh' (gdn2_pipeline.py:52-56,105).  One live
    token (the last of a 16-token chunk; the others have k = q = 0 and g = 0, so
    they leave the state and the gradients alone), D = 1, k = v = 1, w = 0.1,
    b = 0.5, do = 0, h0 = 0, dh_final = 5e4.  By hand: v_new = w v = 0.1, W = 0.5;
    B1: dh = 1e4, dv_new = kg dh = 1e4, dh0 = c(1e4 - W dv_new) = 5e3;
    B3: dkg = v_new dh' = 5e3 (5e4 raw; 1e3 from the sanitized value), so
    dk = 5e3, dv = w d(wv) = 1e3, dw = v d(wv) = 1e4, and dg = 0 (the last
    token's -dkg kg cancels against its g_last term)."""
    x = [np.zeros((1, 16, 1, 1)) for _ in range(6)]
    x[1][:, 15] = 1.0
    x[2][:, 15] = 1.0
    x[3][:, 15] = 0.1
    x[4][:, 15] = 0.5
    got = O.chunked_bwd(*x, 1.0, np.zeros((1, 16, 1, 1)),
                        dh_final=np.full((1, 1, 1, 1), 5e4), BT=16)
    want = [0.0, 5e3, 1e3, 1e4, 0.0, 0.0]
    for i, wv in enumerate(want):
        assert abs(got[i][0, 15, 0, 0] - wv) < 1e-9 and np.all(got[i][0, :15] == 0), i
    assert abs(got[6].item() - 5e3) < 1e-9
