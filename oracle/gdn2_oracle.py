"""CPU oracle for GDN-2 (Gated DeltaNet-2) chunked linear attention.

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this module, and only as the
checker (or, for ``bench.py``, as the timed CPU baseline).  The product path
(``gdn2_package``) never imports it and raises when the HIP library is missing.

Three independent restatements live here, all in numpy:

* ``recurrent_fwd``   -- the token-level recurrence in float64.  Per (batch, head),
  with state ``S`` of shape (Dk, Dv)::

      S_t = (I - k_t (b_t * k_t)^T) Diag(exp g_t) S_{t-1} + k_t (w_t * v_t)^T
      o_t = scale * S_t^T q_t

  This is the math the reference's chunked kernels implement (the WY form of
  gdn2_fwd.py:99-366 reduces to it exactly; see ``chunked_fwd``).
* ``chunked_fwd`` / ``chunked_bwd`` -- a restatement of the reference's own
  chunked algorithm: kernels A (gdn2_fwd.py:93-139), B (gdn2_fwd.py:174-243),
  C (gdn2_fwd.py:264-295), D (gdn2_fwd.py:338-366) and backward kernels
  B1-B5 (gdn2_bwd.py:26-339) assembled as gdn2_pipeline.py:70-137 does, with the
  reference's decay clip (+-20) and sanitize (clip +-1e4, nan->0) semantics.
  The backward uses the chunk-last-axis layout the math requires; the shipped
  pipeline mis-indexes the chunk-first outputs of gdn2_fwd.py:391-397.
* ``assoc_scan_fwd`` -- the chunk recurrence as an associative scan of affine
  maps ``h -> M_c h + N_c`` (log-depth prefix composition).  The reference's
  benchmark baseline is a ``jax.associative_scan`` reference that is not in the
  repository (tests/test_reference.py:4 imports a module that does not exist),
  so this is a restatement from the math, not from its source.

How each function is pinned (tests/test_oracle.py): closed forms (linear
attention, gated linear attention, DeltaNet, T=1, D=1, full reset), brute-force
triple loops for kernel A, ``scipy.linalg.solve_triangular`` for kernel B,
chunk-size invariance, h0 chaining, joint linearity in (v, h0), agreement of the
three restatements with one another, ``torch.autograd`` of ``recurrent_fwd`` and
finite differences for ``chunked_bwd``, and mutation tests that plant a wrong
sign / transposed operand in a copy and check that a pin fails.  The reference
ships no golden vectors or numeric fixtures (its tests check shapes only), and
JAX is not installed, so the reference itself cannot pin anything numerically.
"""

from __future__ import annotations

import numpy as np

# Reference constants: gdn2_fwd.py:29-33, gdn2_pipeline.py:34.
CLIP = 1e4
DECAY_CLIP = 20.0
MB = 16

__all__ = [
    "CLIP", "sanitize", "make_inputs", "recurrent_fwd", "recurrent_grads", "chunk_scores", "wy_solve",
    "recompute_wy", "inter_chunk_combine", "chunked_fwd", "chunked_bwd",
    "assoc_scan_fwd", "to_chunks", "from_chunks",
]


def sanitize(x):
    """gdn2_fwd.py:42-44 (also _sanitize_h0 :334-335, _clip_acc gdn2_bwd.py:26-28,
    _final_sanitize gdn2_pipeline.py:37-41 -- all four are the same map)."""
    return np.nan_to_num(np.clip(x, -CLIP, CLIP), nan=0.0, posinf=CLIP, neginf=-CLIP)


# ----------------------------------------------------------------------------
# Synthetic inputs (distributions from BASELINE.json configs).
# ----------------------------------------------------------------------------
def make_inputs(B, T, H, D, seed=0, g_scale=1.0, dtype=np.float32):
    """Draw q,k,v,w,b,g in that order from ``numpy.random.default_rng(seed)``.

    q,k ~ N(0,1) L2-normalised over D; v ~ N(0,1); w,b = sigmoid(N(0,1));
    g = -softplus(N(0,1)) * g_scale.  Returns float32 arrays (B,T,H,D) unless
    ``dtype`` says otherwise.
    """
    rng = np.random.default_rng(seed)
    shape = (B, T, H, D)
    q = rng.standard_normal(shape)
    k = rng.standard_normal(shape)
    v = rng.standard_normal(shape)
    w = rng.standard_normal(shape)
    b = rng.standard_normal(shape)
    g = rng.standard_normal(shape)
    q = q / np.linalg.norm(q, axis=-1, keepdims=True)
    k = k / np.linalg.norm(k, axis=-1, keepdims=True)
    w = 1.0 / (1.0 + np.exp(-w))
    b = 1.0 / (1.0 + np.exp(-b))
    g = -np.logaddexp(0.0, g) * g_scale
    return tuple(x.astype(dtype) for x in (q, k, v, w, b, g))


# ----------------------------------------------------------------------------
# Token recurrence (float64).
# ----------------------------------------------------------------------------
def recurrent_fwd(q, k, v, w, b, g, scale, h0=None):
    """Token-by-token GDN-2 recurrence in float64.

    Inputs (B,T,H,D); returns out (B,T,H,D) and h_final (B,H,D,D) with the
    state indexed h[b,h,dk,dv] as in gdn2_fwd.py:342,355-357.
    """
    q, k, v, w, b, g = (np.asarray(x, dtype=np.float64) for x in (q, k, v, w, b, g))
    B, T, H, D = q.shape
    Dv = v.shape[-1]
    S = np.zeros((B, H, D, Dv)) if h0 is None else np.array(h0, dtype=np.float64)
    out = np.empty((B, T, H, Dv))
    for t in range(T):
        S = np.exp(g[:, t])[..., None] * S
        pred = np.einsum("bhd,bhde->bhe", b[:, t] * k[:, t], S)
        delta = w[:, t] * v[:, t] - pred
        S = S + np.einsum("bhd,bhe->bhde", k[:, t], delta)
        out[:, t] = scale * np.einsum("bhd,bhde->bhe", q[:, t], S)
    return out, S


def recurrent_grads(q, k, v, w, b, g, scale, do, dh_final=None, h0=None):
    """Gradients (dq,dk,dv,dw,db,dg,dh0) of ``recurrent_fwd`` for the loss
    sum(out * do) + sum(h_final * dh_final), by torch.autograd in float64 on the
    CPU.  Valid for any T (chunk sizes play no part), which ``chunked_bwd``'s
    16-token sub-blocks do not allow; no clipping (the reference's clip is
    inactive at test magnitudes)."""
    import torch
    xs = [torch.tensor(np.asarray(x, dtype=np.float64), requires_grad=True)
          for x in (q, k, v, w, b, g)]
    B, T, H, D = xs[0].shape
    Dv = xs[2].shape[-1]
    S0 = torch.zeros((B, H, D, Dv), dtype=torch.float64) if h0 is None else \
        torch.tensor(np.asarray(h0, dtype=np.float64))
    S0.requires_grad_(True)
    qt, kt, vt, wt, bt, gt = xs
    S, outs = S0, []
    for t in range(T):
        S = torch.exp(gt[:, t])[..., None] * S
        pred = torch.einsum("bhd,bhde->bhe", bt[:, t] * kt[:, t], S)
        S = S + torch.einsum("bhd,bhe->bhde", kt[:, t], wt[:, t] * vt[:, t] - pred)
        outs.append(scale * torch.einsum("bhd,bhde->bhe", qt[:, t], S))
    out = torch.stack(outs, 1) if T else torch.zeros((B, 0, H, Dv), dtype=torch.float64)
    loss = (out * torch.tensor(np.asarray(do, dtype=np.float64))).sum()
    if dh_final is not None:
        loss = loss + (S * torch.tensor(np.asarray(dh_final, dtype=np.float64))).sum()
    loss.backward()
    return tuple(x.grad.numpy() for x in xs) + (S0.grad.numpy(),)


# ----------------------------------------------------------------------------
# Chunk layout helpers: gdn2_fwd.py:79-89.
# ----------------------------------------------------------------------------
def to_chunks(t, BT):
    """(B,L,H,D) -> (B,H,N,BT,D), gdn2_fwd.py:79-82."""
    B, L, H, D = t.shape
    return np.moveaxis(t.reshape(B, L // BT, BT, H, D), (1, 3), (2, 1))


def from_chunks(t):
    """(B,H,N,BT,D) -> (B,L,H,D), gdn2_fwd.py:85-89."""
    B, H, N, BT, D = t.shape
    return np.moveaxis(t, (1, 2, 3), (3, 1, 2)).reshape(B, N * BT, H, D)


def _decay(gc, clip):
    diff = gc[..., :, None, :] - gc[..., None, :, :]
    if clip:
        return np.exp(np.clip(diff, -DECAY_CLIP, DECAY_CLIP)), (np.abs(diff) <= DECAY_CLIP)
    return np.exp(diff), np.ones(diff.shape, dtype=bool)


# ----------------------------------------------------------------------------
# Kernel A: gdn2_fwd.py:93-139.
# ----------------------------------------------------------------------------
def _tiled(fn, tensors, n_out, max_elems=1 << 24):
    """Apply ``fn`` to tiles (M,BT,D)-flattened over the leading axes, in slices
    small enough that the (m,BT,BT,D) decay tensor stays under ``max_elems``."""
    lead = tensors[0].shape[:-2]
    flat = [t.reshape((-1,) + t.shape[-2:]) for t in tensors]
    M = flat[0].shape[0]
    BT, D = tensors[0].shape[-2], tensors[0].shape[-1]
    step = max(1, max_elems // (BT * BT * D))
    outs = [[] for _ in range(n_out)]
    for s in range(0, M, step):
        res = fn(*[t[s:s + step] for t in flat])
        for i in range(n_out):
            outs[i].append(res[i])
    return tuple(np.concatenate(o, axis=0).reshape(lead + o[0].shape[1:]) for o in outs)


def chunk_scores(q, k, b, gc, scale, clip=True):
    """Aqk, Akk for chunk tiles (...,BT,D); ``gc`` is the in-chunk cumsum of g.

    Aqk[i,j] = scale * sum_d q_i k_j exp(gc_i - gc_j), j <= i   (gdn2_fwd.py:124-127,131-135)
    Akk[i,j] =         sum_d (b_i k_i) k_j exp(gc_i - gc_j), j < i  (:128-129,134-136)
    The reference evaluates these per BC x BC sub-block pair (:112-113); blocks
    strictly below the diagonal need no mask, so the full-chunk form is equal.
    """
    BT = q.shape[-2]
    idx = np.arange(BT)
    causal = idx[:, None] >= idx[None, :]
    strict = idx[:, None] > idx[None, :]

    def one(q, k, b, gc):
        E, _ = _decay(gc, clip)
        aqk = scale * np.einsum("...id,...ijd,...jd->...ij", q, E, k) * causal
        akk = np.einsum("...id,...ijd,...jd->...ij", b * k, E, k) * strict
        return sanitize(aqk), sanitize(akk)

    return _tiled(one, (q, k, b, gc), 2)


# ----------------------------------------------------------------------------
# Kernel B: gdn2_fwd.py:174-243.
# ----------------------------------------------------------------------------
def _micro_forward_substitution(T_mb):
    """gdn2_fwd.py:174-189: (I + T)^{-1} of one MB x MB strictly-lower block, row by row."""
    n = T_mb.shape[-1]
    A = np.zeros_like(T_mb)
    for i in range(n):
        onehot = np.zeros(n, dtype=T_mb.dtype)
        onehot[i] = 1.0
        row = onehot - np.einsum("...k,...kj->...j", T_mb[..., i, :], A)
        A[..., i, :] = sanitize(row)
    return A


def _block_solve(T_full):
    """gdn2_fwd.py:192-222: blocked forward substitution with MB micro-blocks."""
    n = T_full.shape[-1]
    nm = n // MB
    blk = {}
    for m in range(nm):
        sm = slice(m * MB, (m + 1) * MB)
        A_mm = sanitize(_micro_forward_substitution(T_full[..., sm, sm]))
        blk[m, m] = A_mm
        for nn in range(m - 1, -1, -1):
            acc = np.zeros_like(A_mm)
            for kk in range(nn, m):
                acc = sanitize(acc + T_full[..., sm, kk * MB:(kk + 1) * MB] @ blk[kk, nn])
            blk[m, nn] = sanitize(-(A_mm @ acc))
    out = np.zeros_like(T_full)
    for (m, nn), a in blk.items():
        out[..., m * MB:(m + 1) * MB, nn * MB:(nn + 1) * MB] = a
    return out


def wy_solve(akk, BC=None):
    """A = (I + Akk)^{-1}, gdn2_fwd.py:225-243.

    With BT == 2*BC the reference solves the two diagonal halves and forms
    A10 = -A11 T10 A00 (:232-238); for any other BT it is the same blocked
    substitution over the whole chunk (exactly equal without saturation).
    """
    BT = akk.shape[-1]
    if BC is None or BT != 2 * BC:
        return _block_solve(akk)
    h = slice(0, BC), slice(BC, 2 * BC)
    A00 = _block_solve(akk[..., h[0], h[0]])
    A11 = _block_solve(akk[..., h[1], h[1]])
    tmp = sanitize(akk[..., h[1], h[0]] @ A00)
    A10 = sanitize(-(A11 @ tmp))
    out = np.zeros_like(akk)
    out[..., h[0], h[0]] = A00
    out[..., h[1], h[0]] = A10
    out[..., h[1], h[1]] = A11
    return out


# ----------------------------------------------------------------------------
# Kernel C: gdn2_fwd.py:264-295.
# ----------------------------------------------------------------------------
def recompute_wy(q, k, v, w, b, gc, A):
    """w_pseudo, u, kg, qg, gc_last for chunk tiles (gdn2_fwd.py:278-289)."""
    w_pseudo = sanitize(A @ (b * k * np.exp(gc)))
    u = sanitize(A @ (w * v))
    gl = gc[..., -1, :]
    kg = sanitize(k * np.exp(gl[..., None, :] - gc))
    qg = sanitize(q * np.exp(gc))
    return w_pseudo, u, kg, qg, sanitize(gl)


# ----------------------------------------------------------------------------
# Kernel D: gdn2_fwd.py:338-397.
# ----------------------------------------------------------------------------
def inter_chunk_combine(aqk, w_pseudo, u, kg, qg, gl, scale, h0):
    """Serial scan over chunks (axis 2 of (B,H,N,...)), gdn2_fwd.py:347-362/378-393.

    Returns o (B,H,N,BT,D), h_final, h_pre_all (B,H,N,D,D), v_new_all (B,H,N,BT,D).
    """
    B, H, N, BT, D = w_pseudo.shape
    h = sanitize(h0)
    o = np.empty(u.shape, dtype=u.dtype)
    h_pre = np.empty((B, H, N) + h.shape[-2:], dtype=u.dtype)
    v_new_all = np.empty(u.shape, dtype=u.dtype)
    for c in range(N):
        h_pre[:, :, c] = h
        v_new = u[:, :, c] - w_pseudo[:, :, c] @ h
        o_c = scale * (qg[:, :, c] @ h) + aqk[:, :, c] @ v_new
        h = sanitize(h * np.exp(gl[:, :, c])[..., None]
                     + np.swapaxes(kg[:, :, c], -1, -2) @ v_new)
        o[:, :, c] = sanitize(o_c)
        v_new_all[:, :, c] = v_new
    return o, h, h_pre, v_new_all


def _prep(q, k, v, w, b, g, BT, dtype):
    B, L, H, D = q.shape
    assert L % BT == 0, f"L={L} must be divisible by BT={BT}."
    qs, ks, vs, ws, bs, gs = (to_chunks(np.asarray(x, dtype=dtype), BT)
                              for x in (q, k, v, w, b, g))
    gc = np.cumsum(gs, axis=-2)
    return qs, ks, vs, ws, bs, gs, gc


def chunked_fwd(q, k, v, w, b, g, scale, h0=None, BT=64, BC=None, clip=True,
                dtype=np.float64, return_residuals=False):
    """Restatement of gdn2_pallas_forward (gdn2_fwd.py:400-424): A -> B -> C -> D.

    ``clip=False`` drops the +-20 decay clip, giving the exact chunked math.
    """
    B, L, H, D = q.shape
    qs, ks, vs, ws, bs, gs, gc = _prep(q, k, v, w, b, g, BT, dtype)
    if h0 is None:
        h0 = np.zeros((B, H, D, v.shape[-1]), dtype=dtype)
    h0 = np.asarray(h0, dtype=dtype)
    aqk, akk = chunk_scores(qs, ks, bs, gc, scale, clip=clip)
    A = wy_solve(akk, BC)
    w_pseudo, u, kg, qg, gl = recompute_wy(qs, ks, vs, ws, bs, gc, A)
    o, h_final, h_pre, v_new = inter_chunk_combine(aqk, w_pseudo, u, kg, qg, gl, scale, h0)
    out = from_chunks(o)
    if not return_residuals:
        return out, h_final
    res = dict(Aqk=aqk, Akk=akk, A=A, w_pseudo=w_pseudo, u=u, kg=kg, qg=qg, gc_last=gl,
               gc=gc, h_pre_all=h_pre, v_new_all=v_new)
    return out, h_final, res


# ----------------------------------------------------------------------------
# Associative scan over chunk affine maps.
# ----------------------------------------------------------------------------
def assoc_scan_fwd(q, k, v, w, b, g, scale, h0=None, BT=64, dtype=np.float64):
    """Chunk recurrence h_{c+1} = M_c h_c + N_c evaluated by a parallel prefix.

    M_c = Diag(exp gc_last) - kg^T w_pseudo, N_c = kg^T u (no clip, no sanitize).
    The inclusive prefix (M, N) o (M', N') = (M M', M N' + N) is built by
    Hillis-Steele doubling, then o_c = scale qg h_c + Aqk (u - w_pseudo h_c).
    """
    B, L, H, D = q.shape
    qs, ks, vs, ws, bs, gs, gc = _prep(q, k, v, w, b, g, BT, dtype)
    N = L // BT
    if h0 is None:
        h0 = np.zeros((B, H, D, v.shape[-1]), dtype=dtype)
    h0 = np.asarray(h0, dtype=dtype)
    aqk, akk = chunk_scores(qs, ks, bs, gc, scale, clip=False)
    eye = np.eye(BT, dtype=dtype)
    A = np.linalg.inv(eye + akk)
    wp = A @ (bs * ks * np.exp(gc))
    u = A @ (ws * vs)
    gl = gc[..., -1, :]
    kg = ks * np.exp(gl[..., None, :] - gc)
    qg = qs * np.exp(gc)
    kgT = np.swapaxes(kg, -1, -2)
    M = np.eye(D, dtype=dtype) * np.exp(gl)[..., :, None] - kgT @ wp   # (B,H,N,D,D)
    Nn = kgT @ u                                                       # (B,H,N,D,Dv)
    # inclusive scan: after it, (M[c], Nn[c]) maps h_0 -> h_{c+1}
    step = 1
    while step < N:
        Mp = M[:, :, :-step]
        Np = Nn[:, :, :-step]
        Mc = M[:, :, step:]
        Nc = Nn[:, :, step:]
        newM = M.copy()
        newN = Nn.copy()
        newM[:, :, step:] = Mc @ Mp
        newN[:, :, step:] = Mc @ Np + Nc
        M, Nn = newM, newN
        step *= 2
    h_after = M @ h0[:, :, None] + Nn                                  # h_{c+1}
    h_pre = np.concatenate([h0[:, :, None], h_after[:, :, :-1]], axis=2)
    v_new = u - wp @ h_pre
    o = scale * (qg @ h_pre) + aqk @ v_new
    return from_chunks(o), h_after[:, :, -1]


# ----------------------------------------------------------------------------
# Backward: gdn2_bwd.py B1-B5 assembled as gdn2_pipeline.py:70-137.
# ----------------------------------------------------------------------------
def _dhu_backward(do, dv_partial, w_pseudo, qg, kg, gl, scale, dht):
    """B1, gdn2_bwd.py:45-80: reverse scan over chunks (axis 2)."""
    N = do.shape[2]
    dh = sanitize(dht)
    dh_all = np.empty(w_pseudo.shape[:3] + dh.shape[-2:], dtype=do.dtype)
    dv_all = np.empty(do.shape, dtype=do.dtype)
    for c in range(N - 1, -1, -1):
        decay = np.exp(gl[:, :, c])[..., None]
        from_out = np.swapaxes(qg[:, :, c], -1, -2) @ (scale * do[:, :, c])
        from_state = dh * decay
        dv_new = sanitize(dv_partial[:, :, c] + kg[:, :, c] @ dh)
        from_vnew = -(np.swapaxes(w_pseudo[:, :, c], -1, -2) @ dv_new)
        dh = sanitize(from_out + from_state + from_vnew)
        dh_all[:, :, c] = dh
        dv_all[:, :, c] = dv_new
    return dh_all, dh, dv_all


def _dav_backward(aqk, v_new, do):
    """B2, gdn2_bwd.py:84-96."""
    BT = aqk.shape[-1]
    idx = np.arange(BT)
    causal = idx[:, None] >= idx[None, :]
    daqk = (do @ np.swapaxes(v_new, -1, -2)) * causal
    dv_new = np.swapaxes(aqk, -1, -2) @ do
    return sanitize(daqk), sanitize(dv_new)


def _wy_dqkg_backward(q, k, b, w, v, gc, A, h_pre, v_new, do, dv, dh_next, scale):
    """B3, gdn2_bwd.py:126-210 (per-chunk tiles, chunk-last-axis layout)."""
    T_ = lambda x: np.swapaxes(x, -1, -2)
    C = q.shape[-2]
    gl = gc[..., -1, :]
    eg = np.exp(gc)
    kbd = b * k * eg
    kg = k * np.exp(gl[..., None, :] - gc)
    qg = q * eg
    wv = w * v
    dqg = (scale * do) @ T_(h_pre)
    dw_pseudo = (-dv) @ T_(h_pre)
    du = dv
    dkg = v_new @ T_(dh_next)
    dA = sanitize(dw_pseudo @ T_(kbd) + du @ T_(wv))
    dkbd = T_(A) @ dw_pseudo
    dwv = T_(A) @ du
    idx = np.arange(C)
    strict = idx[:, None] > idx[None, :]
    tmp = sanitize(dA @ T_(A))
    dakk = -(T_(A) @ tmp) * strict
    dk = dkbd * eg * b
    db = dkbd * eg * k
    dgc = dkbd * kbd
    dx = dkg * kg
    dk = dk + dkg * np.exp(gl[..., None, :] - gc)
    dgc = dgc - dx
    dgl = dx.sum(axis=-2)
    dq = dqg * eg
    dgc = dgc + dqg * qg
    dw = dwv * v
    dv_raw = dwv * w
    dgl = dgl + np.exp(gl) * np.sum(dh_next * h_pre, axis=-1)
    dgc = dgc.copy()
    dgc[..., -1, :] += dgl
    return dict(dq=sanitize(dq), dk=sanitize(dk), db=sanitize(db), dw=sanitize(dw),
                dv_raw=sanitize(dv_raw), dgc=sanitize(dgc), dAkk=sanitize(dakk))


def _intra_backward(daqk, dakk, q, k, b, gc, scale, clip=True, n_sub=2):
    """B4, gdn2_bwd.py:248-339.

    ``n_sub`` sub-blocks of BC = BT / n_sub tokens (the reference's N_SUB = 2,
    BT = N_SUB * BC, gdn2_fwd.py:29-31), visited as the pair loop of
    gdn2_bwd.py:287-328 does -- (si, sj) for si in range(n_sub), sj <= si -- with
    ``_clip_acc`` (gdn2_bwd.py:26-28) on every accumulator after each pair: dq and
    d(bk) of the row block, dk of the column block, then dgc of the row block and
    dgc of the column block (the same rows when si == sj).  The final
    dk + d(bk) b, d(bk) k and the outputs are sanitized (gdn2_bwd.py:330-339).
    ``n_sub=None`` sums every pair first and clips each output once (equal to the
    pair loop wherever no partial sum passes the clip)."""
    BT = q.shape[-2]
    idx = np.arange(BT)
    causal = idx[:, None] >= idx[None, :]
    strict = idx[:, None] > idx[None, :]

    def whole(daqk, dakk, q, k, b, gc):
        E, mask = _decay(gc, clip)
        bk = b * k
        dqk = daqk * causal
        dkk = dakk * strict
        Lq = scale * q
        dq = np.einsum("...ij,...ijd,...jd->...id", dqk, E, k) * scale
        dk = np.einsum("...ij,...ijd,...id->...jd", dqk, E, Lq)
        wq = dqk[..., None] * Lq[..., :, None, :] * k[..., None, :, :] * E * mask
        dbk = np.einsum("...ij,...ijd,...jd->...id", dkk, E, k)
        dk = dk + np.einsum("...ij,...ijd,...id->...jd", dkk, E, bk)
        wk = dkk[..., None] * bk[..., :, None, :] * k[..., None, :, :] * E * mask
        dgc = wq.sum(axis=-2) - wq.sum(axis=-3) + wk.sum(axis=-2) - wk.sum(axis=-3)
        return (sanitize(dq), sanitize(dk + dbk * b), sanitize(dbk * k), sanitize(dgc))

    def pairs(daqk, dakk, q, k, b, gc):
        E, mask = _decay(gc, clip)
        bk = b * k
        BC = BT // n_sub
        sidx = np.arange(BC)
        s_causal = sidx[:, None] >= sidx[None, :]
        s_strict = sidx[:, None] > sidx[None, :]
        dq, dk, dbk, dgc = (np.zeros_like(q) for _ in range(4))
        for si in range(n_sub):
            for sj in range(si + 1):
                I = slice(si * BC, (si + 1) * BC)
                J = slice(sj * BC, (sj + 1) * BC)
                Ep, mp = E[..., I, J, :], mask[..., I, J, :]
                dmq, dmk = daqk[..., I, J], dakk[..., I, J]
                if si == sj:
                    dmq, dmk = dmq * s_causal, dmk * s_strict
                terms = []
                for dm, L, R in ((dmq, scale * q[..., I, :], k[..., J, :]),
                                 (dmk, bk[..., I, :], k[..., J, :])):
                    wgt = dm[..., None] * Ep                      # _dL/_dR/_dgc_pair_sum
                    terms.append((np.einsum("...ijd,...jd->...id", wgt, R),
                                   np.einsum("...ijd,...id->...jd", wgt, L),
                                   (wgt * L[..., :, None, :] * R[..., None, :, :] * mp)))
                (dLq, dRq, wq), (dLk, dRk, wk) = terms
                dq[..., I, :] = sanitize(dq[..., I, :] + dLq * scale)
                dbk[..., I, :] = sanitize(dbk[..., I, :] + dLk)
                dk[..., J, :] = sanitize(dk[..., J, :] + dRq + dRk)
                dgc[..., I, :] = sanitize(dgc[..., I, :] + wq.sum(axis=-2) + wk.sum(axis=-2))
                dgc[..., J, :] = sanitize(dgc[..., J, :] - wq.sum(axis=-3) - wk.sum(axis=-3))
        return (sanitize(dq), sanitize(dk + dbk * b), sanitize(dbk * k), sanitize(dgc))

    if n_sub is not None:
        assert BT % n_sub == 0, f"BT={BT} must split into {n_sub} sub-blocks"
    fn = whole if n_sub is None else pairs
    # _tiled flattens on the shape of its first tensor: pass a (...,BT,D) one first.
    return _tiled(lambda q, k, b, gc, daqk, dakk: fn(daqk, dakk, q, k, b, gc),
                  (q, k, b, gc, daqk, dakk), 4)


def _reverse_cumsum(dgc):
    """B5, gdn2_bwd.py:32-41: dg[i] = sum_{j>=i} dgc[j] within the chunk."""
    return sanitize(np.flip(np.cumsum(np.flip(dgc, axis=-2), axis=-2), axis=-2))


def chunked_bwd(q, k, v, w, b, g, scale, do, dh_final=None, h0=None, BT=64, BC=None,
                clip=True, dtype=np.float64, n_sub=2):
    """Gradients (dq,dk,dv,dw,db,dg,dh0) of chunked_fwd, as gdn2_pipeline.py:70-137.

    Recomputes the forward (gdn2_pipeline.py:77-83), then B2 -> B1 -> B3 -> B4
    -> B5, sums and applies the final clip (:121-135).  Inputs (B,T,H,D),
    ``do`` (B,T,H,D), ``dh_final`` (B,H,D,D) or None (zero).  B1 carries the
    sanitized dh_final (gdn2_bwd.py:53) while B3 receives it raw as the last
    chunk's dh' (gdn2_pipeline.py:52-56,105).  ``n_sub``: B4's sub-blocks per
    chunk (see ``_intra_backward``).
    """
    B, L, H, D = q.shape
    Dv = v.shape[-1]
    if h0 is None:
        h0 = np.zeros((B, H, D, Dv), dtype=dtype)
    if dh_final is None:
        dh_final = np.zeros((B, H, D, Dv), dtype=dtype)
    dh_final = np.asarray(dh_final, dtype=dtype)
    _, _, res = chunked_fwd(q, k, v, w, b, g, scale, h0=h0, BT=BT, BC=BC, clip=clip,
                            dtype=dtype, return_residuals=True)
    qs, ks, vs, ws, bs, gs, gc = _prep(q, k, v, w, b, g, BT, dtype)
    dos = to_chunks(np.asarray(do, dtype=dtype), BT)
    daqk, dv_partial = _dav_backward(res["Aqk"], res["v_new_all"], dos)
    dh_all, dh0, dv_all = _dhu_backward(dos, dv_partial, res["w_pseudo"], res["qg"],
                                        res["kg"], res["gc_last"], scale, dh_final)
    # gdn2_pipeline.py:52-56: dh_next[c] = dh entering chunk c from the right; the
    # last chunk's is dh_final as given (B1 alone sanitizes it, gdn2_bwd.py:53)
    dh_next = np.concatenate([dh_all[:, :, 1:], dh_final[:, :, None]], axis=2)
    b3 = _wy_dqkg_backward(qs, ks, bs, ws, vs, gc, res["A"], res["h_pre_all"],
                           res["v_new_all"], dos, dv_all, dh_next, scale)
    dq4, dk4, db4, dgc4 = _intra_backward(daqk, b3["dAkk"], qs, ks, bs, gc, scale, clip=clip,
                                          n_sub=n_sub)
    dg = _reverse_cumsum(b3["dgc"] + dgc4)
    grads = (b3["dq"] + dq4, b3["dk"] + dk4, b3["dv_raw"], b3["dw"], b3["db"] + db4, dg)
    dq, dk, dv, dw, db, dg = (sanitize(from_chunks(x)) for x in grads)
    return dq, dk, dv, dw, db, dg, sanitize(dh0)
