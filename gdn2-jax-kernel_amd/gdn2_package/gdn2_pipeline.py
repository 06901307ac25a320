"""Trainable GDN-2: drop-in for gdn2_pipeline.py's gdn2_pallas_forward_trainable.

    out, h_final = gdn2_pallas_forward_trainable(q, k, v, w, b, g, scale, h0=None)

A ``torch.autograd.Function`` plays the role of the reference's
``jax.custom_vjp`` (gdn2_pipeline.py:59-140): ``scale`` is non-differentiable,
the cotangents are (d out, d h_final), and the gradients of
(q, k, v, w, b, g, h0) come back in each input's dtype (:129-135).

Residuals.  By default the forward keeps its per-chunk workspace (WY factors,
chunk states, v_new) for the backward.  ``recompute=True`` keeps only the
inputs, as the reference does (:64-67), and re-runs the forward kernels in the
backward (:77-83) -- less memory, one more forward.
"""
from __future__ import annotations

import torch

from . import _lib
from .gdn2_fwd import _Prepared, _raise, _run_forward

# Chunk size of the trainable path (the backward kernels are written for 64).
TRAIN_CHUNK = 64


def _run_backward(p: _Prepared, ws: torch.Tensor, dout, dh_final):
    L = _lib.lib()
    fbytes = L.gdn2_fwd_workspace_bytes(*p.args[:6])
    bbytes = L.gdn2_bwd_workspace_bytes(*p.args[:6])
    bws = torch.empty(max(bbytes, 1), dtype=torch.uint8, device=p.device)
    dout = dout.to(device=p.device, dtype=torch.float32).contiguous()
    if dh_final is not None:
        dh_final = dh_final.to(device=p.device, dtype=torch.float32).contiguous()
    shape = (p.B, p.T, p.H, p.D)
    dq, dk, dv, dw, db = (torch.empty(shape, dtype=p.in_dt, device=p.device) for _ in range(5))
    dg = torch.empty(shape, dtype=p.g_dt, device=p.device)
    dh0 = torch.empty((p.B, p.H, p.D, p.D), dtype=torch.float32, device=p.device)
    rc = L.gdn2_bwd(p.stream(), *p.args, p.ptr(p.q), p.ptr(p.k), p.ptr(p.v), p.ptr(p.w),
                    p.ptr(p.b), p.ptr(p.g), p.ptr(p.h0), p.scale, dout.data_ptr(),
                    p.ptr(dh_final), dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), dw.data_ptr(),
                    db.data_ptr(), dg.data_ptr(), dh0.data_ptr(), ws.data_ptr(), fbytes,
                    bws.data_ptr(), bbytes)
    if rc:
        _raise(rc, "gdn2_bwd")
    return dq, dk, dv, dw, db, dg, dh0


class _GDN2Core(torch.autograd.Function):
    """custom_vjp equivalent of _gdn2_core (gdn2_pipeline.py:59-140)."""

    @staticmethod
    def forward(ctx, q, k, v, w, b, g, h0, scale, chunk_size, recompute):
        # the backward kernels tile 64-token chunks
        p = _Prepared(q, k, v, w, b, g, scale, h0, TRAIN_CHUNK if chunk_size is None
                      else chunk_size)
        out, h_final, ws, _ = _run_forward(p, flags=_lib.FWD_SAVE_A)
        ctx.prep = p
        ctx.ws = None if recompute else ws
        ctx.h0_given = h0 is not None
        ctx.h0_dtype = h0.dtype if h0 is not None else torch.float32
        return out, h_final

    @staticmethod
    def backward(ctx, dout, dh_final):
        p = ctx.prep
        ws = ctx.ws
        if ws is None:
            _, _, ws, _ = _run_forward(p, flags=_lib.FWD_SAVE_A)
        if dout is None:
            dout = torch.zeros((p.B, p.T, p.H, p.D), dtype=torch.float32, device=p.device)
        dq, dk, dv, dw, db, dg, dh0 = _run_backward(p, ws, dout, dh_final)
        ctx.ws = None
        dts = p.in_dtypes
        grads = [x.to(dt) for x, dt in zip((dq, dk, dv, dw, db, dg), dts)]
        dh0 = dh0.to(ctx.h0_dtype) if ctx.h0_given else None
        return (*grads, dh0, None, None, None)


def gdn2_pallas_forward_trainable(q, k, v, w, b, g, scale, h0=None, chunk_size=None,
                                  recompute=False):
    """gdn2_pipeline.py:143-159.  h0 defaults to a zero float32 state.

    T % chunk != 0 (the reference asserts, gdn2_fwd.py:146): the inputs are
    padded with zero tokens up to whole chunks.  A zero token is neutral (k = 0
    adds nothing to the state, g = 0 does not decay it, q = 0 reads nothing), so
    out[:, :T], h_final and every gradient of the real tokens are unchanged;
    the pad costs one copy of the inputs."""
    B, T, H, D = q.shape
    if h0 is None:
        h0 = torch.zeros((B, H, D, D), dtype=torch.float32, device=q.device)
    bt = TRAIN_CHUNK if chunk_size is None else int(chunk_size)
    pad = (-T) % bt if bt > 0 else 0
    if pad:
        xs = [torch.nn.functional.pad(x, (0, 0, 0, 0, 0, pad)) for x in (q, k, v, w, b, g)]
        out, h_final = _GDN2Core.apply(*xs, h0, scale, chunk_size, recompute)
        return out[:, :T], h_final
    return _GDN2Core.apply(q, k, v, w, b, g, h0, scale, chunk_size, recompute)
