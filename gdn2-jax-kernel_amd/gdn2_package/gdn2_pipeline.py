"""Trainable GDN-2: drop-in for gdn2_pipeline.py's gdn2_pallas_forward_trainable.

    out, h_final = gdn2_pallas_forward_trainable(q, k, v, w, b, g, scale, h0=None)

A ``torch.autograd.Function`` plays the role of the reference's
``jax.custom_vjp`` (gdn2_pipeline.py:59-140): ``scale`` is non-differentiable,
the cotangents are (d out, d h_final), and the gradients of
(q, k, v, w, b, g, h0) come back in each input's dtype (:129-135).

Arithmetic.  The trainable path computes in float32 whatever the input dtype,
as the reference upcasts every input before any arithmetic
(gdn2_fwd.py:100-103,266-272; gdn2_bwd.py:130-142), so the residuals the
backward contracts against the state cotangent are float32.  bfloat16 inputs
are read as they are by the float32 kernels (GDN2_BF16_F32), which write the
gradients of q, k, v, w, b in bfloat16; inputs of mixed dtypes are widened to
float32 first.  Gradients come back in each input's dtype.

Residuals.  By default the forward keeps its per-chunk workspace (WY factors,
chunk states, v_new) for the backward.  ``recompute=True`` keeps only the
inputs, as the reference does (:64-67), and re-runs the forward kernels in the
backward (:77-83) -- less memory, one more forward.
"""
from __future__ import annotations

import torch

from . import _lib
from .gdn2_fwd import GDN2ShapeError, _Prepared, _apply_clip, _raise, _run_forward

# Chunk size of the trainable path (the backward kernels are written for 64).
TRAIN_CHUNK = 64


def _run_backward(p: _Prepared, ws: torch.Tensor, dout, dh_final):
    _apply_clip(p.device)   # CLIP as it is when the backward runs
    L = _lib.lib()
    fbytes = ws.numel()   # the residual-keeping forward's workspace (GDN2_FWD_SAVE_A)
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
                      else chunk_size, compute_dtype=torch.float32)
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


class _GDN2VarlenCore(torch.autograd.Function):
    """Variable-length batch on whole chunks: the inputs are (1, total*BT, H, D)
    with sequence s on chunks [cu_chunks[s], cu_chunks[s+1]); forward with
    residuals (gdn2_fwd_varlen, GDN2_FWD_SAVE_A), backward gdn2_bwd_varlen."""

    @staticmethod
    def forward(ctx, q, k, v, w, b, g, h0, scale, cu_chunks):
        p = _Prepared(q, k, v, w, b, g, scale, None, TRAIN_CHUNK, compute_dtype=torch.float32)
        S = cu_chunks.numel() - 1
        total = p.T // p.BT
        dev = p.device
        cu_d = cu_chunks.to(device=dev, dtype=torch.int32)
        cs_d = (torch.arange(total + 1, device=dev, dtype=torch.int32) * p.BT)
        h0c = None if h0 is None else h0.to(device=dev, dtype=torch.float32).contiguous()
        L = _lib.lib()
        nbytes = L.gdn2_fwd_varlen_workspace_bytes(total, p.H, p.D, p.BT, p.code)
        ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=dev)
        out = torch.empty((1, p.T, p.H, p.D), dtype=torch.float32, device=dev)
        h_final = torch.empty((S, p.H, p.D, p.D), dtype=torch.float32, device=dev)
        rc = L.gdn2_fwd_varlen(p.stream(), S, cu_d.data_ptr(), cs_d.data_ptr(), total, p.T,
                               p.H, p.D, p.BT, *p.args[5:], *(p.ptr(x) for x in (
                                   p.q, p.k, p.v, p.w, p.b, p.g)), p.ptr(h0c), p.scale,
                               out.data_ptr(), h_final.data_ptr(), ws.data_ptr(), nbytes,
                               _lib.FWD_SAVE_A)
        if rc:
            _raise(rc, "gdn2_fwd_varlen")
        ctx.prep, ctx.ws, ctx.fbytes, ctx.cu_d, ctx.S = p, ws, nbytes, cu_d, S
        ctx.h0_given = h0 is not None
        ctx.h0_dtype = h0.dtype if h0 is not None else torch.float32
        return out, h_final

    @staticmethod
    def backward(ctx, dout, dh_final):
        p, S = ctx.prep, ctx.S
        total = p.T // p.BT
        _apply_clip(p.device)
        L = _lib.lib()
        bbytes = L.gdn2_bwd_varlen_workspace_bytes(total, p.H, p.D, p.BT, p.code)
        bws = torch.empty(max(bbytes, 1), dtype=torch.uint8, device=p.device)
        if dout is None:
            dout = torch.zeros((1, p.T, p.H, p.D), dtype=torch.float32, device=p.device)
        dout = dout.to(device=p.device, dtype=torch.float32).contiguous()
        if dh_final is not None:
            dh_final = dh_final.to(device=p.device, dtype=torch.float32).contiguous()
        shape = (1, p.T, p.H, p.D)
        dq, dk, dv, dw, db = (torch.empty(shape, dtype=p.in_dt, device=p.device)
                              for _ in range(5))
        dg = torch.empty(shape, dtype=p.g_dt, device=p.device)
        dh0 = torch.empty((S, p.H, p.D, p.D), dtype=torch.float32, device=p.device)
        rc = L.gdn2_bwd_varlen(p.stream(), S, ctx.cu_d.data_ptr(), total, p.H, p.D, p.BT,
                               *p.args[5:], p.ptr(p.q), p.ptr(p.k), p.ptr(p.v), p.ptr(p.w),
                               p.ptr(p.b), p.ptr(p.g), None, p.scale, dout.data_ptr(),
                               p.ptr(dh_final), dq.data_ptr(), dk.data_ptr(), dv.data_ptr(),
                               dw.data_ptr(), db.data_ptr(), dg.data_ptr(), dh0.data_ptr(),
                               ctx.ws.data_ptr(), ctx.fbytes, bws.data_ptr(), bbytes)
        if rc:
            _raise(rc, "gdn2_bwd_varlen")
        ctx.ws = None
        grads = [x.to(dt) for x, dt in zip((dq, dk, dv, dw, db, dg), p.in_dtypes)]
        dh0 = dh0.to(ctx.h0_dtype) if ctx.h0_given else None
        return (*grads, dh0, None, None)


def gdn2_pallas_forward_varlen_trainable(q, k, v, w, b, g, scale, cu_seqlens, h0=None):
    """Trainable forward over a variable-length batch packed along T (inputs
    (1, T, H, D), ``cu_seqlens`` as in ``gdn2_pallas_forward_varlen``; h0
    (num_seqs, H, D, D) or None).  Returns out (1, T, H, D) and h_final
    (num_seqs, H, D, D), differentiable in q..g and h0.  Each sequence is
    placed on whole 64-token chunks with zero tokens after it (neutral: they add
    nothing to the state and do not decay it), so its results and gradients are
    those of the sequence alone.  No reference counterpart (the reference needs
    equal lengths with T % BT == 0, gdn2_fwd.py:145-146)."""
    if q.dim() != 4 or q.shape[0] != 1:
        raise GDN2ShapeError(f"gdn2 varlen: expected packed (1,T,H,D) inputs, got {tuple(q.shape)}")
    _, T, H, D = q.shape
    cu_host = torch.as_tensor(cu_seqlens).detach().to("cpu", torch.int64).reshape(-1)
    if cu_host.numel() < 2 or int(cu_host[0]) != 0 or int(cu_host[-1]) != T or \
            bool((cu_host[1:] < cu_host[:-1]).any()):
        raise GDN2ShapeError("gdn2 varlen: cu_seqlens must start at 0, end at T and not decrease")
    S = cu_host.numel() - 1
    if h0 is not None and tuple(h0.shape) != (S, H, D, D):
        raise GDN2ShapeError(f"gdn2 varlen: h0 must be (num_seqs,H,D,D); got {tuple(h0.shape)}")
    BT = TRAIN_CHUNK
    lens = cu_host[1:] - cu_host[:-1]
    nch = (lens + BT - 1) // BT
    cu_chunks = torch.zeros(S + 1, dtype=torch.int64)
    cu_chunks[1:] = torch.cumsum(nch, 0)
    total = int(cu_chunks[-1])
    # padded row of every packed token row
    seq_of = torch.repeat_interleave(torch.arange(S), lens)
    rows = torch.arange(T) - cu_host[seq_of] + BT * cu_chunks[seq_of]
    idx = rows.to(q.device)
    pad = lambda x: torch.zeros((1, total * BT, H, D), dtype=x.dtype,
                                device=x.device).index_copy(1, idx, x)
    out_p, h_final = _GDN2VarlenCore.apply(*(pad(x) for x in (q, k, v, w, b, g)), h0, scale,
                                           cu_chunks)
    return out_p.index_select(1, idx), h_final