"""The reference's backward kernels one at a time: drop-in for gdn2_bwd.py's five
module functions.

    dg = reverse_cumsum_bwd(dgc, chunk_size)                              # B5
    dh_all, dh0, dv_all = gdn2_dhu_backward(do, dv_partial, w_pseudo, qg, kg,
                                            gc_last, scale, dht=None)     # B1
    dAqk, dv_new = dav_backward_pallas(Aqk, v_new, do)                    # B2
    grads = wy_dqkg_backward_pallas(q, k, b, w, v, gc, A, Akk, h_pre_all,
                                    v_new_all, do, dv, dh_next_all, scale)  # B3
    dq, dk, db, dgc = intra_backward_pallas(dAqk, dAkk, q, k, b, g, scale)  # B4

Same argument order, shapes and meaning as the reference (gdn2_bwd.py:32-375);
float32 in and out, chunk 64, D in {64, 128, 256} (the reference's B4 asserts
128).  Each runs the gfx950 kernels of the fused backward (gdn2_pipeline's
gdn2_bwd entry point) in a mode that forms only the stage's products, plus
layout copies between the reference's (B,H,N,BT,.) tiles and the token rows
and transposed tiles those kernels read.  There is no CPU fallback: without
libgdn2_hip.so every call raises.
"""
from __future__ import annotations

import torch

from . import _lib
from .gdn2_fwd import (BC, CLIP, N_SUB, GDN2Error, GDN2ShapeError, _apply_clip, _raise,
                       _stage_chunk, _STAGE_BT)

__all__ = ["reverse_cumsum_bwd", "gdn2_dhu_backward", "dav_backward_pallas",
           "wy_dqkg_backward_pallas", "intra_backward_pallas", "BC", "N_SUB", "CLIP"]


def _check(x, name, shape, device):
    if not isinstance(x, torch.Tensor):
        raise TypeError(f"gdn2: {name} must be a torch tensor on the ROCm device")
    if tuple(x.shape) != tuple(shape):
        raise GDN2ShapeError(f"gdn2: {name} must have shape {tuple(shape)}; got "
                             f"{tuple(x.shape)}")
    if x.device != device:
        raise GDN2Error(f"gdn2: {name} must live on {device}")
    return x


def _f32(x, name, shape, device):
    return _check(x, name, shape, device).to(torch.float32).contiguous()


def _tiles_of(x, name):
    """(B,H,N,BT,D) and device of a chunk tensor, checked for chunk 64."""
    if not isinstance(x, torch.Tensor) or x.dim() != 5:
        raise GDN2ShapeError(f"gdn2: {name} must be a (B,H,N,BT,D) tensor")
    B, H, N, BT, D = x.shape
    if BT != _stage_chunk(D):
        raise GDN2ShapeError(f"gdn2: chunk tiles of {BT} tokens; the stage functions take "
                             f"{_STAGE_BT}")
    return B, H, N, BT, D, x.device


def _workspace(stage, B, N, H, D, BT, dev):
    """The stage's workspace, once every shape is checked: here the tensors must
    be on the ROCm device."""
    if dev.type != "cuda":
        raise GDN2Error("gdn2: the stage tensors must live on the ROCm device (torch 'cuda')")
    _apply_clip(dev)
    nbytes = _lib.lib().gdn2_bwd_stage_workspace_bytes(stage, B, N, H, D, BT)
    return torch.empty(max(nbytes, 1), dtype=torch.uint8, device=dev), nbytes


def _stream(dev):
    return torch.cuda.current_stream(dev).cuda_stream


def _empty(shape, dev):
    return torch.empty(shape, dtype=torch.float32, device=dev)


def reverse_cumsum_bwd(dgc, chunk_size):
    """B5, gdn2_bwd.py:32-41: dg[i] = sum_{j >= i} dgc[j] over the chunk axis
    (dgc's second-to-last, of length chunk_size), sanitized; float32."""
    if not isinstance(dgc, torch.Tensor):
        raise TypeError("gdn2: dgc must be a torch tensor on the ROCm device")
    C = int(chunk_size)
    if dgc.dim() < 2 or dgc.shape[-2] != C:
        raise GDN2ShapeError(f"gdn2: dgc must end in ({C}, D); got {tuple(dgc.shape)}")
    if dgc.device.type != "cuda":
        raise GDN2Error("gdn2: dgc must live on the ROCm device (torch 'cuda')")
    _apply_clip(dgc.device)
    x = dgc.to(torch.float32).contiguous()
    out = torch.empty_like(x)
    D = x.shape[-1]
    tiles = x.numel() // (C * D) if C * D else 0
    rc = _lib.lib().gdn2_bwd_reverse_cumsum(_stream(x.device), tiles, C, D, x.data_ptr(),
                                            out.data_ptr())
    if rc:
        _raise(rc, "gdn2_bwd_reverse_cumsum")
    return out


def gdn2_dhu_backward(do, dv_partial, w_pseudo, qg, kg, gc_last, scale, dht=None):
    """B1, gdn2_bwd.py:45-80: the reverse scan over chunks.  With dh the
    gradient of the state (dh = sanitize(dht) after the last chunk), per chunk
    c from the last: dv_new = sanitize(dv_partial + kg dh), dh <-
    sanitize(scale qg^T do + e^{gc_last} dh - w_pseudo^T dv_new).  Returns
    dh_all (B,H,N,D,D), the gradient of the state entering each chunk, dh0
    (= dh_all[:, :, 0]) and dv_all (B,H,N,BT,D).  All (B,H,N,BT,D) inputs,
    gc_last (B,H,N,D), dht (B,H,D,D) or None."""
    B, H, N, BT, D, dev = _tiles_of(qg, "qg")
    tile = (B, H, N, BT, D)
    xs = [_f32(x, n, tile, dev) for x, n in ((do, "do"), (dv_partial, "dv_partial"),
                                             (w_pseudo, "w_pseudo"), (qg, "qg"), (kg, "kg"))]
    gl = _f32(gc_last, "gc_last", (B, H, N, D), dev)
    dh_t = None if dht is None else _f32(dht, "dht", (B, H, D, D), dev)
    ws, nbytes = _workspace(_lib.STAGE_DHU, B, N, H, D, BT, dev)
    dh_all, dv_all = _empty((B, H, N, D, D), dev), _empty(tile, dev)
    dh0 = _empty((B, H, D, D), dev)
    rc = _lib.lib().gdn2_bwd_dhu(_stream(dev), B, N, H, D, BT, *(x.data_ptr() for x in xs),
                                 gl.data_ptr(), float(scale),
                                 None if dh_t is None else dh_t.data_ptr(), dh_all.data_ptr(),
                                 dh0.data_ptr(), dv_all.data_ptr(), ws.data_ptr(), nbytes)
    if rc:
        _raise(rc, "gdn2_bwd_dhu")
    return dh_all, dh0, dv_all


def dav_backward_pallas(Aqk, v_new, do):
    """B2, gdn2_bwd.py:84-122: dAqk = sanitize((do v_new^T) . causal) and
    dv_new = sanitize(Aqk^T do) per chunk; Aqk (B,H,N,BT,BT) is read as causal
    (kernel A's output: entries above the diagonal are taken as zero), v_new
    and do (B,H,N,BT,D)."""
    B, H, N, BT, D, dev = _tiles_of(v_new, "v_new")
    aqk = _f32(Aqk, "Aqk", (B, H, N, BT, BT), dev)
    vn, d_o = (_f32(x, n, (B, H, N, BT, D), dev) for x, n in ((v_new, "v_new"), (do, "do")))
    daqk, dvn = _empty(aqk.shape, dev), _empty(vn.shape, dev)
    ws, nbytes = _workspace(_lib.STAGE_DAV, B, N, H, D, BT, dev)
    rc = _lib.lib().gdn2_bwd_dav(_stream(dev), B, N, H, D, BT, aqk.data_ptr(), vn.data_ptr(),
                                 d_o.data_ptr(), daqk.data_ptr(), dvn.data_ptr(),
                                 ws.data_ptr(), nbytes)
    if rc:
        _raise(rc, "gdn2_bwd_dav")
    return daqk, dvn


def wy_dqkg_backward_pallas(q, k, b, w, v, gc, A, Akk, h_pre_all, v_new_all, do, dv,
                            dh_next_all, scale):
    """B3, gdn2_bwd.py:126-244: the gradients through the WY factors, kg and
    qg, per chunk.  q, k, b, w, v, gc (the in-chunk cumsum of g), v_new_all, do,
    dv (B,H,N,BT,D); A (B,H,N,BT,BT); h_pre_all and dh_next_all (B,H,N,D,D).
    Akk is only shape-checked, as in the reference (gdn2_bwd.py:137).  Returns
    dict(dq, dk, db, dw, dv_raw, dgc, dAkk), float32 and sanitized; dgc carries
    the g_last terms on each chunk's last token (gdn2_bwd.py:196-201)."""
    B, H, N, BT, D, dev = _tiles_of(q, "q")
    tile, sq, st = (B, H, N, BT, D), (B, H, N, BT, BT), (B, H, N, D, D)
    xs = [_f32(x, n, tile, dev) for x, n in ((q, "q"), (k, "k"), (b, "b"), (w, "w"),
                                             (v, "v"), (gc, "gc"))]
    a = _f32(A, "A", sq, dev)
    _check(Akk, "Akk", sq, dev)
    hp = _f32(h_pre_all, "h_pre_all", st, dev)
    vn, d_o, d_v = (_f32(x, n, tile, dev) for x, n in
                    ((v_new_all, "v_new_all"), (do, "do"), (dv, "dv")))
    dhn = _f32(dh_next_all, "dh_next_all", st, dev)
    names = ("dq", "dk", "db", "dw", "dv_raw", "dgc")
    outs = {n: _empty(tile, dev) for n in names}
    outs["dAkk"] = _empty(sq, dev)
    ws, nbytes = _workspace(_lib.STAGE_WY, B, N, H, D, BT, dev)
    rc = _lib.lib().gdn2_bwd_wy_dqkg(
        _stream(dev), B, N, H, D, BT, *(x.data_ptr() for x in xs), a.data_ptr(),
        hp.data_ptr(), vn.data_ptr(), d_o.data_ptr(), d_v.data_ptr(), dhn.data_ptr(),
        float(scale), *(outs[n].data_ptr() for n in names + ("dAkk",)), ws.data_ptr(), nbytes)
    if rc:
        _raise(rc, "gdn2_bwd_wy_dqkg")
    return outs


def intra_backward_pallas(dAqk, dAkk, q, k, b, g, scale):
    """B4, gdn2_bwd.py:267-375: the gradients through the score blocks Aqk
    (causal) and Akk (strictly lower).  q, k, b, g (B,L,H,D) as the reference
    takes them (g raw: the in-chunk cumsum is formed here); dAqk, dAkk
    (B,H,N,BT,BT).  Returns dq, dk, db, dgc (B,H,N,BT,D), float32, with the
    reference's clipping after each sub-block pair (gdn2_bwd.py:287-328)."""
    if not isinstance(q, torch.Tensor) or q.dim() != 4:
        raise GDN2ShapeError("gdn2: q must be a (B,L,H,D) tensor")
    B, L, H, D = q.shape
    BT = _stage_chunk(D)
    if L % BT != 0:
        raise GDN2ShapeError(f"gdn2: L={L} must be divisible by BT={BT} (gdn2_bwd.py:350)")
    dev = q.device
    N = L // BT
    xs = [_f32(x, n, (B, L, H, D), dev) for x, n in ((q, "q"), (k, "k"), (b, "b"), (g, "g"))]
    dq_, dk_ = (_f32(x, n, (B, H, N, BT, BT), dev) for x, n in ((dAqk, "dAqk"),
                                                                (dAkk, "dAkk")))
    outs = [_empty((B, H, N, BT, D), dev) for _ in range(4)]
    ws, nbytes = _workspace(_lib.STAGE_INTRA, B, N, H, D, BT, dev)
    rc = _lib.lib().gdn2_bwd_intra(_stream(dev), B, L, H, D, BT, dq_.data_ptr(), dk_.data_ptr(),
                                   *(x.data_ptr() for x in xs), float(scale),
                                   *(o.data_ptr() for o in outs), ws.data_ptr(), nbytes)
    if rc:
        _raise(rc, "gdn2_bwd_intra")
    return tuple(outs)
