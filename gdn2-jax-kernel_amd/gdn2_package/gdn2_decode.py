"""Single-token recurrent decode step on the GDN-2 state (serving).

    out, state = gdn2_decode_step(q, k, v, w, b, g, scale, state=None)

The reference has only the chunked forward; one token is its T = 1 case
(gdn2_fwd.py:400-424) on the float32 state layout of h0 / h_final,
(B,H,D,D) indexed [b][h][dk][dv] (gdn2_fwd.py:342).  Running
``gdn2_pallas_forward`` over a prefix and then ``gdn2_decode_step`` token by
token from its ``h_final`` gives the forward's outputs for the whole sequence.

q,k,v,w,b,g: one token, (B,1,H,D) or (B,H,D), float32 or bfloat16 (g float32,
or bfloat16 with bfloat16 inputs).  Returns ``out`` float32 with the input's
rank and the new state (B,H,D,D) float32; ``inplace=True`` updates ``state``
itself (it must then be a contiguous float32 tensor).
"""
from __future__ import annotations

import torch

from . import _lib
from .gdn2_fwd import GDN2Error, GDN2ShapeError, _apply_clip, _dtype_code, _raise, _SUPPORTED_IN


def gdn2_decode_step(q, k, v, w, b, g, scale, state=None, inplace=False):
    xs = (q, k, v, w, b, g)
    for x in xs:
        if not isinstance(x, torch.Tensor):
            raise TypeError("gdn2_decode_step: q,k,v,w,b,g must be torch tensors")
    if q.dim() == 4:
        if q.shape[1] != 1:
            raise GDN2ShapeError(f"gdn2_decode_step: one token expected, got {tuple(q.shape)}")
        B, _, H, D = q.shape
    elif q.dim() == 3:
        B, H, D = q.shape
    else:
        raise GDN2ShapeError(f"gdn2_decode_step: expected (B,1,H,D) or (B,H,D), got {tuple(q.shape)}")
    for x in xs[1:]:
        if x.shape != q.shape:
            raise GDN2ShapeError(f"gdn2_decode_step: inputs must share shape {tuple(q.shape)}")
    dev = q.device
    if dev.type != "cuda" or any(x.device != dev for x in xs):
        raise GDN2Error("gdn2_decode_step: inputs must live on one ROCm device; no CPU path")
    _apply_clip(dev)
    in_dt = q.dtype if q.dtype in _SUPPORTED_IN else torch.float32
    if any(x.dtype != in_dt for x in (k, v, w, b)):
        in_dt = torch.float32
    g_dt = torch.bfloat16 if (in_dt == torch.bfloat16 and g.dtype == torch.bfloat16) \
        else torch.float32
    tq, tk, tv, tw, tb = (x.to(in_dt).contiguous() for x in xs[:5])
    tg = g.to(g_dt).contiguous()
    if state is not None and tuple(state.shape) != (B, H, D, D):
        raise GDN2ShapeError(f"gdn2_decode_step: state must be (B,H,D,D); got {tuple(state.shape)}")
    if inplace:
        if state is None or state.dtype != torch.float32 or not state.is_contiguous():
            raise GDN2Error("gdn2_decode_step: inplace needs a contiguous float32 state")
        h_in, h_out = state, state
    else:
        h_in = None if state is None else state.to(device=dev, dtype=torch.float32).contiguous()
        h_out = torch.empty((B, H, D, D), dtype=torch.float32, device=dev)
    out = torch.empty((B, H, D), dtype=torch.float32, device=dev)
    L = _lib.lib()
    rc = L.gdn2_decode(torch.cuda.current_stream(dev).cuda_stream, B, H, D, _dtype_code(in_dt),
                       _dtype_code(g_dt), tq.data_ptr(), tk.data_ptr(), tv.data_ptr(),
                       tw.data_ptr(), tb.data_ptr(), tg.data_ptr(), float(scale),
                       None if h_in is None else h_in.data_ptr(), h_out.data_ptr(),
                       out.data_ptr())
    if rc:
        _raise(rc, f"gdn2_decode (B,H,D)=({B},{H},{D})")
    return (out.view(B, 1, H, D) if q.dim() == 4 else out), h_out
