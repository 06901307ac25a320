"""GDN-2 forward on MI355X: drop-in for the reference's gdn2_fwd.py API.

    out, h_final = gdn2_pallas_forward(q, k, v, w, b, g, scale, h0=None)

Same argument order and meaning as gdn2_fwd.py:400 (q,k,v,w,b,g of shape
(B,T,H,D); ``scale`` a Python float; optional float32 ``h0`` (B,H,D,D)).
``out`` (B,T,H,D) and ``h_final`` (B,H,D,D) are float32 (gdn2_fwd.py:163-165,342).
Tensors are torch tensors on the ROCm device; the compute runs in the gfx950
HIP library libgdn2_hip.so (kernels fwd_prep / fwd_state / fwd_out).  There
is no CPU fallback: without the library every call raises.

Chunk size.  ``BT`` below plays the role of gdn2_fwd.py:29 but is read at call
time, so overriding it also reaches the backward (the reference binds it by
value at import, gdn2_bwd.py:23).  ``None`` picks 128 for bfloat16 inputs at
D = 64 and 64 otherwise (see ``chunk_size_for``); 64 and 128 are accepted (128
only with bfloat16 inputs at D <= 128), and the reference's default 256 runs at
the automatic choice.  Results do not depend on the chunk size beyond rounding.

Clip bound.  ``CLIP`` (gdn2_fwd.py:33) is read at call time too: overriding it
(the reference README's ``fwd.CLIP = 1e3``, README.md:87-92) sets the saturation
bound of every stage sanitize in the library (``gdn2_set_clip``) before the
next call on each device.
"""
from __future__ import annotations

import math
import os

import torch

from . import _lib

# Reference constants, gdn2_fwd.py:29-33.  BC/N_SUB/MB describe the reference's
# own sub-blocking and are kept for API compatibility; this implementation
# always works on 16-token sub-blocks.
BT = None
BC = 64
N_SUB = 2
MB = 16
CLIP = 1e4

_SUPPORTED_IN = (torch.float32, torch.bfloat16)

# Stage diagnostics, switched on by the environment at import as in the
# reference (gdn2_fwd.py:36-38): with GDN2_FWD_DIAG=1 the forward keeps the
# per-kernel outputs and reports non-finite or suspiciously large values.
_GDN2_FWD_DIAG = os.environ.get("GDN2_FWD_DIAG", "0") == "1"
_LARGE_THRESHOLD = 1e6


def _stage_diag(tag: str, x: torch.Tensor) -> torch.Tensor:
    """gdn2_fwd.py:47-76: report non-finite entries (count, largest finite
    magnitude) or, when all are finite, a largest magnitude above 1e6.
    Returns x unchanged."""
    if not _GDN2_FWD_DIAG:
        return x
    finite = torch.isfinite(x)
    n_bad = int((~finite).sum().item())
    max_abs = float(torch.where(finite, x, torch.zeros_like(x)).abs().max().item()) \
        if x.numel() else 0.0
    if n_bad:
        print(f"[GDN2-FWD-DIAG] non-finite at output {tag}: n_nonfinite={n_bad}  "
              f"max_abs(finite part)={max_abs:.3e}", flush=True)
    elif max_abs > _LARGE_THRESHOLD:
        print(f"[GDN2-FWD-DIAG] suspiciously large value at output {tag} (still finite, "
              f"possibly a precursor): max_abs={max_abs:.3e}", flush=True)
    return x


class GDN2Error(RuntimeError):
    """A libgdn2_hip call failed."""


class GDN2ShapeError(GDN2Error, AssertionError, ValueError):
    """Invalid shape (the reference raises AssertionError at trace time,
    gdn2_fwd.py:145-146)."""


def _raise(code: int, what: str):
    msg = f"{what}: {_lib.strerror(code)} (code {code})"
    if code in (_lib.ERR_HEAD_DIM, _lib.ERR_SEQ_LEN, _lib.ERR_CHUNK, _lib.ERR_SHAPE):
        raise GDN2ShapeError(msg)
    raise GDN2Error(msg)


def _dtype_code(dt):
    return _lib.GDN2_F32 if dt == torch.float32 else _lib.GDN2_BF16


def chunk_size_for(dtype, chunk_size=None, D=128) -> int:
    """Chunk size: explicit, else the module-level BT override, else 128 for
    bfloat16 inputs with D = 64 and 64 otherwise (float32, and bfloat16 at
    D = 128 and 256: at D = 128 the chunk-64 forward, whose state scan forms the
    outputs, takes 0.48 ms at B8 T8192 H6 against 0.56 ms at chunk 128).

    The reference's default BT = 256 (gdn2_fwd.py:29), explicit or as the
    module constant, runs at the automatic choice: a 256 x 256 float32 inverse
    does not fit a gfx950 workgroup's LDS, and results do not depend on the
    chunk size beyond rounding.  Other sizes than 64 and 128 are refused by the
    library's shape check (GDN2ShapeError)."""
    bt = chunk_size if chunk_size is not None else BT
    if bt is None or int(bt) == 256:
        return 128 if dtype == torch.bfloat16 and D <= 64 else 64
    return int(bt)


# The clip bound set in the library on each device (device index -> value); the
# library starts at the reference's 1e4.
_CLIP_SET: dict = {}


def _clip_value() -> float:
    """The module constant CLIP (gdn2_fwd.py:33), read at call time as the
    reference reads it when it traces; overridable as its README shows
    (README.md:87-92).  It must be finite and positive."""
    try:
        c = float(CLIP)
    except (TypeError, ValueError):
        raise GDN2Error(f"gdn2: CLIP = {CLIP!r} is not a number") from None
    if not (math.isfinite(c) and c > 0.0):
        raise GDN2Error(f"gdn2: CLIP = {CLIP!r} must be finite and positive")
    return c


def _apply_clip(device) -> None:
    """Make CLIP the clip bound of the library's kernels on `device` (a copy into
    each kernel unit's constant memory, made only when CLIP changed; the device
    is synchronised first so that no call in flight sees the change)."""
    c = _clip_value()
    idx = device.index if device.index is not None else torch.cuda.current_device()
    if _CLIP_SET.get(idx, 1e4) == c:
        return
    with torch.cuda.device(idx):
        torch.cuda.synchronize()
        rc = _lib.lib().gdn2_set_clip(c)
    if rc:
        _raise(rc, "gdn2_set_clip")
    _CLIP_SET[idx] = c


class _Prepared:
    """Inputs normalised for the C ABI (contiguous, supported dtypes)."""

    def __init__(self, q, k, v, w, b, g, scale, h0, chunk_size, compute_dtype=None):
        """``compute_dtype=torch.float32`` runs bfloat16 inputs through the
        float32 kernels (the trainable path: the reference upcasts every input
        before any arithmetic, gdn2_fwd.py:100-103,266-272, gdn2_bwd.py:130-142);
        ``in_dtypes`` keeps the caller's dtypes for the gradients."""
        _clip_value()
        xs = (q, k, v, w, b, g)
        for x in xs:
            if not isinstance(x, torch.Tensor):
                raise TypeError("gdn2: q,k,v,w,b,g must be torch tensors on the ROCm device")
        if q.dim() != 4:
            raise GDN2ShapeError(f"gdn2: expected (B,T,H,D) inputs, got shape {tuple(q.shape)}")
        for x in xs[1:]:
            if x.shape != q.shape:
                raise GDN2ShapeError(
                    f"gdn2: all inputs must share shape {tuple(q.shape)}; got {tuple(x.shape)}")
        in_dt = q.dtype if q.dtype in _SUPPORTED_IN else torch.float32
        if any(x.dtype != in_dt for x in (k, v, w, b)):
            in_dt = torch.float32
        g_dt = torch.float32
        if in_dt == torch.bfloat16 and g.dtype == torch.bfloat16:
            g_dt = torch.bfloat16
        code = _dtype_code(in_dt)
        if compute_dtype == torch.float32:
            if in_dt == torch.bfloat16:
                # float32 arithmetic and residuals on the bfloat16 inputs as they are
                # (GDN2_BF16_F32): no float32 copies of the inputs or gradients
                code = _lib.GDN2_BF16_F32
            else:
                in_dt = g_dt = torch.float32
        self.B, self.T, self.H, self.D = q.shape
        self.BT = chunk_size_for(in_dt, chunk_size, self.D)
        # dtype code of the library calls; tile_dt is the workspace / MFMA operand type
        self.code = code
        self.tile_dt = torch.bfloat16 if code == _lib.GDN2_BF16 else torch.float32
        self.args = (self.B, self.T, self.H, self.D, self.BT, code, _dtype_code(g_dt))
        # T % BT != 0: the last chunk is short (GDN2_FWD_PARTIAL_CHUNK); the
        # reference asserts instead (gdn2_fwd.py:146)
        self.N = -(-self.T // self.BT) if self.BT > 0 else 0
        self.partial = self.BT > 0 and self.T % self.BT != 0
        rc = _lib.lib().gdn2_validate(self.B, self.N * self.BT if self.partial else self.T,
                                      *self.args[2:])
        if rc:
            _raise(rc, f"gdn2 (B,T,H,D)={tuple(q.shape)}, BT={self.BT}")
        if h0 is not None and tuple(h0.shape) != (self.B, self.H, self.D, self.D):
            raise GDN2ShapeError(f"gdn2: h0 must be (B,H,D,D); got {tuple(h0.shape)}")
        dev = q.device
        if dev.type != "cuda" or any(x.device != dev for x in xs):
            raise GDN2Error("gdn2: inputs must live on one ROCm device (torch 'cuda'); "
                            "this library has no CPU path")
        _apply_clip(dev)
        self.in_dtypes = tuple(x.dtype for x in xs)
        self.q, self.k, self.v, self.w, self.b = (x.to(in_dt).contiguous() for x in xs[:5])
        self.g = g.to(g_dt).contiguous()
        self.in_dt, self.g_dt = in_dt, g_dt
        self.scale = float(scale)
        self.h0 = None if h0 is None else h0.to(device=dev, dtype=torch.float32).contiguous()
        self.device = dev

    def stream(self):
        return torch.cuda.current_stream(self.device).cuda_stream

    @staticmethod
    def ptr(x):
        return None if x is None else x.data_ptr()


def _run_forward(p: _Prepared, debug_a: bool = False, flags: int = 0):
    """One gdn2_fwd call; `flags` as in include/gdn2.h (GDN2_FWD_SAVE_A,
    GDN2_FWD_SEGMENTS(n)).  The debug path ignores flags."""
    L = _lib.lib()
    if p.partial:
        flags |= _lib.FWD_PARTIAL_CHUNK
    # the debug path keeps every residual tile: sized as the residual-keeping forward
    nbytes = L.gdn2_fwd_workspace_bytes_ex(
        *p.args[:6], (_lib.FWD_PARTIAL_CHUNK | _lib.FWD_SAVE_A) if debug_a else flags)
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=p.device)
    out = torch.empty((p.B, p.T, p.H, p.D), dtype=torch.float32, device=p.device)
    h_final = torch.empty((p.B, p.H, p.D, p.D), dtype=torch.float32, device=p.device)
    common = (p.stream(), *p.args, p.ptr(p.q), p.ptr(p.k), p.ptr(p.v), p.ptr(p.w), p.ptr(p.b),
              p.ptr(p.g), p.ptr(p.h0), p.scale, out.data_ptr(), h_final.data_ptr(),
              ws.data_ptr(), nbytes)
    a_out = None
    if debug_a:
        a_out = torch.empty((p.B, p.H, p.N, p.BT, p.BT), dtype=torch.float32,
                            device=p.device)
        rc = L.gdn2_fwd_debug(*common, a_out.data_ptr())
    else:
        rc = L.gdn2_fwd(*common, flags)
    if rc:
        _raise(rc, "gdn2_fwd")
    return out, h_final, ws, a_out


def gdn2_pallas_forward(q, k, v, w, b, g, scale, h0=None, debug_tag="", chunk_size=None):
    """Forward A->B->C->D (gdn2_fwd.py:400-424) on the gfx950 library.

    T need not be a multiple of the chunk size: the last chunk of each sequence
    is then short, padded inside the kernels with neutral tokens (the reference
    asserts T % BT == 0, gdn2_fwd.py:146).

    ``debug_tag`` prefixes the GDN2_FWD_DIAG stage reports (gdn2_fwd.py:47-76,
    406-419); without GDN2_FWD_DIAG=1 it is unused.
    """
    p = _Prepared(q, k, v, w, b, g, scale, h0, chunk_size)
    if _GDN2_FWD_DIAG:
        out, h_final, res = _forward_with_residuals(p)
        for name, key in (("kernel_A_Aqk", "Aqk"), ("kernel_A_Akk", "Akk"),
                          ("kernel_B_wy_inverse_A", "A"), ("kernel_C_w_pseudo", "w_pseudo"),
                          ("kernel_C_u", "u"), ("kernel_C_kg", "kg"), ("kernel_C_qg", "qg")):
            _stage_diag(f"{debug_tag}:{name}", res[key])
        _diag_kernel_d(debug_tag, out, h_final)
        return out, h_final
    out, h_final, _, _ = _run_forward(p)
    return out, h_final


def _diag_kernel_d(tag: str, out, h_final):
    """The reference's kernel-D reports (gdn2_fwd.py:363,365)."""
    _stage_diag(f"{tag}:kernel_D_h_final", h_final)
    _stage_diag(f"{tag}:kernel_D_o", out)


def _residual_views(p: _Prepared, ws: torch.Tensor):
    """Workspace tensors as (B,H,N,...) views in the reference's layouts."""
    B, H, D, BT, N = p.B, p.H, p.D, p.BT, p.N
    es = 4 if p.tile_dt == torch.float32 else 2
    NC = B * H * N
    sizes = [("W", NC * BT * D * es), ("UT", NC * D * BT * es), ("KgT", NC * D * BT * es),
             ("Qg", NC * BT * D * es), ("Aqk", NC * BT * BT * es), ("GL", NC * D * 4),
             ("HT", NC * D * D * es), ("VnT", NC * D * BT * es)]
    off, views = 0, {}
    for name, nb in sizes:
        dt = torch.float32 if name == "GL" else p.tile_dt
        views[name] = ws[off:off + nb].view(dt)
        off = (off + nb + 255) // 256 * 256
    f = lambda x: x.float()
    shp = (B, H, N)
    idx = torch.arange(BT, device=p.device)
    causal = (idx[:, None] >= idx[None, :])
    # bfloat16 W, UT, KgT, HT, VnT keep their last dimension in chained order
    # (gdn2_common.h kpos): undo it for the views
    chained = p.tile_dt == torch.bfloat16
    nat = lambda x, n: x[..., _kpos_index(n, x.device)] if chained else x
    # float32 W and KgT are in the scans' split pair layout: decode them
    spl = (lambda x: x) if chained else _split_decode
    return {
        "w_pseudo": f(spl(nat(views["W"].view(*shp, BT, D), D))),
        "u": f(nat(views["UT"].view(*shp, D, BT), BT).transpose(-1, -2)),
        "kg": f(spl(nat(views["KgT"].view(*shp, D, BT), BT)).transpose(-1, -2)),
        "qg": f(views["Qg"].view(*shp, BT, D)),
        "Aqk": torch.where(causal, f(views["Aqk"].view(*shp, BT, BT)), 0.0),
        "gc_last": f(views["GL"].view(*shp, D)),
        "h_pre_all": f(nat(views["HT"].view(*shp, D, D), D).transpose(-1, -2)),
        "v_new_all": f(nat(views["VnT"].view(*shp, D, BT), BT).transpose(-1, -2)),
    }


def _split_decode(x: torch.Tensor) -> torch.Tensor:
    """Rows of a float32 tile stored in the split pair layout of the float32
    scans (csrc/gdn2_common.h) as float32: each 128-byte run of 32 elements holds
    the bfloat16 hi parts (bytes 0-63) and lo parts (64-127), chunk j of each
    part the elements 4j..4j+3 and 16+4j..16+4j+3; the value is hi + lo."""
    *lead, L = x.shape
    parts = x.contiguous().view(torch.bfloat16).reshape(*lead, L // 32, 2, 4, 2, 4).float()
    val = parts[..., 0, :, :, :] + parts[..., 1, :, :, :]          # (.., runs, j, half, slot)
    return val.transpose(-3, -2).reshape(*lead, L)                  # element 16 half + 4 j + slot


def _kpos_index(n: int, device) -> torch.Tensor:
    """Stored position of each logical column in the chained order of
    gdn2_common.h kpos: column 16*half + 4*lg + r of a 32-block at 8*lg + 4*half + r."""
    c = torch.arange(n, device=device)
    return (c & ~31) | (((c >> 2) & 3) << 3) | (((c >> 4) & 1) << 2) | (c & 3)


def gdn2_pallas_forward_raw(q, k, v, w, b, g, scale, h0=None, chunk_size=None):
    """Forward from pre-activation inputs, the caller's preparation fused into
    the prep kernel: q,k are L2-normalised over D (divided by max(|x|_2,
    1e-12), as torch.nn.functional.normalize), w,b pass through a sigmoid and
    g becomes -softplus(g) -- the BASELINE input distributions' construction.
    Equal to ``gdn2_pallas_forward`` on the activated inputs; no reference
    counterpart (the reference takes activated inputs, gdn2_fwd.py:400).
    Inference only (no autograd)."""
    p = _Prepared(q, k, v, w, b, g, scale, h0, chunk_size)
    out, h_final, _, _ = _run_forward(p, flags=_lib.FWD_RAW_INPUTS)
    return out, h_final


def gdn2_pallas_forward_varlen(q, k, v, w, b, g, scale, cu_seqlens, h0=None,
                               chunk_size=None, raw=False):
    """Forward over a variable-length batch packed along T.

    q..g are (1, T, H, D) holding num_seqs sequences back to back;
    ``cu_seqlens`` (num_seqs + 1 integers, 0 first, T last, non-decreasing)
    marks their boundaries.  Each sequence is chunked on its own (any length:
    a short last chunk is padded inside the kernels with neutral tokens) and
    scanned from ``h0[s]`` ((num_seqs, H, D, D) float32, default zeros) to
    ``h_final[s]``.  Returns ``out`` (1, T, H, D) float32 and ``h_final``.
    The same as running ``gdn2_pallas_forward`` per sequence.  ``raw=True``
    fuses the input activations (``gdn2_pallas_forward_raw``).  No reference
    counterpart (the reference needs equal lengths with T % BT == 0,
    gdn2_fwd.py:145-146); forward only."""
    if q.dim() != 4 or q.shape[0] != 1:
        raise GDN2ShapeError(f"gdn2 varlen: expected packed (1,T,H,D) inputs, got {tuple(q.shape)}")
    _, T, H, D = q.shape
    cu_host = torch.as_tensor(cu_seqlens).detach().to("cpu", torch.int64).reshape(-1)
    if cu_host.numel() < 2 or int(cu_host[0]) != 0 or int(cu_host[-1]) != T or \
            bool((cu_host[1:] < cu_host[:-1]).any()):
        raise GDN2ShapeError("gdn2 varlen: cu_seqlens must start at 0, end at T and not decrease")
    S = cu_host.numel() - 1
    # reuse the (B,T,H,D) checks with T padded to a whole chunk
    p_chk = _Prepared(*(x[:, :0] for x in (q, k, v, w, b, g)), scale, None, chunk_size)
    BT = p_chk.BT
    dev = q.device
    if h0 is not None and tuple(h0.shape) != (S, H, D, D):
        raise GDN2ShapeError(f"gdn2 varlen: h0 must be (num_seqs,H,D,D); got {tuple(h0.shape)}")
    lens = cu_host[1:] - cu_host[:-1]
    nch = (lens + BT - 1) // BT
    cu_chunks = torch.zeros(S + 1, dtype=torch.int64)
    cu_chunks[1:] = torch.cumsum(nch, 0)
    total = int(cu_chunks[-1])
    seq_of = torch.repeat_interleave(torch.arange(S), nch)
    cstart = torch.empty(total + 1, dtype=torch.int64)
    cstart[:total] = cu_host[seq_of] + (torch.arange(total) - cu_chunks[seq_of]) * BT
    cstart[total] = T
    cu_d = cu_chunks.to(torch.int32).to(dev)
    cs_d = cstart.to(torch.int32).to(dev)
    in_dt, g_dt = p_chk.in_dt, p_chk.g_dt
    xs = [x.to(in_dt).contiguous() for x in (q, k, v, w, b)] + [g.to(g_dt).contiguous()]
    h0c = None if h0 is None else h0.to(device=dev, dtype=torch.float32).contiguous()
    L = _lib.lib()
    nbytes = L.gdn2_fwd_varlen_workspace_bytes(total, H, D, BT, _dtype_code(in_dt))
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=dev)
    out = torch.empty((1, T, H, D), dtype=torch.float32, device=dev)
    h_final = torch.empty((S, H, D, D), dtype=torch.float32, device=dev)
    rc = L.gdn2_fwd_varlen(torch.cuda.current_stream(dev).cuda_stream, S, cu_d.data_ptr(),
                           cs_d.data_ptr(), total, T, H, D, BT, _dtype_code(in_dt),
                           _dtype_code(g_dt), *(x.data_ptr() for x in xs),
                           None if h0c is None else h0c.data_ptr(), float(scale),
                           out.data_ptr(), h_final.data_ptr(), ws.data_ptr(), nbytes,
                           _lib.FWD_RAW_INPUTS if raw else 0)
    if rc:
        _raise(rc, f"gdn2_fwd_varlen (T,H,D)=({T},{H},{D}), {S} sequences")
    return out, h_final


def gdn2_pallas_forward_with_residuals(q, k, v, w, b, g, scale, h0=None, debug_tag="",
                                       chunk_size=None):
    """gdn2_fwd.py:427-457: forward plus the per-chunk intermediates.

    Residual keys follow the reference (:452-456), all float32 in (B,H,N,...)
    layout: Aqk, Akk, A, h_pre_all, v_new_all, w_pseudo, u, kg, qg, gc_last.
    ``Akk`` is not materialised by the kernels; it is recovered here as
    strict_tril(A^{-1}) for inspection.
    """
    p = _Prepared(q, k, v, w, b, g, scale, h0, chunk_size)
    return _forward_with_residuals(p)


def _forward_with_residuals(p: _Prepared):
    out, h_final, ws, a_out = _run_forward(p, debug_a=True)
    res = _residual_views(p, ws)
    res["A"] = a_out
    eye = torch.eye(p.BT, device=p.device, dtype=torch.float64)
    res["Akk"] = torch.tril(torch.linalg.inv(a_out.double()) - eye, -1).float()
    return out, h_final, res


# ---------------------------------------------------------------------------
# The forward's stages one at a time (the reference's module-level kernels).
# Each runs a HIP kernel of libgdn2_hip.so in float32 at chunk 64 and returns
# float32 tensors in the reference's (B,H,N,BT,...) layouts.
_STAGE_BT = 64


def _stage_chunk(D: int) -> int:
    """The stage functions run at chunk 64 (float32 tiles); a module BT
    override to another size is refused, as the reference asserts its
    shapes against BT (gdn2_fwd.py:144,249)."""
    bt = chunk_size_for(torch.float32, None, D)
    if bt != _STAGE_BT:
        raise GDN2ShapeError(f"gdn2: the per-kernel stage functions run at chunk "
                             f"{_STAGE_BT}; BT = {bt} is not supported for them")
    return _STAGE_BT


def _stage_inputs(q, k, v, w, b, g, scale):
    D = q.shape[-1] if isinstance(q, torch.Tensor) and q.dim() == 4 else 0
    p = _Prepared(q, k, v, w, b, g, scale, None, _stage_chunk(D),
                  compute_dtype=torch.float32)
    if p.partial:
        raise GDN2ShapeError(f"gdn2: L={p.T} must be divisible by BT={p.BT} "
                             f"(gdn2_fwd.py:145,301)")
    return p


def _chunk_tensor(x, name, shape, device):
    if not isinstance(x, torch.Tensor):
        raise TypeError(f"gdn2: {name} must be a torch tensor on the ROCm device")
    if tuple(x.shape) != tuple(shape):
        raise GDN2ShapeError(f"gdn2: {name} must have shape {tuple(shape)}; got "
                             f"{tuple(x.shape)}")
    if x.device != device:
        raise GDN2Error(f"gdn2: {name} must live on {device}")
    return x.to(torch.float32).contiguous()


def build_chunk_scores_pallas(q, k, b, g, scale):
    """Kernel A, gdn2_fwd.py:142-170: per chunk, Aqk = scale * causal
    sum_d q_i k_j e^{gc_i - gc_j} and Akk = strictly lower sum_d (b k)_i k_j
    e^{gc_i - gc_j}, each (B,H,N,BT,BT) float32 and sanitized.  The HIP kernel
    is the forward's fwd_prep run to its score blocks (stage kPrepScores).
    D may be 64, 128 or 256 (the reference asserts 128)."""
    p = _stage_inputs(q, k, k, k, b, g, scale)
    aqk = torch.empty((p.B, p.H, p.N, p.BT, p.BT), dtype=torch.float32, device=p.device)
    akk = torch.empty_like(aqk)
    rc = _lib.lib().gdn2_chunk_scores(p.stream(), *p.args, p.ptr(p.q), p.ptr(p.k), p.ptr(p.b),
                                      p.ptr(p.g), p.scale, aqk.data_ptr(), akk.data_ptr())
    if rc:
        _raise(rc, "gdn2_chunk_scores")
    return aqk, akk


def wy_solve_pallas(Akk):
    """Kernel B, gdn2_fwd.py:246-260: A = (I + Akk)^{-1} per chunk, for Akk of
    shape (..., BT, BT) (only its strictly lower part is read), float32."""
    if not isinstance(Akk, torch.Tensor):
        raise TypeError("gdn2: Akk must be a torch tensor on the ROCm device")
    BT = _stage_chunk(128)
    if Akk.dim() < 2 or tuple(Akk.shape[-2:]) != (BT, BT):
        raise GDN2ShapeError(f"gdn2: Akk must end in ({BT},{BT}); got {tuple(Akk.shape)}")
    if Akk.device.type != "cuda":
        raise GDN2Error("gdn2: Akk must live on the ROCm device (torch 'cuda')")
    _apply_clip(Akk.device)
    akk = Akk.to(torch.float32).contiguous()
    a = torch.empty_like(akk)
    n = akk.numel() // (BT * BT)
    rc = _lib.lib().gdn2_wy_solve(torch.cuda.current_stream(akk.device).cuda_stream, n, BT,
                                  akk.data_ptr(), a.data_ptr())
    if rc:
        _raise(rc, "gdn2_wy_solve")
    return a


def recompute_wy_pallas(q, k, v, w, b, g, A):
    """Kernel C, gdn2_fwd.py:298-330: w_pseudo = A (b k e^gc), u = A (w v),
    kg = k e^{gc_last - gc}, qg = q e^gc (each (B,H,N,BT,D)) and gc_last
    (B,H,N,D), float32 and sanitized, from the inputs and the given A
    (B,H,N,BT,BT)."""
    p = _stage_inputs(q, k, v, w, b, g, 1.0)
    a = _chunk_tensor(A, "A", (p.B, p.H, p.N, p.BT, p.BT), p.device)
    shp = (p.B, p.H, p.N, p.BT, p.D)
    w_pseudo, u, kg, qg = (torch.empty(shp, dtype=torch.float32, device=p.device)
                           for _ in range(4))
    gc_last = torch.empty((p.B, p.H, p.N, p.D), dtype=torch.float32, device=p.device)
    rc = _lib.lib().gdn2_recompute_wy(p.stream(), *p.args, p.ptr(p.q), p.ptr(p.k), p.ptr(p.v),
                                      p.ptr(p.w), p.ptr(p.b), p.ptr(p.g), a.data_ptr(),
                                      w_pseudo.data_ptr(), u.data_ptr(), kg.data_ptr(),
                                      qg.data_ptr(), gc_last.data_ptr())
    if rc:
        _raise(rc, "gdn2_recompute_wy")
    return w_pseudo, u, kg, qg, gc_last


def _combine(Aqk, w_pseudo, u, kg, qg, gc_last, scale, h0, debug_tag, with_state):
    if not isinstance(w_pseudo, torch.Tensor) or w_pseudo.dim() != 5:
        raise GDN2ShapeError("gdn2: w_pseudo must be a (B,H,N,BT,D) tensor")
    B, H, N, BT, D = w_pseudo.shape
    if BT != _stage_chunk(D):
        raise GDN2ShapeError(f"gdn2: chunk tiles of {BT} tokens; the stage functions take "
                             f"{_STAGE_BT}")
    dev = w_pseudo.device
    if dev.type != "cuda":
        raise GDN2Error("gdn2: the chunk tiles must live on the ROCm device (torch 'cuda')")
    aqk = _chunk_tensor(Aqk, "Aqk", (B, H, N, BT, BT), dev)
    wp, uu, kk, qq = (_chunk_tensor(x, n, (B, H, N, BT, D), dev) for x, n in
                      ((w_pseudo, "w_pseudo"), (u, "u"), (kg, "kg"), (qg, "qg")))
    gl = _chunk_tensor(gc_last, "gc_last", (B, H, N, D), dev)
    h0c = None if h0 is None else _chunk_tensor(h0, "h0", (B, H, D, D), dev)
    _apply_clip(dev)
    L = _lib.lib()
    nbytes = L.gdn2_chunk_combine_workspace_bytes(B, N, H, D, BT)
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=dev)
    out = torch.empty((B, N * BT, H, D), dtype=torch.float32, device=dev)
    h_final = torch.empty((B, H, D, D), dtype=torch.float32, device=dev)
    h_pre = v_new = None
    if with_state:
        h_pre = torch.empty((B, H, N, D, D), dtype=torch.float32, device=dev)
        v_new = torch.empty((B, H, N, BT, D), dtype=torch.float32, device=dev)
    ptr = lambda x: None if x is None else x.data_ptr()
    rc = L.gdn2_chunk_combine(torch.cuda.current_stream(dev).cuda_stream, B, N, H, D, BT,
                              aqk.data_ptr(), wp.data_ptr(), uu.data_ptr(), kk.data_ptr(),
                              qq.data_ptr(), gl.data_ptr(), ptr(h0c), float(scale),
                              out.data_ptr(), h_final.data_ptr(), ptr(h_pre), ptr(v_new),
                              ws.data_ptr(), nbytes)
    if rc:
        _raise(rc, "gdn2_chunk_combine")
    # the reference returns o per chunk: (B,L,H,D) -> (B,H,N,BT,D)
    o = out.view(B, N, BT, H, D).permute(0, 3, 1, 2, 4).contiguous()
    h_final = _stage_diag(f"{debug_tag}:kernel_D_h_final", h_final)
    o = _stage_diag(f"{debug_tag}:kernel_D_o", o)
    return (o, h_final, h_pre, v_new) if with_state else (o, h_final)


def gdn2_inter_chunk_combine(Aqk, w_pseudo, u, kg, qg, gc_last, scale, h0=None, debug_tag=""):
    """Kernel D, gdn2_fwd.py:338-366: the serial state scan over the chunks
    and the outputs, from the per-chunk tiles of kernels A and C.  Returns o
    (B,H,N,BT,D) and h_final (B,H,D,D), float32.  h0 is sanitized first."""
    return _combine(Aqk, w_pseudo, u, kg, qg, gc_last, scale, h0, debug_tag, False)


def gdn2_inter_chunk_combine_with_state(Aqk, w_pseudo, u, kg, qg, gc_last, scale, h0=None,
                                        debug_tag=""):
    """gdn2_fwd.py:369-397: as gdn2_inter_chunk_combine, plus h_pre_all
    (B,H,N,D,D), the state entering each chunk, and v_new_all (B,H,N,BT,D).
    These two come in the (B,H,N,...) layout the backward consumes; the
    reference's lax.scan stacks them chunk-first, (N,B,H,...)."""
    return _combine(Aqk, w_pseudo, u, kg, qg, gc_last, scale, h0, debug_tag, True)
