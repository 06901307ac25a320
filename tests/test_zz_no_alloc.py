"""gdn2_fwd_noalloc (the forward whose workspace is the library's fixed device
array) through the C ABI against gdn2_fwd with a caller workspace: bit-equal
outputs on two calls in a row, the second smaller (the scratch then holds the
first call's tiles), for bfloat16 and float32 inputs; a workload beyond the
scratch and GDN2_FWD_SAVE_A are rejected before any launch."""
import numpy as np
import pytest
import torch

from oracle import gdn2_oracle as O

pytestmark = pytest.mark.gpu


def _run(L, dev, xs, h0, scale, BT, dtype, noalloc, flags=0):
    from gdn2_package import _lib
    B, T, H, D = xs[0].shape
    out = torch.empty((B, T, H, D), dtype=torch.float32, device=dev)
    hf = torch.empty((B, H, D, D), dtype=torch.float32, device=dev)
    code = _lib.GDN2_F32 if dtype == torch.float32 else _lib.GDN2_BF16
    common = (torch.cuda.current_stream().cuda_stream, B, T, H, D, BT, code, _lib.GDN2_F32,
              *(x.data_ptr() for x in xs), None if h0 is None else h0.data_ptr(), scale,
              out.data_ptr(), hf.data_ptr())
    if noalloc:
        rc = L.gdn2_fwd_noalloc(*common, flags)
    else:
        nb = L.gdn2_fwd_workspace_bytes_ex(B, T, H, D, BT, code, flags)
        ws = torch.empty(max(nb, 1), dtype=torch.uint8, device=dev)
        rc = L.gdn2_fwd(*common, ws.data_ptr(), nb, flags)
    torch.cuda.synchronize()
    return rc, out, hf


def _inputs(B, T, H, D, dtype, dev, seed):
    xs = O.make_inputs(B, T, H, D, seed=seed)
    t = [torch.tensor(x, device=dev) for x in xs]
    return [x.to(dtype).contiguous() for x in t[:5]] + [t[5].contiguous()]


@pytest.mark.parametrize("dtype,BT,D,segs", [
    (torch.bfloat16, 128, 128, 0),      # the scan forms the outputs
    (torch.float32, 64, 64, 0),         # idem, float32
    (torch.bfloat16, 64, 64, 0),        # a separate output pass (h^T / v_new^T tiles)
    (torch.bfloat16, 64, 128, 4),       # segmented scan (the SEG region, its flag slot)
])
def test_noalloc_matches_gdn2_fwd(dev, dtype, BT, D, segs):
    from gdn2_package import _lib
    L = _lib.lib()
    for (B, T, H), seed in (((2, 1024, 4), 1), ((1, 200, 2), 2)):   # second call smaller
        xs = _inputs(B, T, H, D, dtype, dev, seed)
        h0 = 0.1 * torch.randn((B, H, D, D), device=dev)
        flags = _lib.FWD_PARTIAL_CHUNK | (_lib.FWD_SEGMENTS(segs) if segs else 0)
        rc1, o1, h1 = _run(L, dev, xs, h0, D ** -0.5, BT, dtype, True, flags)
        rc2, o2, h2 = _run(L, dev, xs, h0, D ** -0.5, BT, dtype, False, flags)
        assert rc1 == 0 and rc2 == 0, (rc1, rc2)
        assert torch.equal(o1, o2) and torch.equal(h1, h2), (B, T, H)
        ro, rh = O.recurrent_fwd(*[x.float().cpu().numpy() for x in xs], D ** -0.5,
                                 h0=h0.cpu().numpy())
        tol = 1e-4 if dtype == torch.float32 else 2e-2
        assert np.abs(o1.cpu().numpy() - ro).max() <= tol + tol * np.abs(ro).max()
        assert np.abs(h1.cpu().numpy() - rh).max() <= tol + tol * np.abs(rh).max()


def test_noalloc_rejects_before_launch(dev):
    from gdn2_package import _lib
    L = _lib.lib()
    # 2 x 32768 x 16 heads of bf16 at chunk 128 needs ~0.8 GB of workspace
    B, T, H, D = 2, 32768, 16, 128
    code = _lib.GDN2_BF16
    p = torch.empty(16, dtype=torch.uint8, device=dev).data_ptr()   # never dereferenced
    stream = torch.cuda.current_stream().cuda_stream
    rc = L.gdn2_fwd_noalloc(stream, B, T, H, D, 128, code, _lib.GDN2_F32, p, p, p, p, p, p, None,
                            0.1, p, p, 0)
    assert rc == _lib.ERR_SCRATCH
    assert L.gdn2_strerror(rc).decode().startswith("workload too large")
    rc = L.gdn2_fwd_noalloc(stream, 1, 256, 1, D, 128, code, _lib.GDN2_F32, p, p, p, p, p, p,
                            None, 0.1, p, p, _lib.FWD_SAVE_A)
    assert rc == _lib.ERR_FLAGS
