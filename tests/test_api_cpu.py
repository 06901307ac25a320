"""Package surface and host-side behaviour of the Python drop-in -- CPU only.

Mirrors the reference's tests/test_imports.py:3-12 (exports and __version__)
and its trace-time shape assertions (gdn2_fwd.py:145-146)."""
import pytest
import torch


def test_imports():
    from gdn2_package import gdn2_pallas_forward, gdn2_pallas_forward_trainable
    assert gdn2_pallas_forward_trainable is not None
    assert gdn2_pallas_forward is not None


def test_version():
    import gdn2_package
    assert hasattr(gdn2_package, "__version__")


def test_reference_constants_exist():
    from gdn2_package import gdn2_fwd
    assert gdn2_fwd.CLIP == 1e4 and gdn2_fwd.MB == 16


def _inputs(shape, dtype=torch.float32):
    return [torch.zeros(shape, dtype=dtype) for _ in range(6)]


@pytest.mark.parametrize("shape", [(1, 512, 2, 96), (1, 500, 2, 64)])
def test_shape_errors_are_assertion_errors(shape):
    import gdn2_package as gp
    with pytest.raises(AssertionError):
        gp.gdn2_pallas_forward(*_inputs(shape), 0.1)
    with pytest.raises(gp.GDN2ShapeError):
        gp.gdn2_pallas_forward(*_inputs(shape), 0.1)


def test_mismatched_input_shapes_rejected():
    import gdn2_package as gp
    xs = _inputs((1, 128, 2, 64))
    xs[3] = torch.zeros((1, 128, 2, 32))
    with pytest.raises(gp.GDN2ShapeError):
        gp.gdn2_pallas_forward(*xs, 0.1)


def test_no_cpu_fallback():
    """Host tensors are refused: the only compute path is the gfx950 library."""
    import gdn2_package as gp
    with pytest.raises(gp.GDN2Error):
        gp.gdn2_pallas_forward(*_inputs((1, 128, 2, 64)), 0.1)


def test_chunk_size_resolution():
    from gdn2_package import gdn2_fwd
    assert gdn2_fwd.chunk_size_for(torch.bfloat16) == 128
    assert gdn2_fwd.chunk_size_for(torch.float32) == 64
    old = gdn2_fwd.BT
    try:
        gdn2_fwd.BT = 64              # README.md:87-92 style override, read at call time
        assert gdn2_fwd.chunk_size_for(torch.bfloat16) == 64
    finally:
        gdn2_fwd.BT = old
    import gdn2_package as gp
    with pytest.raises(gp.GDN2ShapeError):   # fp32 with a 128-token chunk is not supported
        gp.gdn2_pallas_forward(*_inputs((1, 256, 2, 64)), 0.1, chunk_size=128)
