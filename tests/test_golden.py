"""The committed fixtures (tests/golden/*.npz) re-derived by the oracle -- CPU."""
from pathlib import Path

import numpy as np

from oracle import gdn2_oracle as O

GOLD = Path(__file__).resolve().parent / "golden"


def load(name):
    with np.load(GOLD / name, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def test_fwd_config1_fixture():
    z = load("fwd_config1.npz")
    xs = [z[n] for n in "qkvwbg"]
    ref = O.make_inputs(1, 512, 2, 64, seed=0)
    for a, b in zip(xs, ref):
        np.testing.assert_array_equal(a, b)
    out, h = O.chunked_fwd(*xs, float(z["scale"]), BT=64, clip=False)
    assert np.max(np.abs(out - z["out"])) < 1e-12
    assert np.max(np.abs(h - z["h_final"])) < 1e-12
    # the reference's own algorithm (with its +-20 decay clip) agrees to far below 1e-4
    out_c, h_c = O.chunked_fwd(*xs, float(z["scale"]), BT=64, clip=True, dtype=np.float32)
    assert np.max(np.abs(out_c - z["out"])) < 1e-5
    assert np.max(np.abs(h_c - z["h_final"])) < 1e-4


def test_bwd_small_fixture():
    z = load("bwd_small.npz")
    xs = [z[n] for n in "qkvwbg"]
    got = O.chunked_bwd(*xs, float(z["scale"]), z["do"], z["dh"], h0=z["h0"], BT=32,
                        clip=False)
    for name, g in zip(["dq", "dk", "dv", "dw", "db", "dg", "dh0"], got):
        assert np.max(np.abs(g - z[name])) < 1e-10 * max(1.0, np.abs(z[name]).max()), name
