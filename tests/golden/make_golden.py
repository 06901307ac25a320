"""Write the golden fixtures under tests/golden/ from the float64 oracle.

    python tests/golden/make_golden.py

fwd_config1.npz: BASELINE configs[0] -- (B=1,T=512,H=2,D=64) float32 inputs,
  seed 0, scale 1/8, chunk 64; expected out and h_final from the token
  recurrence (float64, stored as float64).
bwd_small.npz: (B=1,T=128,H=2,D=64), seed 0, h0 ~ 0.1 N(0,1), cotangents
  d_out ~ N(0,1) and d_h_final ~ N(0,1) (seed 1); expected gradients of
  (q,k,v,w,b,g,h0) from the oracle's chunked backward (float64), which the
  CPU tests pin against torch.autograd of the recurrence.
The reference ships no numeric fixtures (its tests check shapes only), so
these are the build's own vectors; tests/test_golden.py re-derives them.
"""
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))
from oracle import gdn2_oracle as O  # noqa: E402


def fwd_config1():
    xs = O.make_inputs(1, 512, 2, 64, seed=0)
    out, h = O.recurrent_fwd(*xs, 64 ** -0.5)
    return dict(q=xs[0], k=xs[1], v=xs[2], w=xs[3], b=xs[4], g=xs[5], scale=64 ** -0.5,
                out=out, h_final=h)


def bwd_small():
    xs = O.make_inputs(1, 128, 2, 64, seed=0)
    rng = np.random.default_rng(1)
    h0 = (0.1 * rng.standard_normal((1, 2, 64, 64))).astype(np.float32)
    do = rng.standard_normal((1, 128, 2, 64)).astype(np.float32)
    dh = rng.standard_normal((1, 2, 64, 64)).astype(np.float32)
    grads = O.chunked_bwd(*xs, 64 ** -0.5, do, dh, h0=h0, BT=64, clip=False)
    out, h = O.recurrent_fwd(*xs, 64 ** -0.5, h0=h0)
    names = ["dq", "dk", "dv", "dw", "db", "dg", "dh0"]
    return dict(q=xs[0], k=xs[1], v=xs[2], w=xs[3], b=xs[4], g=xs[5], h0=h0, do=do, dh=dh,
                scale=64 ** -0.5, out=out, h_final=h, **dict(zip(names, grads)))


if __name__ == "__main__":
    np.savez_compressed(HERE / "fwd_config1.npz", **fwd_config1())
    np.savez_compressed(HERE / "bwd_small.npz", **bwd_small())
    for f in sorted(HERE.glob("*.npz")):
        print(f.name, f.stat().st_size)
