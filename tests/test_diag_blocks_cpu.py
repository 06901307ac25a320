"""The exact sums of a diagonal 16 x 16 score block under strong decay, pinned
on the CPU.

fwd_prep and gram_bwd factorise a diagonal block around its 8th token,
q_i e^{lc_i - lc_m} . k_j e^{lc_m - lc_j}; past kMaxDiagExp of decay on either
side of that token they take the hierarchical sums instead
(diag_block_exact in csrc/gdn2_fwd.hip, diag_grads_exact in
csrc/gdn2_bwd.hip): for groups of G = 16, 8, 4, 2 tokens the pairs with i in
the upper and j in the lower half of one group, factorised around the group's
boundary token b = G*(i//G) + G/2 - 1, then the diagonal i = j.  This file
restates that level structure in numpy and checks what makes it exact: every
pair i >= j is summed exactly once, no factor exceeds 1 for g <= 0, the float32
sums match the float64 direct sums where the single-center factors overflow,
and the kernels' threshold keeps the single-center operands finite and normal.
"""
import re
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[1]


def max_diag_exp():
    src = (ROOT / "gdn2-jax-kernel_amd" / "csrc" / "gdn2_common.h").read_text()
    return float(re.search(r"constexpr float kMaxDiagExp = ([0-9.]+)f;", src).group(1))


def levels():
    """(G, boundary, upper, cross mask) per level, as the kernels form them."""
    li = np.arange(16)
    out = []
    for L in range(5):
        G = 16 >> L
        half = G // 2
        upper = (li % G) >= half
        bnd = (li // G) * G + half - 1
        i, j = li[:, None], li[None, :]
        if L < 4:
            cross = (i // G == j // G) & (i % G >= half) & (j % G < half)
        else:
            cross = i == j
        out.append((L, G, bnd, upper, cross))
    return out


def hier_sums(q, k, lc, cap):
    """float32 sum_d q_i k_j e^{lc_i - lc_j} over the levels (lanes = tokens)."""
    acc = np.zeros((16, 16), np.float32)
    for L, G, bnd, upper, cross in levels():
        lb = lc[bnd]                                   # the boundary's cumsum, per token
        ex = np.where(upper[:, None], lc - lb, lb - lc)
        f = np.ones_like(lc) if L == 4 else np.exp(np.minimum(ex, cap)).astype(np.float32)
        t = (q * f) @ (k * f).T
        acc += np.where(cross, t, np.float32(0))
    return acc


def test_levels_partition_the_lower_triangle():
    count = np.zeros((16, 16), int)
    for *_, cross in levels():
        count += cross
    i, j = np.indices((16, 16))
    assert (count[i >= j] == 1).all() and (count[i < j] == 0).all()


def test_factors_never_exceed_one_for_decay():
    rng = np.random.default_rng(0)
    g = -np.abs(rng.standard_normal((16, 8))) * 50
    lc = np.cumsum(g, axis=0)
    for L, G, bnd, upper, cross in levels()[:4]:
        lb = lc[bnd]
        ex = np.where(upper[:, None], lc - lb, lb - lc)
        assert (ex <= 0).all(), L


def test_hierarchical_sums_exact_where_single_center_overflows():
    rng = np.random.default_rng(1)
    D = 64
    q = rng.standard_normal((16, D)).astype(np.float32)
    k = rng.standard_normal((16, D)).astype(np.float32)
    g = (-30.0 * np.log1p(np.exp(rng.standard_normal((16, D))))).astype(np.float32)
    lc = np.cumsum(g, axis=0, dtype=np.float32)
    cap = max_diag_exp()
    ref = np.einsum("id,jd,ijd->ij", q.astype(np.float64), k.astype(np.float64),
                    np.exp(lc[:, None, :].astype(np.float64) - lc[None, :, :]))
    low = np.tril(np.ones((16, 16), bool))
    got = hier_sums(q, k, lc, cap)
    scale = np.einsum("id,jd,ijd->ij", np.abs(q), np.abs(k),
                      np.exp(np.minimum(lc[:, None, :] - lc[None, :, :], 0.0)))
    assert np.all(np.abs(got - ref)[low] <= 1e-5 * scale[low] + 1e-30)
    # the single-center factors of this block leave float32's range: the
    # kernels' criterion (a channel past kMaxDiagExp) holds, so they take the
    # sums above
    lm = lc[7]
    assert np.abs(lc - lm).max() > cap
    with np.errstate(over="ignore"):
        assert not np.isfinite(np.exp(np.abs(lc - lm)).astype(np.float32)).all()


def test_threshold_keeps_single_center_operands_finite_and_normal():
    cap = np.float32(max_diag_exp())
    big, small = np.exp(cap, dtype=np.float32), np.exp(-cap, dtype=np.float32)
    tiny = np.finfo(np.float32).tiny            # also bfloat16's smallest normal
    # operands up to kClip times the largest factor stay finite
    assert np.isfinite(np.float32(1e4) * big)
    # operands down to 2e-12 times the smallest factor stay normal
    assert np.float32(2e-12) * small >= tiny
    # the largest exponent float32 holds is ~88.7: the threshold sits below it
    assert cap < np.log(np.finfo(np.float32).max)
