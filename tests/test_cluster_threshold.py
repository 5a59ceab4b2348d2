"""The GPU clustering decides the reference's Jaccard test
d = 1 - (float)inter / (float)uni <= thr (clustering_sylos_labini.cpp:35-46,
:97) without the division whenever inter / uni lies more than a small margin
from 1 - thr (JaccardTest in xspmm_amd/csrc/cluster_gpu.hip).  This checks the
margin argument in float32 arithmetic: over every (inter, uni) with
uni <= 3000, and over sampled pairs up to the kernel's 2^19 column blocks, a
fast decision never contradicts the IEEE float evaluation, at thresholds that
put exact ties (inter / uni = 1 - thr) on the grid.  The GPU permutations
themselves are compared with the host's bit for bit in test_gpu_cluster.py.
"""
import numpy as np

f32 = np.float32


def fast_decisions(inter, uni, thr):
    """(definitely close, definitely not close), evaluated in float32 as the
    kernel does: a = 1 - thr, a_hi = a + 2^-20, a_lo = a - 2^-20."""
    a = f32(1.0) - f32(thr)
    a_hi = f32(a + f32(2.0 ** -20))
    a_lo = f32(a - f32(2.0 ** -20))
    fi = inter.astype(f32)
    fu = uni.astype(f32)
    return fi >= (a_hi * fu).astype(f32), fi < (a_lo * fu).astype(f32)


def reference_close(inter, uni, thr):
    d = f32(1.0) - (inter.astype(f32) / uni.astype(f32)).astype(f32)
    return d.astype(f32) <= f32(thr)


THRESHOLDS = [0.5, 0.0, 1.0, 0.25, 0.75, 1.0 / 3.0, 0.1, 0.9, 0.3, 0.6, 2.0 ** -10,
              1 - 2.0 ** -12, 0.5 + 2.0 ** -24, 0.5 - 2.0 ** -25]


def check(inter, uni, thr):
    yes, no = fast_decisions(inter, uni, thr)
    ref = reference_close(inter, uni, thr)
    assert not np.any(yes & no)
    bad_yes = yes & ~ref
    bad_no = no & ref
    assert not bad_yes.any(), (thr, inter[bad_yes][:5], uni[bad_yes][:5])
    assert not bad_no.any(), (thr, inter[bad_no][:5], uni[bad_no][:5])
    return (yes | no).mean()


def test_every_small_pair():
    u = np.arange(1, 3001, dtype=np.int64)
    uni = np.repeat(u, u + 1)
    inter = np.concatenate([np.arange(k + 1) for k in u])
    for thr in THRESHOLDS:
        decided = check(inter, uni, thr)
        assert decided > 0.99  # the division is the rare case


def test_sampled_large_pairs():
    rng = np.random.default_rng(0)
    uni = rng.integers(1, 1 << 19, size=2_000_000)
    for thr in THRESHOLDS + list(rng.random(8)):
        # near the threshold: inter around (1 - thr) * uni, +- a few
        centre = np.floor((1.0 - thr) * uni).astype(np.int64)
        inter = np.clip(centre + rng.integers(-3, 4, size=uni.size), 0, uni)
        check(inter, uni, thr)
        inter = rng.integers(0, uni + 1)
        check(inter, uni, thr)
