"""The gating filter kernel's lane networks (csrc/moe_gating.hip), restated
over the 16 lanes of a row and checked on every 0/1 input.  Each network is a
circuit of min and max only, so by the 0-1 principle a circuit that orders
(or selects from) all 2^16 0/1 inputs correctly does so for every input.

A stage (x, bit): lane p meets lane p ^ x and keeps the minimum when
p & bit, else the maximum.  The DPP patterns the kernel uses map to
x = 1 (quad_perm [1,0,3,2]), 3 ([3,2,1,0]), 2 ([2,3,0,1]), 7 (row_half_mirror),
15 (row_mirror) and 4 (two row rotations)."""
import numpy as np

LANES = np.arange(16)
ALL01 = ((np.arange(1 << 16)[:, None] >> LANES) & 1).astype(np.int8)

SORT16 = [(1, 1), (3, 2), (1, 1), (7, 4), (2, 2), (1, 1), (15, 8), (4, 4), (2, 2), (1, 1)]


def _stage(v, x, bit):
    w = v[:, LANES ^ x]
    return np.where((LANES & bit) != 0, np.minimum(v, w), np.maximum(v, w))


def test_sort16_desc_sorts_every_01_input():
    """sort16_desc / sort16_desc_g: lane p ends with the p-th largest."""
    v = ALL01
    for x, bit in SORT16:
        v = _stage(v, x, bit)
    np.testing.assert_array_equal(v, -np.sort(-ALL01, axis=1))


def test_eighth_of16_selects_the_eighth_largest():
    """eighth_of16_g: the first six stages of the sort (each 8-lane half
    sorted), the larger of each lane and its mirror, then the minimum over
    lanes p ^ 1, p ^ 2 and p ^ 7: every lane holds the 8th largest."""
    v = ALL01
    for x, bit in SORT16[:6]:
        v = _stage(v, x, bit)
    v = np.maximum(v, v[:, LANES ^ 15])
    for x in (1, 2, 7):
        v = np.minimum(v, v[:, LANES ^ x])
    want = -np.sort(-ALL01, axis=1)[:, 7]
    np.testing.assert_array_equal(v, np.repeat(want[:, None], 16, axis=1))


def test_two_list_merge_keeps_the_top16():
    """The 17..32-candidate path: two sorted lists a, b; lane t keeps
    max(a[t], b[15 - t]) and the half-cleaners at distances 8, 4, 2, 1 sort
    the resulting bitonic sequence (checked on all pairs of sorted 0/1 lists)."""
    a = np.array([[1] * i + [0] * (16 - i) for i in range(17)], np.int8)
    pairs = np.array([(i, j) for i in range(17) for j in range(17)])
    top = np.maximum(a[pairs[:, 0]], a[pairs[:, 1]][:, ::-1])
    for x, bit in [(8, 8), (4, 4), (2, 2), (1, 1)]:
        top = _stage(top, x, bit)
    union = np.concatenate([a[pairs[:, 0]], a[pairs[:, 1]]], axis=1)
    np.testing.assert_array_equal(top, -np.sort(-union, axis=1)[:, :16])
