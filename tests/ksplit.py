"""K ranges of the in-group K split (SG_KSPLIT in csrc/sgemm_gfx950.hip), for
the tests that compare the split kernel with the one-group kernel on its two
halves (tests/test_vm.py, tests/test_gpu_parity.py)."""


def k_split_ranges(k, dk):
    """The K ranges [0, k0) and [k1, k) that the two groups of the in-group K
    split sum: ktiles = ceil(k / dk) tiles with the first one shifted by
    kshift; group 0 takes the first h = ceil(ktiles / 2), group 1 the last h,
    whose first tile is group 0's last (loaded as zeros) when ktiles is odd.
    A group with one shifted tile takes the slow path, whose tiles start at
    k = 0 with no shift (the last one cut at k)."""
    ktiles = -(-k // dk)
    kshift = (-k) % dk
    h = (ktiles + 1) // 2
    if h < 2:
        kshift = 0
    k0 = min(max(h * dk - kshift, 0), k)
    k1 = min(max((ktiles - h + (ktiles & 1)) * dk - kshift, 0), k)
    return k0, k1
