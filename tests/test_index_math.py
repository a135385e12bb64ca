"""Host-side checks of the integer tricks the HIP kernels rely on (CPU only).

``csrc/qk_norm_rope.hip`` maps a thread index u < 1024 to its head as
``(u * uph_magic) >> 21`` with ``uph_magic = 2^21 // (D / 16) + 1`` instead of
dividing by the per-head unit count D / 16. This test checks that identity for
every unit count the kernel accepts (D / 16 <= 1024) and every thread index,
in the 32-bit unsigned arithmetic the kernel uses.
"""

import numpy as np


def test_unit_to_head_multiply_shift_is_exact():
    u = np.arange(1024, dtype=np.uint64)
    for d in range(1, 1025):
        magic = (1 << 21) // d + 1
        prod = u * np.uint64(magic)
        assert int(prod.max()) < (1 << 32), "the product must fit the kernel's 32 bits"
        got = (prod >> np.uint64(21)).astype(np.int64)
        np.testing.assert_array_equal(got, (u // np.uint64(d)).astype(np.int64), err_msg=f"D/16={d}")


def test_multiply_shift_catches_a_wrong_magic():
    # Planted mistake: dropping the +1 breaks exactness for some unit count.
    u = np.arange(1024, dtype=np.uint64)
    broken = any(
        not np.array_equal((u * np.uint64((1 << 21) // d)) >> np.uint64(21), u // np.uint64(d))
        for d in range(1, 1025))
    assert broken
