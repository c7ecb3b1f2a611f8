"""CPU checks of the test-side restatement of the kernels' B-operand
fragment layout (tests/helpers.shuffle_b), against the element formula
written out with explicit loops."""
import numpy as np

from helpers import shuffle_b


def test_shuffle_b_matches_element_formula():
    rng = np.random.default_rng(0)
    rows, k = 70, 130  # ragged: 3 row blocks, 3 K blocks
    b = rng.standard_normal((rows, k)).astype(np.float32)
    got = shuffle_b(b)
    kb_n = 3
    assert got.size == 96 * 192
    for r in range(96):
        for kk in range(192):
            rb, kb = r // 32, kk // 64
            s, rem = (kk % 64) // 16, kk % 16
            lane = (r % 32) + 32 * (rem // 8)
            idx = (rb * kb_n + kb) * 2048 + (s * 64 + lane) * 8 + rem % 8
            exp = b[r, kk] if r < rows and kk < k else 0.0
            assert got[idx] == exp, (r, kk)
