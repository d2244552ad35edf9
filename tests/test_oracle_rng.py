"""Pins the sampler's uniform stream (oracle/rng.c) on the CPU: Philox4x32-10
against the known-answer vectors published with it (Salmon et al., SC 2011),
and the law of the derived uniforms."""

import numpy as np
from scipy import stats

import oracle

KAT = [  # (counter, key, output) of Philox4x32-10
    ([0, 0, 0, 0], [0, 0], [0x6627e8d5, 0xe169c58d, 0xbc57ac4c, 0x9b00dbd8]),
    ([0xffffffff] * 4, [0xffffffff] * 2, [0x408f276d, 0x41c83b0e, 0xa20bc7c6, 0x6d5451fd]),
    ([0x243f6a88, 0x85a308d3, 0x13198a2e, 0x03707344], [0xa4093822, 0x299f31d0],
     [0xd16cfe09, 0x94fdcceb, 0x5001e420, 0x24126ea1]),
]


def test_philox_known_answers():
    for ctr, key, out in KAT:
        assert oracle.philox4x32_10(ctr, key).tolist() == out


def test_uniforms_take_the_block_words_in_order():
    """u(c, i) uses word i % 4 of block i / 4 of counter (c_lo, c_hi, i / 4, 0)."""
    seed, event = 0x0123456789ABCDEF, (7 << 32) + 5
    u = oracle.philox_uniforms(seed, event, 9)
    key = [seed & 0xffffffff, seed >> 32]
    for i in range(9):
        w = oracle.philox4x32_10([5, 7, i // 4, 0], key)[i % 4]
        assert u[i] == np.float32((int(w) >> 8) * 2.0 ** -24)


def test_uniform_law_and_independence_across_events():
    u = np.concatenate([oracle.philox_uniforms(42, c, 5) for c in range(20000)]).astype(np.float64)
    assert u.min() >= 0.0 and u.max() < 1.0
    assert abs(u.mean() - 0.5) < 4 * np.sqrt(1 / 12 / u.size)
    assert abs(u.var() - 1 / 12) < 0.003
    assert stats.kstest(u, "uniform").pvalue > 1e-3
    # neighbouring events and slots are uncorrelated
    m = u.reshape(20000, 5)
    assert abs(np.corrcoef(m[:-1, 0], m[1:, 0])[0, 1]) < 0.03
    assert abs(np.corrcoef(m[:, 0], m[:, 4])[0, 1]) < 0.03
    # a different seed gives a different stream
    assert not np.array_equal(oracle.philox_uniforms(43, 0, 5), oracle.philox_uniforms(42, 0, 5))
