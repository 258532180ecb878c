"""The oracle's sampler (orc_random_unit, orc_choose_token) against closed
forms and an independent numpy form (moonlight_chat.c:89-131)."""
import math

import numpy as np
import pytest

import oracle_lib as O
from sampler_util import nucleus_choice, xorshift_unit


def test_random_unit_is_xorshift64():
    import ctypes
    state = ctypes.c_uint64(0x9E3779B97F4A7C15)
    mine = 0x9E3779B97F4A7C15
    for _ in range(1000):
        got = O.lib().orc_random_unit(ctypes.byref(state))
        u, mine = xorshift_unit(mine)
        assert got == u and state.value == mine
        assert 0.0 <= got < 1.0


def test_greedy_first_index_of_maximum():
    rng = np.random.default_rng(3)
    for vocab in (1, 7, 512, 163840):
        lg = rng.standard_normal(vocab).astype(np.float32)
        assert O.choose_token(lg, 0.0, 0.9, 5)[0] == int(np.argmax(lg))
        assert O.choose_token(lg, 0.0, 0.9, 5)[1] == 5  # the state does not move
    lg = rng.standard_normal(1000).astype(np.float32)
    lg[[17, 400]] = 9.0  # ties: the lower index
    assert O.choose_token(lg, 0.0, 1.0)[0] == 17
    lg[3] = np.nan  # a NaN never replaces the running best ...
    assert O.choose_token(lg, 0.0, 1.0)[0] == 17
    lg[0] = np.nan  # ... and a NaN at index 0 is never replaced
    assert O.choose_token(lg, 0.0, 1.0)[0] == 0


def test_small_top_p_is_greedy():
    """A nucleus of one candidate: every draw returns the argmax."""
    rng = np.random.default_rng(4)
    lg = (3.0 * rng.standard_normal(4096)).astype(np.float32)
    best = int(np.argmax(lg))
    state = 77
    for _ in range(50):
        tok, state = O.choose_token(lg, 1.0, 1e-6, state)
        assert tok == best


def test_equal_logits_pick_by_count():
    """Equal logits: p = 1/V each, candidates in token order, so the draw u
    returns token ceil(u * count) - 1 of the nucleus of count tokens."""
    for vocab, top_p in ((1000, 0.5), (4096, 0.9), (163840, 0.95), (300, 1.0)):
        lg = np.full(vocab, 0.25, np.float32)
        p = float(np.float32(1.0) / np.float32(vocab))
        count = max(1, math.ceil(np.float64(np.float32(top_p)) / p) - 2)
        while count < vocab and count * p < np.float64(np.float32(top_p)):
            count += 1
        state = 1234567
        for _ in range(20):
            u, nxt = xorshift_unit(state)
            tok, state = O.choose_token(lg, 0.8, top_p, state)
            assert state == nxt
            assert tok == max(math.ceil(u * count) - 1, 0), (vocab, top_p, u)


@pytest.mark.parametrize("temperature,top_p", [(1.0, 0.9), (0.7, 0.5), (1.5, 1.0), (0.3, 0.95)])
def test_matches_numpy_form(temperature, top_p):
    rng = np.random.default_rng(int(temperature * 10 + top_p * 100))
    lg = (2.0 * rng.standard_normal(20000)).astype(np.float32)
    lg[rng.integers(0, 20000, 200)] = lg[5]  # equal probabilities: token order
    state, compared = 99, 0
    for _ in range(40):
        u, _ = xorshift_unit(state)
        want, margin, _ = nucleus_choice(lg, temperature, top_p, u)
        tok, state = O.choose_token(lg, temperature, top_p, state)
        if margin > 1e-6:
            assert tok == want
            compared += 1
    assert compared >= 35
