"""GPU parity of the device sampler (choose_token, moonlight_chat.c:96-131)
through mlk_sample on chosen logits, against `nucleus_choice` (the device
arithmetic restated in numpy: exp in double rounded once to fp32, stable
descending order, serial double running sums) and, where the draw is not
within 1e-6 of a boundary, the oracle's choose_token (glibc expf).

The cases drive each path of the radix selection: random logits at the full
163,840-token vocabulary (a candidate list of a few hundred keys), all-equal
logits (every key equal: the list overflows and the final workgroup scans
all keys, the tie is the j-th token of 163,840), logits of eight distinct
values (ties of ~20,000 equal keys), a block of exactly equal top logits (a
tie ranked inside the list), top_p at 0 and 1, temperatures that underflow
most probabilities to zero mass, tiny vocabularies, and non-finite logits.
"""
import numpy as np
import pytest

import oracle_lib as O
from floyd_amd import native
from sampler_util import nucleus_choice, xorshift_unit

pytestmark = pytest.mark.gpu

V_FULL = 163840


def device_tokens(logits, draws):
    """mlk_sample over one upload of `logits` for each (temperature, top_p, u)."""
    d = native.DeviceBuffer.from_array(np.asarray(logits, np.float32))
    try:
        return [native.sample(d, len(logits), t, p, u) for t, p, u in draws]
    finally:
        d.close()


def check_draws(logits, draws, min_compared):
    got = device_tokens(logits, draws)
    compared = 0
    for (t, p, u), tok in zip(draws, got):
        want, margin, count = nucleus_choice(logits, t, p, u)
        assert tok == want, (t, p, u, count, margin)
        compared += 1
    assert compared >= min_compared
    return got


def draw_grid(temps, tops, seed, per=4):
    rng = np.random.default_rng(seed)
    out = []
    for t in temps:
        for p in tops:
            us = [0.0, 0.999999] + list(rng.random(per))
            out += [(t, p, float(u)) for u in us]
    return out


def test_sampler_random_full_vocab(device):
    print(f"[gpu] sampler random logits V={V_FULL}", flush=True)
    rng = np.random.default_rng(1)
    logits = (rng.standard_normal(V_FULL) * 3.0).astype(np.float32)
    draws = draw_grid((0.7, 1.0, 2.0), (0.9, 0.5, 0.99, 1.0), seed=2)
    check_draws(logits, draws, len(draws))


def test_sampler_matches_oracle_choose_token(device):
    """The oracle's choose_token (glibc expf, qsort) on the same logits and
    xorshift state, away from cumulative boundaries."""
    print("[gpu] sampler vs oracle choose_token", flush=True)
    rng = np.random.default_rng(3)
    logits = (rng.standard_normal(V_FULL) * 2.0).astype(np.float32)
    compared = 0
    state = 12345
    for t, p in ((0.7, 0.9), (1.0, 0.95), (0.3, 0.8)):
        for _ in range(6):
            u, nxt = xorshift_unit(state)
            e_tok, e_state = O.choose_token(logits, t, p, state)
            assert e_state == nxt
            tok = device_tokens(logits, [(t, p, u)])[0]
            if nucleus_choice(logits, t, p, u)[1] > 1e-6:
                assert tok == e_tok, (t, p, u)
                compared += 1
            state = nxt
    assert compared >= 12


def test_sampler_all_equal_logits(device):
    """Every key equal: the draw picks the j-th token in token order."""
    print(f"[gpu] sampler all-equal logits V={V_FULL}", flush=True)
    logits = np.full(V_FULL, 0.25, np.float32)
    draws = [(1.0, 0.9, 0.0), (1.0, 0.9, 0.5), (1.0, 0.9, 0.999999), (0.7, 1.0, 0.3),
             (1.0, 0.0, 0.7), (1.0, 0.37, 0.123)]
    got = check_draws(logits, draws, len(draws))
    assert got[0] == 0 and got[4] == 0


def test_sampler_few_distinct_values(device):
    print(f"[gpu] sampler eight distinct logits V={V_FULL}", flush=True)
    rng = np.random.default_rng(5)
    logits = (rng.integers(0, 8, V_FULL) * 0.75).astype(np.float32)
    draws = draw_grid((0.5, 1.0, 3.0), (0.3, 0.9, 1.0), seed=6, per=3)
    check_draws(logits, draws, len(draws))


def test_sampler_tied_top_block(device):
    """37 exactly equal largest logits among random ones: the crossing lands
    inside the tie, ranked from the candidate list."""
    print("[gpu] sampler tied top block", flush=True)
    rng = np.random.default_rng(7)
    logits = (rng.standard_normal(V_FULL) - 6.0).astype(np.float32)
    tied = rng.choice(V_FULL, 37, replace=False)
    logits[tied] = 4.0
    draws = [(1.0, p, float(u)) for p in (0.05, 0.5, 0.9) for u in rng.random(5)]
    got = check_draws(logits, draws, len(draws))
    assert set(got) <= set(tied.tolist())


def test_sampler_underflow_and_extremes(device):
    """Temperatures at which most probabilities are exactly 0 (zero mass),
    top_p 0 (the largest p, lowest token) and 1 (every candidate)."""
    print("[gpu] sampler underflow / top_p extremes", flush=True)
    rng = np.random.default_rng(9)
    logits = (rng.standard_normal(V_FULL) * 4.0).astype(np.float32)
    draws = [(0.01, 1.0, 0.5), (0.01, 0.9, 0.999999), (0.05, 1.0, 0.0), (0.05, 1.0, 0.999999),
             (1.0, 0.0, 0.5), (2.0, 1.0, 0.75)]
    got = check_draws(logits, draws, len(draws))
    assert got[4] == int(np.argmax(logits))


@pytest.mark.parametrize("vocab", [1, 2, 7, 1000, 1024, 1025, 4097])
def test_sampler_small_vocab(device, vocab):
    print(f"[gpu] sampler V={vocab}", flush=True)
    rng = np.random.default_rng(vocab)
    logits = (rng.standard_normal(vocab) * 2.0).astype(np.float32)
    draws = draw_grid((0.5, 1.0), (0.5, 0.9, 1.0), seed=vocab + 1, per=2)
    check_draws(logits, draws, len(draws))


def test_sampler_greedy_and_nonfinite(device):
    print("[gpu] sampler greedy / non-finite", flush=True)
    rng = np.random.default_rng(11)
    logits = rng.standard_normal(5000).astype(np.float32)
    logits[[17, 4000]] = logits.max() + 1.0  # equal maxima: the lower index
    assert device_tokens(logits, [(0.0, 0.9, 0.5)]) == [17]
    bad = logits.copy()
    bad[123] = np.nan
    d = native.DeviceBuffer.from_array(bad)
    try:
        with pytest.raises(native.NativeError, match="not finite"):
            native.sample(d, bad.size, 1.0, 0.9, 0.5)
        assert native.sample(d, bad.size, 0.0, 0.9, 0.5) == 17  # NaN never wins the arg-max
    finally:
        d.close()
