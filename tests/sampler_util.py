"""Checks for the caller-side sampler (choose_token, moonlight_chat.c:96-131).

`xorshift_unit` restates Marsaglia's xorshift64 with shifts (13, 7, 17), the
generator random_unit (moonlight_chat.c:89-94) uses, independently of the
oracle's C.  `nucleus_choice` is a vectorised numpy form of the device
arithmetic (exp in double rounded once to fp32, stable descending order,
cumulative sums): it returns the token and how far the draw lies from the
nearest cumulative boundary, so a comparison can skip draws that a one-ulp
difference in a probability (glibc expf against a correctly rounded exp)
could move to the neighbouring candidate.
"""
import numpy as np

MASK = (1 << 64) - 1


def xorshift_unit(state):
    x = state
    x ^= (x << 13) & MASK
    x ^= x >> 7
    x ^= (x << 17) & MASK
    return (x >> 11) * (1.0 / 9007199254740992.0), x


def nucleus_choice(logits, temperature, top_p, u):
    logits = np.asarray(logits, np.float32)
    m = logits[int(np.argmax(logits))]
    e = (logits - m) / np.float32(temperature)
    p = np.exp(e.astype(np.float64)).astype(np.float32)
    p = p / np.float32(p.astype(np.float64).sum())
    order = np.lexsort((np.arange(p.size), -p.astype(np.float64)))
    cs = np.cumsum(p[order].astype(np.float64))
    reach = np.nonzero(cs >= np.float64(np.float32(top_p)))[0]
    count = min(int(reach[0]), p.size - 1) + 1 if reach.size else p.size
    sample = u * cs[count - 1]
    idx = int(np.argmax(cs[:count] >= sample)) if np.any(cs[:count] >= sample) else count - 1
    margin = float(np.min(np.abs(cs[:count] - sample))) / max(float(cs[count - 1]), 1e-300)
    return int(order[idx]), margin, count
