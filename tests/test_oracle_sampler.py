"""Pins the oracle's restatement of the reference samplers (orc_sample:
Sampler.selectSampler, CategoricalSampler, ToppSampler) before it checks the
device sampler.

Checks, independent of the oracle's code: temperature 0 is the first-maximum
argmax; categorical sampling over uniform logits picks floor(coin * n); a
float64 brute force of temperature, softmax, nucleus selection (candidates by
probability, descending, until the mass exceeds topp) and the inverse-CDF walk
picks the oracle's token wherever the decision is not within 1e-6 of a
boundary; topp outside (0, 1) falls back to categorical; a vanishing topp
keeps only the most probable token; and plausible mistakes in that brute force
(no temperature, mass compared with >= instead of >, ascending order, the draw
not scaled by the nucleus mass) disagree with the oracle.  The reference's heap
extracts the nucleus out of descending order in some cases (ToppSampler.java:128
passes i - 1 as the heap size); the oracle reproduces it and flags it, and a
three-token case pins that behaviour.
"""
import numpy as np
import pytest

import oracle.oracle as orc


def brute(logits, temperature, topp, coin, mistake=None, probs=None):
    """float64 restatement: (token, margin) of the intended sampler semantics
    (probs: use these probabilities instead of the float64 softmax)."""
    x = np.asarray(logits, dtype=np.float64)
    n = x.size
    if temperature == 0.0:
        return int(np.argmax(x)), 1.0
    if mistake != "no_temperature":
        x = x / temperature
    e = np.exp(x - x.max())
    p = e / e.sum() if probs is None else np.asarray(probs, dtype=np.float64)
    if topp <= 0 or topp >= 1:
        c = np.cumsum(p)
        i = int(np.searchsorted(c, coin, side="right"))
        i = min(i, n - 1)
        lo = c[i - 1] if i > 0 else 0.0
        return i, min(c[i] - coin, coin - lo)
    cutoff = (1.0 - topp) / (n - 1)
    cand = np.flatnonzero(p >= cutoff)
    order = cand[np.lexsort((cand, -p[cand]))] if mistake != "ascending" else cand[np.lexsort((cand, p[cand]))]
    c = np.cumsum(p[order])
    k = int(np.searchsorted(c, topp, side="left" if mistake == "ge" else "right")) + 1
    k = min(k, order.size)
    mass = c[k - 1]
    margin = abs(mass - topp)
    if k > 1:
        margin = min(margin, abs(topp - c[k - 2]))
    r = coin * (mass if mistake != "unscaled" else 1.0)
    j = min(int(np.searchsorted(c[:k], r, side="right")), k - 1)
    lo = c[j - 1] if j > 0 else 0.0
    return int(order[j]), min(margin, c[j] - r, r - lo)


def cases(seed, count, n_lo=2, n_hi=5000):
    rng = np.random.default_rng(seed)
    for _ in range(count):
        n = int(rng.integers(n_lo, n_hi))
        x = (rng.standard_normal(n) * rng.uniform(0.5, 4.0)).astype(np.float32)
        yield x, float(rng.uniform(0.3, 1.5)), float(rng.choice([0.0, 1.0, rng.uniform(0.2, 0.99)])), \
            float(np.float32(rng.random()))


def test_temperature_zero_is_first_maximum():
    x = np.float32([0.5, 2.0, -1.0, 2.0])
    for coin in (0.0, 0.5, 0.99):
        assert orc.sample(x, 0.0, 0.9, coin)[0] == 1


def test_categorical_uniform_is_floor():
    for n in (2, 7, 1000, 128256):
        x = np.zeros(n, dtype=np.float32)
        for coin in np.float32([0.0, 0.123, 0.5, 0.777, 0.9999]):
            tok, exact, margin, _, _ = orc.sample(x, 1.0, 0.0, float(coin))
            want = int(np.floor(np.float64(coin) * n))
            if margin > 1e-6:
                assert exact == want, (n, coin)
                if n < 10000:  # the float cumulative sum of 128256 terms drifts past the boundary gaps
                    assert tok == want, (n, coin)


def test_matches_float64_brute_force():
    checked = 0
    for x, t, p, coin in cases(11, 300):
        tok, exact, margin, quirk, _ = orc.sample(x, t, p, coin)
        b, bm = brute(x, t, p, coin)
        if min(margin, bm) > 1e-6:
            assert exact == b, (x.size, t, p, coin)
            if not quirk and margin > 1e-6 + 2 * orc.sample.last_shift:
                assert tok == b, (x.size, t, p, coin)
            checked += 1
    assert checked > 200


def test_topp_outside_unit_interval_is_categorical():
    for x, t, _, coin in cases(12, 50):
        cat = orc.sample(x, t, 0.0, coin)[0]
        assert orc.sample(x, t, 1.0, coin)[0] == cat
        assert orc.sample(x, t, -0.5, coin)[0] == cat
        assert orc.sample(x, t, 1.5, coin)[0] == cat


def test_vanishing_topp_keeps_the_top_token():
    for x, t, _, coin in cases(13, 50):
        assert orc.sample(x, t, 1e-7, coin)[0] == int(np.argmax(x))


@pytest.mark.parametrize("mistake", ["no_temperature", "ascending", "unscaled"])
def test_planted_mistakes_disagree(mistake):
    differ = 0
    for x, t, p, coin in cases(14, 200, n_lo=5):
        if not 0 < p < 1 and mistake in ("ascending", "unscaled"):
            continue
        tok, exact, margin, _, _ = orc.sample(x, t, p, coin)
        b, bm = brute(x, t, p, coin, mistake)
        differ += b != exact
    assert differ > 0, mistake


def test_mass_must_exceed_topp():
    """Probabilities 0.5, 0.25, 0.25 (exact in binary) and topp 0.75: after two
    tokens the mass equals topp, which does not exceed it, so the nucleus takes
    the third (ToppSampler.java:125 compares with >); stopping at >= would scale
    the draw by 0.75 and pick the second token for coin 0.9."""
    x = np.log(np.float32([0.5, 0.25, 0.25])).astype(np.float32)
    p = orc.softmax(x)
    assert list(p) == [0.5, 0.25, 0.25]  # exact in float
    tok, exact, _, _, nucleus = orc.sample(x, 1.0, 0.75, 0.9)
    # the two 0.25 tokens tie: the reference's heap may visit them in either order
    assert exact == 2 and nucleus == 3 and tok in (1, 2)
    assert brute(x, 1.0, 0.75, 0.9, probs=p)[0] == 2 and brute(x, 1.0, 0.75, 0.9, "ge", probs=p)[0] == 1


def test_reference_heap_order():
    """ToppSampler's heap on probabilities [0.5, 0.3, 0.2] with topp 0.99:
    extraction 0.5, then (the bound i - 1 leaves 0.3 unsifted) 0.2, then 0.3."""
    x = np.log(np.float32([0.5, 0.3, 0.2])).astype(np.float32)
    # r = coin * mass walks 0.5 | 0.2 | 0.3 in the reference, 0.5 | 0.3 | 0.2 in exact order
    tok, exact, _, quirk, nucleus = orc.sample(x, 1.0, 0.99, 0.6)
    assert (tok, exact, quirk, nucleus) == (2, 1, 1, 3)
    assert orc.sample(x, 1.0, 0.99, 0.1)[:2] == (0, 0)
