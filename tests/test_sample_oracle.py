"""Pins the CPU restatement of the reference's token sampling (oracle/sample_oracle.c).

  * java.util.Random: published outputs of new Random(0) / new Random(42) (nextInt, nextDouble);
  * AutoregressiveModel.sampleToken (AutoregressiveModel.java:323-386): greedy first maximum for
    temperature <= 0 without a draw; closed-form categorical draws (two outcomes, nucleus cuts
    worked by hand, equal probabilities kept in index order); the empirical distribution of many
    draws against softmax(logits / T) and its nucleus (a temperature multiplied instead
    of divided, a dropped renormalisation or a wrong cut fails these);
  * the sample function of AutoregressiveModel.of (:413-425) with DistributionFeatures.softmax
    (DistributionFeatures.java:129-141): a logit of exactly 0 gets probability 0, the maximum
    exp(eps), and sampleToken's second softmax at temperature 1 -- worked by hand.
No GPU is used.
"""
import math

import numpy as np
import pytest

import oracle


def test_java_random_published_values():
    assert oracle.JavaRandom(0).next_int() == -1155484576
    assert oracle.JavaRandom(42).next_int() == -1170105035
    assert oracle.JavaRandom(0).next_double() == 0.730967787376657
    assert oracle.JavaRandom(42).next_double() == 0.7275636800328681
    r = oracle.JavaRandom(7)
    a = [r.next_double() for _ in range(1000)]
    assert all(0.0 <= x < 1.0 for x in a) and len(set(a)) == 1000


def test_greedy_takes_the_first_maximum_and_draws_nothing():
    v = [1.0, 3.0, 3.0, 2.0]
    for t in (0.0, -1.0):
        rng = oracle.JavaRandom(3)
        before = rng.state.value
        assert oracle.sample_token(v, t, 0.9, rng)[0] == 1
        assert rng.state.value == before
    assert oracle.sample_token(v, 1.0, 1.0, None)[0] == 1     # random == null
    assert oracle.model_sample(v, 0.0, oracle.JavaRandom(1))[0] == 1


def _draws(fn, n_seeds=400):
    out = []
    for seed in range(n_seeds):
        rng = oracle.JavaRandom(seed)
        r_expect = oracle.JavaRandom(seed).next_double()
        k, r, _ = fn(rng)
        assert r == r_expect  # exactly one nextDouble per sampled token
        out.append((k, r))
    return out


def test_two_outcomes_closed_form():
    # softmax([0, ln 3]) = [1/4, 3/4]: index 0 exactly when r < 1/4
    for k, r in _draws(lambda g: oracle.sample_token([0.0, math.log(3.0)], 1.0, 1.0, g)):
        assert k == (0 if r < 0.25 else 1)
    # temperature 2 halves the logits: softmax([0, ln 9 / 2]) = [1/4, 3/4] again
    for k, r in _draws(lambda g: oracle.sample_token([0.0, math.log(9.0)], 2.0, 1.0, g)):
        assert k == (0 if r < 0.25 else 1)


def test_nucleus_cuts_by_hand():
    logits = [math.log(x) for x in (1.0, 2.0, 3.0, 4.0)]  # probabilities .1 .2 .3 .4
    # top_p .5: sorted .4, .3 -> .7 >= .5, keep {3, 2}, renormalised 3/7, 4/7 (index order 2, 3)
    for k, r in _draws(lambda g: oracle.sample_token(logits, 1.0, 0.5, g)):
        assert k == (2 if r < 3 / 7 else 3)
    # top_p .39: the largest alone
    for k, r in _draws(lambda g: oracle.sample_token(logits, 1.0, 0.39, g)):
        assert k == 3
    # top_p .75: .4 + .3 + .2 -> keep {1, 2, 3}: .2/.9, .3/.9, .4/.9
    for k, r in _draws(lambda g: oracle.sample_token(logits, 1.0, 0.75, g)):
        assert k == (1 if r < 2 / 9 else (2 if r < 5 / 9 else 3))
    # top_p <= 0 keeps exactly one value (the loop's first step already reaches it)
    for k, r in _draws(lambda g: oracle.sample_token(logits, 1.0, 0.0, g), 50):
        assert k == 3


def test_nucleus_keeps_equal_probabilities_in_index_order():
    # four equal logits: .25 each; the stable sort keeps 0, 1 for top_p .5 (.25 + .25 >= .5)
    for k, r in _draws(lambda g: oracle.sample_token([1.0] * 4, 1.0, 0.5, g)):
        assert k == (0 if r < 0.5 else 1)
    # ties below a larger value: [2, 1, 1, 1] -> the largest first, then the lowest tied index
    e = np.exp(np.array([2.0, 1, 1, 1]) - 2.0)
    p = e / e.sum()
    cut = p[0] + p[1]
    assert cut > 0.6
    for k, r in _draws(lambda g: oracle.sample_token([2.0, 1.0, 1.0, 1.0], 1.0, 0.6, g)):
        assert k == (0 if r < p[0] / cut else 1)


@pytest.mark.parametrize("temperature,top_p", [(0.7, 1.0), (1.5, 1.0), (1.0, 0.8)])
def test_empirical_distribution(temperature, top_p):
    rng = np.random.default_rng(5)
    logits = rng.normal(0, 1.5, 6)
    p = np.exp(logits / temperature - (logits / temperature).max())
    p /= p.sum()
    if top_p < 1.0:
        order = np.argsort(-p, kind="stable")
        keep = order[: int(np.searchsorted(np.cumsum(p[order]), top_p) + 1)]
        q = np.zeros_like(p)
        q[keep] = p[keep]
        p = q / q.sum()
    n = 20000
    counts = np.zeros(6)
    g = oracle.JavaRandom(12345)  # one generator: first draws of consecutive seeds are correlated
    for _ in range(n):
        counts[oracle.sample_token(logits, temperature, top_p, g)[0]] += 1
    expect = p * n
    live = expect > 0
    assert counts[~live].sum() == 0
    chi2 = (((counts - expect) ** 2)[live] / expect[live]).sum()
    assert chi2 < 30.0, (counts, expect)  # 5 degrees of freedom: p < 2e-5 under the right law


def test_softmax_ignore_zero():
    x = oracle.softmax_ignore_zero([0.0, math.log(3.0), 2.5])
    eps = 2.220446049250313e-16
    e = np.array([0.0, math.exp(math.log(3.0) - 2.5), math.exp(eps)])
    np.testing.assert_allclose(x, e / e.sum(), rtol=1e-15, atol=0)
    assert x[0] == 0.0


def test_model_sample_function_by_hand():
    # logits [0, 2] at T = 1: the 0 logit gets probability 0 and the maximum exp(eps) ~ 1, so
    # the softmax is [0, 1]; sampleToken's second softmax gives [e^-1, 1] / (1 + e^-1)
    p0 = math.exp(-1.0) / (1.0 + math.exp(-1.0))
    for k, r in _draws(lambda g: oracle.model_sample([0.0, 2.0], 1.0, g)):
        assert k == (0 if r < p0 else 1)
    # the second softmax flattens: with V = 1000 and one dominant logit (probability ~1 after the
    # first softmax) every index keeps weight e^-1 against its 1, so 300 draws hit ~260 indices
    lg = np.zeros(1000)
    lg[7] = 50.0
    g = oracle.JavaRandom(99)
    ks = [oracle.model_sample(lg, 1.0, g)[0] for _ in range(300)]
    assert len(set(ks)) > 200
