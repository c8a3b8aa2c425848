"""CPU checks that pin the token-sampler oracle (oracle/sample.py): the Philox4x32-10 known-answer
vectors published with Random123, an independent scalar Philox, the uniform mapping, the sampled
distribution against softmax(logits / T) (the reference's chat.py:103-107), the greedy and
no-candidate cases, and planted mistakes that the distribution test must catch."""
import numpy as np
import pytest
from scipy import stats

from oracle import sample as osample

# philox4x32 with 10 rounds: (counter, key) -> output, from Random123's kat_vectors
KAT = [
    ((0x00000000, 0x00000000, 0x00000000, 0x00000000), (0x00000000, 0x00000000),
     (0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8)),
    ((0xFFFFFFFF, 0xFFFFFFFF, 0xFFFFFFFF, 0xFFFFFFFF), (0xFFFFFFFF, 0xFFFFFFFF),
     (0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD)),
    ((0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344), (0xA4093822, 0x299F31D0),
     (0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1)),
]


@pytest.mark.parametrize("ctr,key,want", KAT)
def test_philox_known_answers(ctr, key, want):
    got = tuple(int(x) for x in osample.philox4x32(*ctr, *key))
    assert got == want


def scalar_philox(ctr, key):
    """Philox4x32-10 on Python ints, written from the paper's round function independently of the
    vectorised oracle."""
    x0, x1, x2, x3 = ctr
    k0, k1 = key
    for r in range(10):
        prod_a = 0xD2511F53 * x0
        prod_b = 0xCD9E8D57 * x2
        x0, x1, x2, x3 = ((prod_b >> 32) ^ x1 ^ k0, prod_b & 0xFFFFFFFF,
                          (prod_a >> 32) ^ x3 ^ k1, prod_a & 0xFFFFFFFF)
        k0 = (k0 + 0x9E3779B9) & 0xFFFFFFFF
        k1 = (k1 + 0xBB67AE85) & 0xFFFFFFFF
    return x0, x1, x2, x3


def test_vectorised_philox_matches_scalar():
    rng = np.random.default_rng(0)
    for _ in range(50):
        ctr = tuple(int(x) for x in rng.integers(0, 2**32, 4))
        key = tuple(int(x) for x in rng.integers(0, 2**32, 2))
        assert tuple(int(x) for x in osample.philox4x32(*ctr, *key)) == scalar_philox(ctr, key)


def test_uniform_mapping_and_counter_layout():
    seed, offset = 0x1234_5678_9ABC_DEF0, (7 << 32) + 3
    u = osample.uniforms(3, 11, seed, offset)
    assert np.all(u > 0) and np.all(u < 1)
    assert np.all(u.astype(np.float32).astype(np.float64) == u)   # exact in fp32
    for row in range(3):
        for v in range(11):
            w = scalar_philox((v // 4, row, offset & 0xFFFFFFFF, offset >> 32),
                              (seed & 0xFFFFFFFF, seed >> 32))[v % 4]
            assert u[row, v] == (2 * (w >> 9) + 1) * 2.0 ** -24


def test_uniforms_are_uniform():
    u = osample.uniforms(200, 1000, 5, 0).ravel()
    assert stats.kstest(u, "uniform").pvalue > 1e-3


LOGITS6 = np.array([1.0, -0.5, 2.0, 0.0, 0.7, -2.0])


def chi2_pvalue(tokens, probs):
    counts = np.bincount(tokens, minlength=len(probs))
    return stats.chisquare(counts, probs * len(tokens)).pvalue


def softmax(x):
    e = np.exp(x - x.max())
    return e / e.sum()


def draw(logits, n, temperature, seed=11, offset=0, score=None):
    batch = np.tile(logits, (n, 1))
    if score is None:
        return osample.sample(batch, temperature, seed, offset)
    u = osample.uniforms(n, len(logits), seed, offset)
    return np.argmax(score(batch, temperature, u), axis=1)


@pytest.mark.parametrize("temperature", [1.0, 0.5, 2.0])
def test_samples_follow_the_softmax(temperature):
    tokens = draw(LOGITS6, 40000, temperature)
    assert chi2_pvalue(tokens, softmax(LOGITS6 / temperature)) > 1e-4


@pytest.mark.parametrize("name,score", [
    ("temperature dropped", lambda lg, t, u: lg - np.log(-np.log(u))),
    ("sign of the noise flipped", lambda lg, t, u: lg / t + np.log(-np.log(u))),
    ("E used in place of ln E", lambda lg, t, u: lg / t + np.log(u)),
])
def test_planted_mistakes_fail_the_distribution_test(name, score):
    tokens = draw(LOGITS6, 40000, 0.5, score=score)
    assert chi2_pvalue(tokens, softmax(LOGITS6 / 0.5)) < 1e-6, name


def test_greedy_and_special_values():
    lg = np.array([[0.0, 3.0, 3.0, -1.0],            # tie: lowest index
                   [np.nan, -np.inf, 0.5, np.nan],   # NaN never wins
                   [-np.inf, -np.inf, -np.inf, -np.inf],
                   [np.nan, np.nan, np.nan, np.nan]])
    assert osample.sample(lg, 0.0, 1, 0).tolist() == [1, 2, -1, -1]
    s = osample.sample(lg, 1.0, 1, 0).tolist()
    assert s[1] == 2 and s[2:] == [-1, -1]


def test_tiny_temperature_is_greedy_and_offsets_give_fresh_draws():
    rng = np.random.default_rng(1)
    lg = rng.normal(size=(64, 500))
    assert (osample.sample(lg, 1e-4, 3, 0) == lg.argmax(1)).all()
    a = osample.sample(lg, 1.0, 3, 0)
    assert (a == osample.sample(lg, 1.0, 3, 0)).all()
    assert (a != osample.sample(lg, 1.0, 3, 1)).mean() > 0.5
    assert (a != osample.sample(lg, 1.0, 4, 0)).mean() > 0.5
