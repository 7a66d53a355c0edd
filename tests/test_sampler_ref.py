"""The oracle's restatement of Sampler::sample (src/sampler.rs:28-76), pinned
by the reference's own tests (src/sampler.rs:85-130: greedy pick, top-k
truncation) and by closed forms: a plain softmax at top_k 0 / top_p 1, a
one-hot at top_k 1, the temperature limit, and a hand-worked top-p cut."""
import numpy as np

from oracle import numpy_ref


def test_plain_softmax():
    z = np.array([0.5, -1.0, 2.0, 0.0])
    for T in (0.5, 1.0, 3.0):
        e = np.exp(z / T)
        assert np.allclose(numpy_ref.sampler_probs(z, T, 0, 1.0), e / e.sum(), rtol=1e-12)


def test_top_k_one_is_argmax_and_ties_keep_index_order():
    assert np.array_equal(numpy_ref.sampler_probs([1.0, 3.0, 2.0], 1.0, 1, 1.0), [0, 1, 0])
    # equal logits: the stable sort keeps the lower index first
    assert np.array_equal(numpy_ref.sampler_probs([2.0, 5.0, 5.0, 1.0], 1.0, 1, 1.0), [0, 1, 0, 0])


def test_top_k_truncates_like_the_reference_test():
    # src/sampler.rs top_k_truncates: logits [10, 1, 1, 1], k = 2 keeps tokens 0 and 1
    p = numpy_ref.sampler_probs([10.0, 1.0, 1.0, 1.0], 1.0, 2, 1.0)
    assert p[2] == 0 and p[3] == 0 and p[0] > 0.99 and p[1] > 0


def test_top_p_cut_by_hand():
    # probabilities 0.5, 0.3, 0.2 (logits their logs): top_p 0.6 keeps the first
    # two (0.5 < 0.6 <= 0.8), renormalised to 0.625 / 0.375
    z = np.log([0.2, 0.5, 0.3])
    p = numpy_ref.sampler_probs(z, 1.0, 0, 0.6)
    assert np.allclose(p, [0.0, 0.625, 0.375])
    # exactly reaching top_p stops there (cumsum >= top_p)
    assert np.allclose(numpy_ref.sampler_probs(z, 1.0, 0, 0.5), [0, 1, 0])


def test_cold_temperature_is_greedy():
    z = np.array([0.1, 0.3, 0.2])
    assert np.allclose(numpy_ref.sampler_probs(z, 1e-4, 0, 1.0), [0, 1, 0])
