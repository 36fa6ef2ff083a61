"""The router oracle's selection rules on hand-made rows (CPU)."""

import numpy as np

from oracle import route_oracle as R


def test_ties_go_to_the_lower_expert():
    logits = np.zeros((1, 6), np.float32)
    ids, w, _ = R.route(logits, 3, sigmoid=True, bias=np.zeros(6, np.float32))
    assert ids.tolist() == [[0, 1, 2]]
    assert np.allclose(w, 1.0 / 3)


def test_bias_selects_but_does_not_weigh():
    logits = np.array([[0.0, 1.0, 2.0, 3.0]], np.float32)
    bias = np.array([10.0, 0.0, 0.0, 0.0], np.float32)
    ids, w, _ = R.route(logits, 2, sigmoid=True, bias=bias, renormalize=False, scale=2.0)
    assert ids.tolist() == [[0, 3]]
    s = 0.5 * np.tanh(0.5 * np.array([0.0, 3.0], np.float32)) + 0.5
    assert np.allclose(w[0], 2.0 * s)


def test_renormalized_weights_sum_to_scale():
    rng = np.random.default_rng(0)
    logits = rng.standard_normal((20, 64)).astype(np.float32)
    ids, w, _ = R.route(logits, 8, sigmoid=True, bias=np.zeros(64, np.float32), scale=2.5)
    assert np.allclose(w.sum(1), 2.5, rtol=1e-6)


def test_softmax_order_is_the_logit_order():
    rng = np.random.default_rng(1)
    logits = rng.standard_normal((10, 32)).astype(np.float32)
    ids, w, _ = R.route(logits, 4, sigmoid=False, renormalize=False)
    want = np.argsort(-logits, axis=1, kind="stable")[:, :4]
    assert np.array_equal(ids, want)
    p = np.exp(logits - logits.max(1, keepdims=True))
    p /= p.sum(1, keepdims=True)
    assert np.allclose(w, np.take_along_axis(p, want, 1), rtol=1e-5)
