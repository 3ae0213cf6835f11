"""The margin/gradient oracle (oracle/vjp.py) pinned against things other than itself: the
hidden gradient equals a central finite difference of the margin through the head logits (so the
formula W[t] - softmax(competitors) @ W is checked, not retyped), the two-class closed forms,
torch's own logsumexp/argmax on the same logits, argmax ties going to the first index, and the
pre-projection gradient equal to the gradient of <post, o_proj(x)> by finite differences."""

import numpy as np
import torch

from oracle import vjp


def test_hidden_gradient_is_the_margin_derivative():
    rng = np.random.default_rng(0)
    vocab, dim = 37, 6
    weight = rng.standard_normal((vocab, dim))
    hidden = rng.standard_normal((1, dim))
    _, targets, _, _ = vjp.margin_stats(vjp.head_logits(hidden, weight))
    grad = vjp.hidden_gradient(vjp.head_logits(hidden, weight), targets, weight)[0]
    step = 1e-6
    for d in range(dim):
        plus, minus = hidden.copy(), hidden.copy()
        plus[0, d] += step
        minus[0, d] -= step
        fd = (vjp.margin_stats(vjp.head_logits(plus, weight), targets)[0][0]
              - vjp.margin_stats(vjp.head_logits(minus, weight), targets)[0][0]) / (2 * step)
        np.testing.assert_allclose(grad[d], fd, rtol=1e-6, atol=1e-8)


def test_two_class_closed_forms():
    weight = np.array([[1.0, 2.0], [-3.0, 0.5]])
    logits = np.array([[0.25, 4.0]])
    margins, targets, peak, total = vjp.margin_stats(logits)
    assert targets[0] == 1 and margins[0] == 4.0 - 0.25 and peak[0] == 0.25 and total[0] == 1.0
    np.testing.assert_array_equal(vjp.hidden_gradient(logits, targets, weight)[0],
                                  weight[1] - weight[0])


def test_margins_match_torch():
    rng = np.random.default_rng(1)
    logits = rng.standard_normal((3, 50)) * 4
    margins, targets, _, _ = vjp.margin_stats(logits)
    t = torch.from_numpy(logits)
    expect_targets = t.argmax(dim=-1)
    competitors = t.scatter(1, expect_targets[:, None], -torch.inf)
    expect = t.gather(1, expect_targets[:, None]).squeeze(1) - torch.logsumexp(competitors, -1)
    np.testing.assert_array_equal(targets, expect_targets.numpy())
    np.testing.assert_allclose(margins, expect.numpy(), rtol=1e-13)


def test_argmax_ties_take_the_first_index():
    logits = np.array([[1.0, 5.0, 5.0, 2.0]])
    assert vjp.margin_stats(logits)[1][0] == 1


def test_due_scales_rows_and_pre_gradient_is_a_derivative():
    rng = np.random.default_rng(2)
    logits = rng.standard_normal((2, 9))
    weight = rng.standard_normal((9, 4))
    targets = np.array([3, 0])
    full = vjp.hidden_gradient(logits, targets, weight)
    scaled = vjp.hidden_gradient(logits, targets, weight, np.array([1.0, 0.0]))
    np.testing.assert_array_equal(scaled[0], full[0])
    np.testing.assert_array_equal(scaled[1], 0.0)
    # o_proj: y = W_o x, objective <post, y>; its gradient in x is post @ W_o.
    post = rng.standard_normal(5)
    o_weight = rng.standard_normal((5, 7))
    gate = rng.standard_normal(7)
    x = rng.standard_normal(7)
    step = 1e-6
    for q in range(7):
        e = np.zeros(7)
        e[q] = step
        fd = (post @ (o_weight @ (x + e)) - post @ (o_weight @ (x - e))) / (2 * step)
        np.testing.assert_allclose(vjp.pre_gradient(post, o_weight)[q], fd, rtol=1e-7)
    np.testing.assert_allclose(vjp.pre_gradient(post, o_weight, gate),
                               vjp.pre_gradient(post, o_weight) * gate, rtol=1e-15)
