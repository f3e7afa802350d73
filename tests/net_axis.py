"""The net-axis problem of :func:`hawk_amd.examples.net_loss_for` — TEST
INFRASTRUCTURE: K small models in one launch (reference
tests/test_net_axis.py), with the numpy loop over the nets that gives each
net's loss and its gradient wrt its weights."""

from __future__ import annotations

import numpy as np

from hawk_amd import examples as E


def net_problem(k: int, s: int, seed: int, pick=None):
    """``(w, x, y, mask, loss, grad)`` for ``k`` nets of ``s`` samples: per-net
    weights ``w[k, 24]``, inputs ``x``, targets ``y`` and unit masks (widths 8,
    3, 5, 1, 6, repeated); ``loss`` and ``grad`` by a loop over the nets in
    ``pick`` (default: all of them), in that order."""
    H, P = E.NET_UNITS, E.NET_WEIGHTS
    g = np.random.default_rng(seed)
    w = g.normal(size=(k, P)) * 0.7
    x, y = g.normal(size=(k, s)), g.normal(size=(k, s))
    mask = (np.arange(H)[None, :] < np.resize([8, 3, 5, 1, 6], k)[:, None]).astype(np.float64)
    pick = np.arange(k) if pick is None else np.asarray(pick)
    loss, grad = np.zeros(len(pick)), np.zeros((len(pick), P))
    for j, i in enumerate(pick):
        a, b, c = w[i, 0::3], w[i, 1::3], w[i, 2::3]
        t = np.tanh(a[:, None] * x[i] + b[:, None])
        r = (mask[i] * c) @ t - y[i]
        loss[j] = r @ r
        lead = (2 * mask[i] * c)[:, None] * (1 - t * t) * r
        grad[j, 0::3] = (lead * x[i]).sum(axis=1)
        grad[j, 1::3] = lead.sum(axis=1)
        grad[j, 2::3] = ((2 * mask[i])[:, None] * t * r).sum(axis=1)
    return w, x, y, mask, loss, grad
