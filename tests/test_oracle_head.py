"""Pins of the LM-head oracle (oracle/head.py) against torch float64 (cross_entropy, its autograd
gradient with respect to the hidden states, Categorical entropy, logsumexp, argmax) and of the
chunked running-state merge against the whole-row form, including ragged last chunks and chunks
where the row maximum moves."""

import numpy as np
import torch

from oracle import head


def _inputs(n=40, v=1000, d=64, seed=0):
    rng = np.random.default_rng(seed)
    y = rng.standard_normal((n, d)).astype(np.float16)
    emb = (rng.standard_normal((v, d)) * 0.3).astype(np.float16)
    tgt = rng.integers(0, v, n).astype(np.int32)
    tgt[::7] = -1
    return y, emb, tgt


def test_head_matches_torch_cross_entropy_and_autograd():
    y, emb, tgt = _inputs()
    g = 0.25
    stats, dy = head.head(y, emb, tgt, g)
    x = torch.from_numpy(head.logits16(y, emb).astype(np.float64))
    t = torch.from_numpy(tgt.astype(np.int64))
    valid = t >= 0
    ce = torch.nn.functional.cross_entropy(x, t.clamp(min=0), reduction="none") * valid
    np.testing.assert_allclose(stats[:, 0], ce.numpy(), rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(stats[:, 1], torch.distributions.Categorical(logits=x).entropy().numpy(),
                               rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(stats[:, 3], torch.logsumexp(x, 1).numpy(), rtol=1e-12)
    np.testing.assert_array_equal(stats[:, 2], ((x.argmax(1) == t) & valid).numpy().astype(float))
    # d(g * sum CE)/dy through the fp16-valued logits x = y E^T (exact products here)
    yt = torch.from_numpy(y.astype(np.float64)).requires_grad_(True)
    xe = yt @ torch.from_numpy(emb.astype(np.float64)).T
    loss = (torch.nn.functional.cross_entropy(xe, t.clamp(min=0), reduction="none") * valid).sum() * g
    loss.backward()
    # the oracle's softmax uses the fp16-rounded logits: agreement to fp16 logit rounding
    np.testing.assert_allclose(dy, yt.grad.numpy(), rtol=0, atol=2e-3 * g)
    assert np.all(dy[~valid.numpy()] == 0)


def test_chunked_merge_equals_whole_row():
    y, emb, tgt = _inputs(n=30, v=1000, seed=3)
    x = head.logits16(y, emb)
    # make the maximum of some rows sit in a late chunk, and a tie across chunks
    x[1, 900] = 30.0
    x[2, 10] = 25.0
    x[2, 700] = 25.0
    stats, _ = head.head(y, emb, tgt, 1.0, x16=x)
    for chunk in (64, 128, 384, 1000):
        lse, ent, am, xt = head.chunked_state(x, tgt, chunk)
        np.testing.assert_allclose(lse, stats[:, 3], rtol=1e-12)
        np.testing.assert_allclose(ent, stats[:, 1], rtol=1e-9, atol=1e-11)
        np.testing.assert_array_equal(am, np.asarray(x, np.float64).argmax(1))   # first index on ties
        valid = tgt >= 0
        np.testing.assert_array_equal(xt[valid], np.asarray(x, np.float64)[np.arange(30), tgt][valid])
    assert head.chunked_state(x, tgt, 128)[2][2] == 10
