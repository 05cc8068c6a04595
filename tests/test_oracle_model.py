"""Pins of the whole-step reference (oracle/model.py) on a tiny configuration: its autograd LoRA
gradients against a central finite difference of the loss, and the structural zeros (with B = 0
no gradient reaches A; the dropout mask gates A's gradient column by column)."""

import numpy as np
import torch

from oracle import model

NQ, NKV, HD, DM, INTER, V = 4, 2, 16, 64, 48, 50


def _params(seed, zero_b=False):
    g = torch.Generator().manual_seed(seed)
    lens = [5, 7]
    n = sum(lens)
    r = 4

    def rn(*s, scale=1.0):
        return (torch.randn(*s, generator=g) * scale).double()
    cos_sin = torch.arange(8, dtype=torch.float64)[:, None] * (
        1e6 ** (-torch.arange(0, HD, 2, dtype=torch.float64) / HD))[None, :]
    emb2 = torch.cat((cos_sin, cos_sin), 1)
    layers = []
    for _ in range(2):
        layers.append(dict(
            wqkv=rn((NQ + 2 * NKV) * HD, DM, scale=0.2), bias=rn((NQ + 2 * NKV) * HD, scale=0.1),
            wo=rn(DM, NQ * HD, scale=0.2), wgu=rn(2 * INTER, DM, scale=0.2), wd=rn(DM, INTER, scale=0.2),
            w_in=1 + rn(DM, scale=0.1), w_post=1 + rn(DM, scale=0.1),
            Aq=rn(r, DM, scale=0.3), Bq=rn(NQ * HD, r, scale=0.0 if zero_b else 0.3),
            Av=rn(r, DM, scale=0.3), Bv=rn(NKV * HD, r, scale=0.0 if zero_b else 0.3),
            mq=(torch.rand(n, DM, generator=g) > 0.2).to(torch.uint8),
            mv=(torch.rand(n, DM, generator=g) > 0.2).to(torch.uint8)))
    tgt = torch.randint(0, V, (n,), generator=g)
    tgt[4] = -1
    tgt[11] = -1
    p = dict(x0=rn(n, DM), emb=rn(V, DM, scale=0.5), tgt=tgt,
             pos=torch.cat([torch.arange(L) for L in lens]), cos=emb2.cos(), sin=emb2.sin(),
             w_final=1 + rn(DM, scale=0.1), eps=1e-6, ks=1 / 0.8, s=2.0, layers=layers)
    return p, lens


def test_lora_gradients_match_finite_difference():
    p, lens = _params(0)
    loss, grads = model.qwen_step(p, lens, NQ, NKV, HD)
    for li, key, gi, idx in ((1, "Bq", 1, (3, 2)), (0, "Bv", 3, (5, 1)), (0, "Aq", 0, (1, 7)),
                             (1, "Av", 2, (2, 30))):
        h = 1e-6
        up, dn = _params(0)[0], _params(0)[0]
        up["layers"][li][key][idx] += h
        dn["layers"][li][key][idx] -= h
        fd = (model.qwen_step(up, lens, NQ, NKV, HD)[0] - model.qwen_step(dn, lens, NQ, NKV, HD)[0]) / (2 * h)
        got = float(grads[li][gi][idx])
        assert abs(got - fd) <= 1e-6 * max(1.0, abs(fd)), (li, key, got, fd)
    assert np.isfinite(loss) and loss > 0


def test_structural_zeros():
    p, lens = _params(1, zero_b=True)
    _, grads = model.qwen_step(p, lens, NQ, NKV, HD)
    for dAq, dBq, dAv, dBv in grads:
        assert torch.count_nonzero(dAq) == 0 and torch.count_nonzero(dAv) == 0   # B = 0 blocks A
        assert torch.count_nonzero(dBq) > 0 and torch.count_nonzero(dBv) > 0
