"""CPU restatement of the packed-batch causal GQA attention, forward and backward.  TEST
INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg,
never by the product path.

qkv [N, (nq + 2 nkv) hd] holds each token's query heads, key heads, value heads; the sequences of
lengths `lens` are packed one after another; query head h attends to key / value head
h // (nq // nkv) of the earlier-or-same tokens of its own sequence (solution/k_attn.py:1-26).
With sm = 1 / sqrt(hd), per sequence and head, in float64:
    S = sm q k^T (causal),  P = softmax(S),  out = P v,  lse = log2(sum_n exp(S_n))
(the exp2-domain statistic m + log2(l) of solution/k_attn.py:72-80)
backward (solution/k_attn.py:84-182):
    delta = rowsum(out * dout),  dP = dout v^T,  dS = P * (dP - delta)
    dq = sm dS k,  dk_h = sm dS^T q,  dv_h = P^T dout     (dk_h, dv_h per query head h)
"""

import numpy as np


def _split(qkv, nq, nkv, hd):
    x = np.asarray(qkv, np.float64)
    n = x.shape[0]
    q = x[:, :nq * hd].reshape(n, nq, hd)
    k = x[:, nq * hd:(nq + nkv) * hd].reshape(n, nkv, hd)
    v = x[:, (nq + nkv) * hd:].reshape(n, nkv, hd)
    return q, k, v


def _probs(q, k, sm):
    """P and the natural-log logsumexp of one sequence and head (causal)."""
    s = sm * (q @ k.T)
    n = s.shape[0]
    s = np.where(np.tril(np.ones((n, n), bool)), s, -np.inf)
    mx = s.max(1, keepdims=True)
    e = np.exp(s - mx)
    z = e.sum(1, keepdims=True)
    return e / z, (mx + np.log(z))[:, 0]


def attention_fwd(qkv, lens, nq, nkv, hd):
    """(out [N, nq hd] float64, lse [nq, N] float64, exp2 domain)."""
    q, k, v = _split(qkv, nq, nkv, hd)
    n, g, sm = q.shape[0], nq // nkv, 1.0 / np.sqrt(hd)
    out = np.zeros((n, nq, hd))
    lse = np.zeros((nq, n))
    s0 = 0
    for L in lens:
        sl = slice(s0, s0 + L)
        for h in range(nq):
            p, lz = _probs(q[sl, h], k[sl, h // g], sm)
            out[sl, h] = p @ v[sl, h // g]
            lse[h, sl] = lz / np.log(2.0)
        s0 += L
    return out.reshape(n, nq * hd), lse


def attention_bwd(qkv, dout, lens, nq, nkv, hd, out=None):
    """(dq, dkp, dvp) float64, each [N, nq hd]; dkp / dvp per query head.  delta uses `out` when
    given (the saved forward output, as the reference's backward does), else the exact output."""
    q, k, v = _split(qkv, nq, nkv, hd)
    n, g, sm = q.shape[0], nq // nkv, 1.0 / np.sqrt(hd)
    do = np.asarray(dout, np.float64).reshape(n, nq, hd)
    o_saved = None if out is None else np.asarray(out, np.float64).reshape(n, nq, hd)
    dq, dkp, dvp = (np.zeros((n, nq, hd)) for _ in range(3))
    s0 = 0
    for L in lens:
        sl = slice(s0, s0 + L)
        for h in range(nq):
            kk, vv = k[sl, h // g], v[sl, h // g]
            p, _ = _probs(q[sl, h], kk, sm)
            o = p @ vv if o_saved is None else o_saved[sl, h]
            delta = (o * do[sl, h]).sum(1, keepdims=True)
            ds = p * (do[sl, h] @ vv.T - delta)
            dq[sl, h] = sm * (ds @ kk)
            dkp[sl, h] = sm * (ds.T @ q[sl, h])
            dvp[sl, h] = p.T @ do[sl, h]
        s0 += L
    return dq.reshape(n, -1), dkp.reshape(n, -1), dvp.reshape(n, -1)
