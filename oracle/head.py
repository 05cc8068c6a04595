"""CPU restatement of the LM head's loss, statistics and hidden-state gradient.  TEST
INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg,
never by the product path.

Per token row with hidden y and target t (-1 = none), over the whole vocabulary, as
solution/k_head.py:1-33 defines them (logits are the fp16 GEMM output, everything after in exact
arithmetic here):
    x = fp16(y E^T);  lse = log sum_v e^(x_v);  p = e^(x - lse)
    loss = lse - x_t (0 without a target);  entropy = -sum_v p_v log p_v;  hit = [argmax x == t]
    (first index on ties);  dY = grad_scale (sum_v p_v E_v - E_t) for rows with a target, else 0
`chunked_state` restates the kernel's running merge over vocabulary chunks (solution/k_head.py:
50-123) so that its algebra can be checked against the whole-row form.
"""

import numpy as np

F16 = np.float16


def logits16(y16, emb16):
    """fp16(y E^T) with an exact (float64) accumulation before the single rounding."""
    return (np.asarray(y16, np.float64) @ np.asarray(emb16, np.float64).T).astype(F16)


def head(y16, emb16, tgt, grad_scale, x16=None):
    """(stats [N, 4] = (loss, entropy, hit, lse), dY [N, D] float64) in token order; x16 are the
    fp16 logits to use (default: logits16(y16, emb16))."""
    x = np.asarray(logits16(y16, emb16) if x16 is None else x16, np.float64)
    e = np.asarray(emb16, np.float64)
    tgt = np.asarray(tgt)
    n = x.shape[0]
    mx = x.max(1, keepdims=True)
    z = np.exp(x - mx)
    s = z.sum(1, keepdims=True)
    lse = (mx + np.log(s))[:, 0]
    p = z / s
    ent = -(p * (x - lse[:, None])).sum(1)
    valid = tgt >= 0
    xt = np.where(valid, x[np.arange(n), np.where(valid, tgt, 0)], 0.0)
    stats = np.stack([np.where(valid, lse - xt, 0.0), ent,
                      (valid & (x.argmax(1) == tgt)).astype(np.float64), lse], 1)
    dy = p @ e
    dy[valid] -= e[tgt[valid]]
    dy[~valid] = 0.0
    return stats, grad_scale * dy


def chunked_state(x16, tgt, chunk):
    """The running (m, s, t, argmax, x_t) after merging every chunk of each row, in float64, with
    the kernel's merge rules; returns (lse, entropy, argmax, x_t)."""
    x = np.asarray(x16, np.float64)
    n, v = x.shape
    m = np.full(n, -np.inf)
    s = np.zeros(n)
    t = np.zeros(n)
    am = np.zeros(n)
    xt = np.zeros(n)
    tgt = np.asarray(tgt)
    for v0 in range(0, v, chunk):
        c = x[:, v0:v0 + chunk]
        mc = c.max(1)
        ac = c.argmax(1)
        z = c - mc[:, None]
        sc = np.exp(z).sum(1)
        tc = (np.exp(z) * z).sum(1)
        m_new = np.maximum(m, mc)
        a_old = np.exp(m - m_new)
        a_new = np.exp(mc - m_new)
        with np.errstate(invalid="ignore"):
            t_old = np.where(s > 0, a_old * (t + s * (m - m_new)), 0.0)
        t = t_old + a_new * (tc + sc * (mc - m_new))
        s = s * a_old + sc * a_new
        am = np.where(mc > m, ac + v0, am)
        loc = tgt - v0
        inside = (loc >= 0) & (loc < c.shape[1])
        xt = np.where(inside, c[np.arange(n), np.clip(loc, 0, c.shape[1] - 1)], xt)
        m = m_new
    return m + np.log(s), np.log(s) - t / s, am, xt
