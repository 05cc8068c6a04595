"""Pins of the attention oracle (oracle/attn.py) against formulations that do not share its code:
torch float64 scaled_dot_product_attention with GQA by repeat_interleave and its autograd (the
check solution/test_kernels.py:272-305 runs), and closed forms (one-token sequences, uniform
attention when every query is zero)."""

import math

import numpy as np
import torch

from oracle import attn

NQ, NKV, HD = 12, 2, 128


def _qkv(lens, seed, scale=0.8):
    rng = np.random.default_rng(seed)
    return (rng.standard_normal((sum(lens), (NQ + 2 * NKV) * HD)) * scale).astype(np.float16)


def _torch_ref(qkv, lens, dout):
    n, g = qkv.shape[0], NQ // NKV
    t = torch.from_numpy(qkv.astype(np.float64))
    q = t[:, :NQ * HD].view(n, NQ, HD).clone().requires_grad_(True)
    k = t[:, NQ * HD:(NQ + NKV) * HD].view(n, NKV, HD).clone().requires_grad_(True)
    v = t[:, (NQ + NKV) * HD:].view(n, NKV, HD).clone().requires_grad_(True)
    outs, s0 = [], 0
    for L in lens:
        sl = slice(s0, s0 + L)
        qq = q[sl].transpose(0, 1)
        kk = k[sl].transpose(0, 1).repeat_interleave(g, 0)
        vv = v[sl].transpose(0, 1).repeat_interleave(g, 0)
        o = torch.nn.functional.scaled_dot_product_attention(qq[None], kk[None], vv[None],
                                                             is_causal=True, scale=1 / math.sqrt(HD))
        outs.append(o[0].transpose(0, 1))
        s0 += L
    ref = torch.cat(outs).reshape(n, NQ * HD)
    ref.backward(torch.from_numpy(dout.astype(np.float64)))
    return ref.detach().numpy(), q.grad.reshape(n, -1).numpy(), k.grad.numpy(), v.grad.numpy()


def test_oracle_matches_torch_sdpa_and_autograd():
    lens = [1, 37, 64, 70]
    qkv = _qkv(lens, 3)
    dout = np.random.default_rng(4).standard_normal((sum(lens), NQ * HD)).astype(np.float16)
    out, lse = attn.attention_fwd(qkv, lens, NQ, NKV, HD)
    ref, gq, gk, gv = _torch_ref(qkv, lens, dout)
    np.testing.assert_allclose(out, ref, rtol=1e-10, atol=1e-12)
    dq, dkp, dvp = attn.attention_bwd(qkv, dout, lens, NQ, NKV, HD)
    n, g = qkv.shape[0], NQ // NKV
    np.testing.assert_allclose(dq, gq, rtol=1e-9, atol=1e-11)
    np.testing.assert_allclose(dkp.reshape(n, NKV, g, HD).sum(2), gk, rtol=1e-9, atol=1e-11)
    np.testing.assert_allclose(dvp.reshape(n, NKV, g, HD).sum(2), gv, rtol=1e-9, atol=1e-11)
    # lse reproduces the output: out = sum_n 2^(s_n log2(e) - lse) v_n for token 40 (position 2 of
    # the sequence starting at token 38) and one head
    h, i = 5, 40
    qv = qkv.astype(np.float64)
    s = (qv[i, h * HD:(h + 1) * HD] @ qv[38:41, (NQ + h // g) * HD:(NQ + h // g + 1) * HD].T) / math.sqrt(HD)
    w = np.exp2(s * math.log2(math.e) - lse[h, i])
    vv = qv[38:41, (NQ + NKV + h // g) * HD:(NQ + NKV + h // g + 1) * HD]
    np.testing.assert_allclose(w @ vv, out[i, h * HD:(h + 1) * HD], rtol=1e-10, atol=1e-12)


def test_oracle_closed_forms():
    lens = [1, 5]
    qkv = _qkv(lens, 7).astype(np.float64)
    out, lse = attn.attention_fwd(qkv, lens, NQ, NKV, HD)
    g = NQ // NKV
    for h in (0, 7):
        kv = h // g
        q0 = qkv[0, h * HD:(h + 1) * HD]
        k0 = qkv[0, (NQ + kv) * HD:(NQ + kv + 1) * HD]
        v0 = qkv[0, (NQ + NKV + kv) * HD:(NQ + NKV + kv + 1) * HD]
        np.testing.assert_allclose(out[0, h * HD:(h + 1) * HD], v0, rtol=0, atol=1e-12)   # one key
        np.testing.assert_allclose(lse[h, 0], (q0 @ k0) / math.sqrt(HD) * math.log2(math.e), rtol=1e-12)
    # zero queries: uniform weights over the causal prefix of each sequence
    z = qkv.copy()
    z[:, :NQ * HD] = 0
    out, lse = attn.attention_fwd(z, lens, NQ, NKV, HD)
    vv = z[1:, (NQ + NKV + 1) * HD:(NQ + NKV + 2) * HD]
    for i in range(5):
        np.testing.assert_allclose(out[1 + i, 11 * HD:12 * HD], vv[:i + 1].mean(0), rtol=1e-12, atol=1e-12)
        np.testing.assert_allclose(lse[11, 1 + i], math.log2(i + 1), rtol=0, atol=1e-12)
    # no key of another sequence leaks in: the 1-token sequence's gradient sees only itself
    dout = np.ones((6, NQ * HD))
    dq, dkp, dvp = attn.attention_bwd(qkv, dout, lens, NQ, NKV, HD)
    np.testing.assert_allclose(dvp[0], dout[0], rtol=0, atol=1e-12)   # P = 1 on token 0
    np.testing.assert_allclose(dq[0], 0, atol=1e-12)                   # softmax of one key


def test_block_tables():
    """block_table follows solution/k_attn.py:185-191 (sequence-major, 128-row starts); the
    backward's table holds the same blocks, ordered by the rows from a block's start to its
    sequence's end, longest first, ties in block_table order."""
    from decentrik_prime_amd import k_attn
    lens = [1, 37, 300, 129, 512, 200]
    tab = k_attn.block_table(lens, 128)
    want = [(s, st) for s, n in enumerate(lens) for st in range(0, n, 128)]
    assert [(tab[i], tab[i + 1]) for i in range(0, len(tab), 2)] == want
    bt = k_attn.bwd_block_table(lens, 128)
    got = [(bt[i], bt[i + 1]) for i in range(0, len(bt), 2)]
    assert sorted(got) == sorted(want)
    rows = [lens[s] - st for s, st in got]
    assert rows == sorted(rows, reverse=True)
    # stable: equal walks keep block_table order
    for a, b in zip(got, got[1:]):
        if lens[a[0]] - a[1] == lens[b[0]] - b[1]:
            assert want.index(a) < want.index(b)
    # four sequences of 512: every sequence's first block, then every second block, ...
    bt = k_attn.bwd_block_table([512] * 4, 128)
    assert [(bt[i], bt[i + 1]) for i in range(0, len(bt), 2)] == \
        [(s, st) for st in (0, 128, 256, 384) for s in range(4)]
