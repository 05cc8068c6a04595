"""GPU parity of the vocabulary-chunked LM head (dk_head_chunk / dk_head_finalize between the
fp16-weight GEMMs) with the oracle: loss, entropy, argmax hit and lse per row, and d(hidden), on a
ragged last chunk, rows without a target, and a batch with no targets at all."""

import numpy as np
import pytest

from tests.helpers import assert_close, host, log

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch():
    import torch as t
    return t


def _case(n, v, d, seed, frac_no_target):
    rng = np.random.default_rng(seed)
    y = rng.standard_normal((n, d)).astype(np.float16)
    emb = (rng.standard_normal((v, d)) * 0.05).astype(np.float16)
    tgt = rng.integers(0, v, n).astype(np.int32)
    tgt[rng.random(n) < frac_no_target] = -1
    return y, emb, tgt


# chunk widths from 1024 to 65,536 columns (the full-vocabulary test below: 32,768 and a last
# chunk of 20,864), with a ragged last chunk in each case but the second
@pytest.mark.parametrize("n,v,chunk,frac,gscale", [(300, 9984, 4096, 0.2, 4.0),
                                                   (64, 4096, 1024, 1.0, 1.0),
                                                   (64, 20480, 16384, 0.5, 1.0),
                                                   (48, 70016, 65536, 0.8, 2.0)])
def test_streamed_head(torch, n, v, chunk, frac, gscale):
    from decentrik_prime_amd import k_head
    from oracle import head
    d = 1536
    log(f"LM head N={n} V={v} chunk={chunk}")
    y, emb, tgt = _case(n, v, d, 11 + n, frac)
    perm = np.concatenate([np.nonzero(tgt >= 0)[0], np.nonzero(tgt < 0)[0]]).astype(np.int32)
    tgt_sorted = tgt[perm]
    n_lab = int((tgt >= 0).sum())
    temb = torch.from_numpy(emb).cuda()
    src = k_head.ResidentEmbedding(temb, chunk)
    tps = torch.from_numpy(tgt_sorted).cuda()
    et = temb.index_select(0, tps[:n_lab].long()).contiguous()
    loss, stats, dy = k_head.streamed_head(torch.from_numpy(y).cuda(), src, tps,
                                           torch.from_numpy(perm).cuda(), n_lab, et, gscale)
    torch.cuda.synchronize()
    ref_stats, ref_dy = head.head(y, emb, tgt, gscale)
    got = np.empty_like(ref_stats)
    got[perm] = host(stats)                       # sorted order -> token order
    assert_close(got[:, 0], ref_stats[:, 0], 2e-3, 2e-3, "loss")
    assert_close(got[:, 1], ref_stats[:, 1], 2e-3, 2e-3, "entropy")
    assert_close(got[:, 3], ref_stats[:, 3], 1e-3, 2e-3, "lse")
    # argmax hits agree wherever the top two logits are not within a GEMM rounding of each other
    x = np.sort(head.logits16(y, emb).astype(np.float64), 1)
    clear = (x[:, -1] - x[:, -2]) > 2e-2
    assert np.array_equal(got[clear, 2], ref_stats[clear, 2]), "argmax hits"
    assert abs(float(loss) - ref_stats[:, 0].sum()) <= 2e-3 * max(1.0, abs(ref_stats[:, 0].sum()))
    s = float(np.abs(ref_dy).max()) or 1.0
    assert_close(host(dy).astype(np.float64) / s, ref_dy / s, 1e-2, 2e-2, "d(hidden)")
    assert not np.any(host(dy)[tgt < 0]), "rows without a target get a zero gradient"


def test_streamed_head_full_vocabulary(torch):
    """Qwen2.5's 151,936-token vocabulary at the default chunk (four full chunks of 32,768 and a
    partial last chunk of 20,864), a few dozen rows: targets in the last partial chunk and on
    chunk boundaries, and argmax ties planted across chunk boundaries and inside the last chunk
    (two identical embedding rows that are a row's clear maximum: the first index is the argmax,
    so the hit is 1 only when the target is the first of the pair)."""
    from decentrik_prime_amd import k_head
    from oracle import head
    n, v, d = 48, 151936, 1536
    chunk = k_head.CHUNK
    log(f"LM head N={n} V={v} chunk={chunk}")
    y, emb, tgt = _case(n, v, d, 123, 0.1)
    rng = np.random.default_rng(124)
    last0 = (v // chunk) * chunk                       # first column of the partial last chunk
    tgt[8:32] = rng.integers(last0, v, 24)             # targets in the last partial chunk
    tgt[32:36] = [chunk - 1, chunk, 2 * chunk - 1, last0]   # targets on chunk boundaries
    # (row, first column of an identical pair or None for a single planted maximum, target)
    planted = [(0, chunk - 1, chunk - 1), (1, 2 * chunk - 1, 2 * chunk), (2, v - 2, v - 1),
               (3, None, last0), (4, 3 * chunk - 1, 3 * chunk - 1), (5, 3 * chunk + 7, 3 * chunk + 8)]
    cols = [c for _, c, t in planted for c in ((t,) if c is None else (c, c + 1))]
    assert len(set(cols)) == len(cols), "planted columns overlap"
    for row, c, t in planted:
        e = (y[row].astype(np.float32) * 0.01).astype(np.float16)
        if c is None:
            emb[t] = e
        else:
            emb[c] = emb[c + 1] = e
        tgt[row] = t
    perm = np.concatenate([np.nonzero(tgt >= 0)[0], np.nonzero(tgt < 0)[0]]).astype(np.int32)
    tgt_sorted = tgt[perm]
    n_lab = int((tgt >= 0).sum())
    temb = torch.from_numpy(emb).cuda()
    src = k_head.ResidentEmbedding(temb)
    assert src.chunk == chunk and src.n_chunks == 5
    tps = torch.from_numpy(tgt_sorted).cuda()
    et = temb.index_select(0, tps[:n_lab].long()).contiguous()
    loss, stats, dy = k_head.streamed_head(torch.from_numpy(y).cuda(), src, tps,
                                           torch.from_numpy(perm).cuda(), n_lab, et, 2.0)
    torch.cuda.synchronize()
    ref_stats, ref_dy = head.head(y, emb, tgt, 2.0)
    got = np.empty_like(ref_stats)
    got[perm] = host(stats)
    assert_close(got[:, 0], ref_stats[:, 0], 2e-3, 2e-3, "loss")
    assert_close(got[:, 1], ref_stats[:, 1], 2e-3, 2e-3, "entropy")
    assert_close(got[:, 3], ref_stats[:, 3], 1e-3, 2e-3, "lse")
    for row, c, t in planted:
        want = 1.0 if (c is None or t == c) else 0.0
        assert got[row, 2] == want == ref_stats[row, 2], f"row {row}: argmax hit at target {t}"
    x = np.sort(head.logits16(y, emb).astype(np.float64), 1)
    clear = (x[:, -1] - x[:, -2]) > 2e-2
    assert np.array_equal(got[clear, 2], ref_stats[clear, 2]), "argmax hits"
    assert abs(float(loss) - ref_stats[:, 0].sum()) <= 2e-3 * max(1.0, abs(ref_stats[:, 0].sum()))
    s = float(np.abs(ref_dy).max()) or 1.0
    assert_close(host(dy).astype(np.float64) / s, ref_dy / s, 1e-2, 2e-2, "d(hidden)")
    assert not np.any(host(dy)[tgt < 0]), "rows without a target get a zero gradient"
