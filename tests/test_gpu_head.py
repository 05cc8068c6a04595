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


@pytest.mark.parametrize("n,v,chunk,frac,gscale", [(300, 9984, 4096, 0.2, 4.0),
                                                   (64, 4096, 1024, 1.0, 1.0)])
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
