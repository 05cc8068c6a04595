"""GPU parity of the packed-batch causal GQA attention (dk_attn_fwd / dk_attn_bwd) with the
oracle, on the reference test's batches (solution/test_kernels.py:272-305: lens [1, 37, 64, 200]
and [512, 511, 3, 129], qkv ~ 0.8 N(0, 1), out to 3e-3, gradients to 3e-2 / 2e-2) and a config-like
batch of four 512-token sequences; the per-query-head dK/dV partials are checked head by head and
through the QKV epilogue backward that sums them (GIN = 6)."""

import numpy as np
import pytest

from tests.helpers import host, log

pytestmark = pytest.mark.gpu
NQ, NKV, HD = 12, 2, 128


@pytest.fixture(scope="module")
def torch():
    import torch as t
    return t


def _close(got, want, rtol, atol, what):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    bad = np.abs(got - want) > atol + rtol * np.abs(want)
    assert not bad.any(), f"{what}: {bad.sum()} of {bad.size} beyond tolerance, max err " \
                          f"{np.abs(got - want).max():.3g}"


@pytest.mark.parametrize("lens", [[1, 37, 64, 200], [512, 511, 3, 129], [512, 512, 512, 512]])
def test_varlen_causal_gqa_attention(torch, lens):
    from decentrik_prime_amd import k_attn, k_rope
    from oracle import attn, rope
    log(f"attention fwd+bwd, lens {lens}")
    n, g = sum(lens), NQ // NKV
    rng = np.random.default_rng(sum(lens))
    qkv = (rng.standard_normal((n, (NQ + 2 * NKV) * HD)) * 0.8).astype(np.float16)
    dout = rng.standard_normal((n, NQ * HD)).astype(np.float16)
    meta = k_attn.meta_for(lens, "cuda")
    tq = torch.from_numpy(qkv).cuda()
    out, lse = k_attn.attention_forward(tq, meta, NQ, NKV, HD)
    td = torch.from_numpy(dout).cuda()
    dq, dkp, dvp = k_attn.attention_backward(tq, out, lse, td, meta, NQ, NKV, HD)
    torch.cuda.synchronize()
    o_ref, lse_ref = attn.attention_fwd(qkv, lens, NQ, NKV, HD)
    _close(host(out), o_ref, 3e-3, 3e-3, "attention out")
    _close(host(lse), lse_ref, 1e-5, 2e-4, "lse (log2 domain)")
    dq_ref, dkp_ref, dvp_ref = attn.attention_bwd(qkv, dout, lens, NQ, NKV, HD, out=host(out))
    _close(host(dq), dq_ref, 3e-2, 2e-2, "dq")
    _close(host(dkp), dkp_ref, 3e-2, 2e-2, "dk per query head")
    _close(host(dvp), dvp_ref, 3e-2, 2e-2, "dv per query head")
    _close(host(dkp).reshape(n, NKV, g, HD).sum(2), dkp_ref.reshape(n, NKV, g, HD).sum(2), 3e-2,
           2e-2, "dk")
    _close(host(dvp).reshape(n, NKV, g, HD).sum(2), dvp_ref.reshape(n, NKV, g, HD).sum(2), 3e-2,
           2e-2, "dv")
    # the partials through the QKV epilogue backward (transposed rotation + GQA sums)
    pos = np.concatenate([np.arange(L) for L in lens]).astype(np.int32)
    cos, sin = rope.rope_tables(max(lens), HD)
    tqkv_grad = torch.empty(n, (NQ + 2 * NKV) * HD, dtype=torch.float16, device="cuda")
    k_rope.qkv_epilogue_backward(dq, dkp.view(n, NQ * HD), dvp.view(n, NQ * HD),
                                 torch.from_numpy(pos).cuda(), torch.from_numpy(cos).cuda(),
                                 torch.from_numpy(sin).cuda(), tqkv_grad, NQ, NKV, HD, g)
    torch.cuda.synchronize()
    want = rope.qkv_epilogue_bwd(dq_ref.astype(np.float32), dkp_ref.astype(np.float32),
                                 dvp_ref.astype(np.float32), pos, cos, sin, NQ, NKV, HD, g)
    _close(host(tqkv_grad), want, 3e-2, 3e-2, "dqkv through the QKV epilogue backward")


@pytest.mark.parametrize("nq,nkv", [(4, 4), (8, 2), (2, 1)])
def test_attention_head_configs(torch, nq, nkv):
    """Other head counts than Qwen2.5-1.5B's 12 / 2: plain multi-head (every query head its own
    K/V head), a group of 4 and a group of 2, forward and backward against the oracle."""
    from decentrik_prime_amd import k_attn
    from oracle import attn
    lens = [64, 200, 129]
    log(f"attention fwd+bwd, {nq} query / {nkv} KV heads, lens {lens}")
    n = sum(lens)
    rng = np.random.default_rng(7 * nq + nkv)
    qkv = (rng.standard_normal((n, (nq + 2 * nkv) * HD)) * 0.8).astype(np.float16)
    dout = rng.standard_normal((n, nq * HD)).astype(np.float16)
    meta = k_attn.meta_for(lens, "cuda")
    tq = torch.from_numpy(qkv).cuda()
    out, lse = k_attn.attention_forward(tq, meta, nq, nkv, HD)
    dq, dkp, dvp = k_attn.attention_backward(tq, out, lse, torch.from_numpy(dout).cuda(), meta,
                                             nq, nkv, HD)
    torch.cuda.synchronize()
    o_ref, lse_ref = attn.attention_fwd(qkv, lens, nq, nkv, HD)
    _close(host(out), o_ref, 3e-3, 3e-3, "attention out")
    _close(host(lse), lse_ref, 1e-5, 2e-4, "lse (log2 domain)")
    dq_ref, dkp_ref, dvp_ref = attn.attention_bwd(qkv, dout, lens, nq, nkv, HD, out=host(out))
    _close(host(dq), dq_ref, 3e-2, 2e-2, "dq")
    _close(host(dkp), dkp_ref, 3e-2, 2e-2, "dk per query head")
    _close(host(dvp), dvp_ref, 3e-2, 2e-2, "dv per query head")


def test_attention_argument_checks(torch):
    from decentrik_prime_amd import k_attn
    meta = k_attn.meta_for([5, 7], "cuda")
    qkv = torch.zeros(12, (NQ + 2 * NKV) * HD, dtype=torch.float16, device="cuda")
    with pytest.raises(ValueError):
        k_attn.attention_forward(qkv, meta, NQ, NKV, 64)             # head size
    with pytest.raises(ValueError):
        k_attn.attention_forward(qkv, meta, NQ, NKV, HD, block_m=64)  # fixed blocks
    with pytest.raises(ValueError):
        k_attn.attention_forward(qkv[:11], meta, NQ, NKV, HD)         # rows != tokens
    bad = k_attn.AttnMeta(meta.cu, meta.tab_fwd[:1], meta.tab_bwd, 1, meta.n_bwd, 12)
    with pytest.raises(ValueError):
        k_attn.attention_forward(qkv, bad, NQ, NKV, HD)               # table length


def test_attention_rescale_and_table_order(torch):
    """Scores that grow along the keys: every 64-key tile raises a row's maximum by about 16 in
    log2 units, far past the 2^8 rescale threshold, so the forward rescales its output on every
    tile, not only the first.  The backward gives the same bits with the sequence-major table as
    with the longest-first one, and the same bits again when repeated."""
    from decentrik_prime_amd import k_attn
    from oracle import attn
    lens = [300, 77, 512]
    log(f"attention rescale path and table order, lens {lens}")
    n = sum(lens)
    rng = np.random.default_rng(7)
    qkv = (rng.standard_normal((n, (NQ + 2 * NKV) * HD)) * 0.3).astype(np.float32)
    pos = np.concatenate([np.arange(L) for L in lens]).astype(np.float32)
    for kh in range(NKV):
        qkv[:, (NQ + kh) * HD] = 0.25 * pos        # key component 0 grows with the position
    for h in range(NQ):
        qkv[:, h * HD] = 8.0                        # score += 2 * key position
    qkv = qkv.astype(np.float16)
    dout = rng.standard_normal((n, NQ * HD)).astype(np.float16)
    meta = k_attn.meta_for(lens, "cuda")
    seq_major = k_attn.AttnMeta(meta.cu, meta.tab_fwd,
                                torch.tensor(k_attn.block_table(lens, k_attn.BWD_BLOCK),
                                             dtype=torch.int32, device="cuda"),
                                meta.n_fwd, meta.n_bwd, meta.n_tokens)
    assert not torch.equal(seq_major.tab_bwd, meta.tab_bwd)
    tq = torch.from_numpy(qkv).cuda()
    td = torch.from_numpy(dout).cuda()
    out, lse = k_attn.attention_forward(tq, meta, NQ, NKV, HD)
    g1 = k_attn.attention_backward(tq, out, lse, td, meta, NQ, NKV, HD)
    g2 = k_attn.attention_backward(tq, out, lse, td, seq_major, NQ, NKV, HD)
    g3 = k_attn.attention_backward(tq, out, lse, td, meta, NQ, NKV, HD)
    torch.cuda.synchronize()
    for a, b, c, nm in zip(g1, g2, g3, ("dq", "dk", "dv")):
        assert torch.equal(a, b), f"{nm}: table order changed the result"
        assert torch.equal(a, c), f"{nm}: repeat changed the result"
    o_ref, lse_ref = attn.attention_fwd(qkv, lens, NQ, NKV, HD)
    _close(host(out), o_ref, 3e-3, 3e-3, "attention out")
    _close(host(lse), lse_ref, 1e-5, 2e-3, "lse (log2 domain)")
    dq_ref, dkp_ref, dvp_ref = attn.attention_bwd(qkv, dout, lens, NQ, NKV, HD, out=host(out))
    _close(host(g1[0]), dq_ref, 3e-2, 2e-2, "dq")
    _close(host(g1[1]), dkp_ref, 3e-2, 2e-2, "dk per query head")
    _close(host(g1[2]), dvp_ref, 3e-2, 2e-2, "dv per query head")


def test_table_entries_without_rows_are_skipped(torch):
    """Block-table entries that name no rows: an empty sequence (cu[s] == cu[s + 1]) and blocks
    starting at or past their sequence's end.  The kernels skip such workgroups before any load,
    so the results are bit-identical to the run on the clean tables."""
    from decentrik_prime_amd import k_attn
    lens = [37, 0, 200]
    log(f"attention with table entries that name no rows, lens {lens}")
    n = sum(lens)
    rng = np.random.default_rng(99)
    qkv = torch.from_numpy((rng.standard_normal((n, (NQ + 2 * NKV) * HD)) * 0.8)
                           .astype(np.float16)).cuda()
    dout = torch.from_numpy(rng.standard_normal((n, NQ * HD)).astype(np.float16)).cuda()
    clean = k_attn.meta_for(lens, "cuda")
    extra = [1, 0, 0, 128, 2, 256, 1, 128]   # empty sequence; starts at or past the end
    i32 = dict(dtype=torch.int32, device="cuda")
    tf = torch.cat([clean.tab_fwd, torch.tensor(extra, **i32)])
    tb = torch.cat([torch.tensor(extra, **i32), clean.tab_bwd])
    dirty = k_attn.AttnMeta(clean.cu, tf, tb, tf.numel() // 2, tb.numel() // 2, n)
    results = []
    for meta in (clean, dirty):
        out, lse = k_attn.attention_forward(qkv, meta, NQ, NKV, HD)
        dq, dkp, dvp = k_attn.attention_backward(qkv, out, lse, dout, meta, NQ, NKV, HD)
        results.append([host(t) for t in (out, lse, dq, dkp, dvp)])
    torch.cuda.synchronize()
    for name, a, b in zip(("out", "lse", "dq", "dk", "dv"), *results):
        assert np.array_equal(a.view(np.uint8), b.view(np.uint8)), f"{name} changed"
