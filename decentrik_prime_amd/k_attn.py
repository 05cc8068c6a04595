"""Variable-length causal GQA attention of the padding-free packed batch, forward and backward.

Drop-in for the attention kernels of the reference's solution/k_attn.py (``block_table``,
``AttnMeta``, ``attention_forward``, ``attention_backward``, ``warmup_specs``: same names,
arguments and results), running the gfx950 kernels ``dk_attn_fwd`` / ``dk_attn_bwd`` of
libdk.so.  The packed tokens' queries, keys and values live in one row of the fused QKV buffer
[N, (nq + 2 nkv) hd] fp16; blocks of 128 rows (queries in the forward and dQ, keys in dK/dV) never
straddle two sequences, so the mask is ``key <= query`` inside a sequence.

forward   online softmax in the exp2 domain (scores scaled by log2(e) / sqrt(hd)), fp32 running
          max and sum, P rounded to fp16 for the P V product; out fp16 [N, nq hd], lse fp32
          [nq, N] = m + log2(l)
backward  delta = rowsum(O dO); dQ fp32 [N, nq hd]; dK, dV fp32 per query head [N, nq hd], which
          the QKV epilogue backward sums over each group of nq / nkv heads (gin)

The reference's block sizes are parameters of its Triton kernels; here the blocks are fixed by
the kernels (128 rows per workgroup, tiles of 64), and ``block_table`` must be built for
FWD_BLOCK_M and BWD_BLOCK.
"""

import torch

from . import _lib

FWD_BLOCK_M, FWD_BLOCK_N = 128, 64
BWD_BLOCK = 128
ATTN_WARPS = 4
HEAD_DIM = 128


def block_table(lens, block):
    """Flat [seq, start, seq, start, ...] for every block of `block` rows of every sequence
    (solution/k_attn.py:185-191)."""
    tab = []
    for s, n in enumerate(lens):
        for start in range(0, n, block):
            tab += (s, start)
    return tab


def bwd_block_table(lens, block):
    """``block_table``'s blocks ordered by the rows from a block's start to its sequence's end,
    longest first (stable).  The backward launch runs its dK/dV blocks in table order and its dQ
    blocks in reverse order, dealt to the XCDs round-robin, so this order starts the longest walks
    first and gives every XCD a balanced share; any order gives the same results."""
    tab = block_table(lens, block)
    pairs = [(tab[i], tab[i + 1]) for i in range(0, len(tab), 2)]
    pairs.sort(key=lambda p: -(int(lens[p[0]]) - p[1]))
    return [v for p in pairs for v in p]


class AttnMeta:
    """Per-batch tables (device int32 tensors) for the attention kernels
    (solution/k_attn.py:194-199)."""

    def __init__(self, cu, tab_fwd, tab_bwd, n_fwd, n_bwd, n_tokens):
        self.cu, self.tab_fwd, self.tab_bwd = cu, tab_fwd, tab_bwd
        self.n_fwd, self.n_bwd, self.n_tokens = n_fwd, n_bwd, n_tokens


def meta_for(lens, device):
    """AttnMeta of a packed batch with sequence lengths `lens` (as solution/test_kernels.py:261-269
    builds it)."""
    cu = [0]
    for n in lens:
        cu.append(cu[-1] + int(n))
    tf, tb = block_table(lens, FWD_BLOCK_M), bwd_block_table(lens, BWD_BLOCK)
    i32 = dict(dtype=torch.int32, device=device)
    return AttnMeta(torch.tensor(cu, **i32), torch.tensor(tf, **i32), torch.tensor(tb, **i32),
                    len(tf) // 2, len(tb) // 2, cu[-1])


def _t(t, dtypes, what, shape=None):
    if t.dtype not in dtypes or not t.is_cuda or not t.is_contiguous():
        raise ValueError(f"{what} must be a contiguous CUDA tensor of {dtypes}")
    if shape is not None and tuple(t.shape) != tuple(shape):
        raise ValueError(f"{what} has shape {tuple(t.shape)}, expected {tuple(shape)}")
    return t


def _check(qkv, meta, nq, nkv, hd, tab, n_blocks):
    if hd != HEAD_DIM or nq % nkv:
        raise ValueError(f"head size {HEAD_DIM} and nq a multiple of nkv (got {hd}, {nq}, {nkv})")
    n = meta.n_tokens
    _t(qkv, (torch.float16,), "qkv", (n, (nq + 2 * nkv) * hd))
    _t(meta.cu, (torch.int32,), "meta.cu")
    _t(tab, (torch.int32,), "block table", (2 * n_blocks,))
    if meta.cu.dim() != 1 or meta.cu.numel() < 2:
        raise ValueError("meta.cu must hold at least one sequence")


def attention_forward(qkv, meta, nq, nkv, hd, block_m=FWD_BLOCK_M, block_n=FWD_BLOCK_N,
                      warps=ATTN_WARPS):
    """(out [N, nq hd] fp16, lse [nq, N] fp32).  meta.tab_fwd must be the block table for
    FWD_BLOCK_M (solution/k_attn.py:202-212)."""
    if (block_m, block_n) != (FWD_BLOCK_M, FWD_BLOCK_N):
        raise ValueError(f"the forward kernel's blocks are {FWD_BLOCK_M} x {FWD_BLOCK_N}")
    _check(qkv, meta, nq, nkv, hd, meta.tab_fwd, meta.n_fwd)
    n = meta.n_tokens
    out = torch.empty((n, nq * hd), dtype=torch.float16, device=qkv.device)
    lse = torch.empty((nq, n), dtype=torch.float32, device=qkv.device)
    rc = _lib.lib().dk_attn_fwd(_lib.ptr(qkv), _lib.ptr(meta.cu), meta.cu.numel() - 1,
                                _lib.ptr(meta.tab_fwd), meta.n_fwd, n, nq, nkv, hd, _lib.ptr(out),
                                _lib.ptr(lse), _lib.stream_handle(qkv.device))
    _lib.check(rc, "dk_attn_fwd")
    return out, lse


def attention_backward(qkv, out, lse, dout, meta, nq, nkv, hd, block=BWD_BLOCK, warps=ATTN_WARPS):
    """fp32 dq [N, nq hd] and per-query-head dk, dv partials [N, nq hd].  meta.tab_bwd must be
    the block table for BWD_BLOCK (solution/k_attn.py:215-245)."""
    if block != BWD_BLOCK:
        raise ValueError(f"the backward kernels' block is {BWD_BLOCK}")
    _check(qkv, meta, nq, nkv, hd, meta.tab_bwd, meta.n_bwd)
    n = meta.n_tokens
    _t(out, (torch.float16,), "out", (n, nq * hd))
    _t(dout, (torch.float16,), "dout", (n, nq * hd))
    _t(lse, (torch.float32,), "lse", (nq, n))
    dev = qkv.device
    delta = torch.empty((nq, n), dtype=torch.float32, device=dev)
    dq = torch.empty((n, nq * hd), dtype=torch.float32, device=dev)
    dkp = torch.empty((n, nq * hd), dtype=torch.float32, device=dev)
    dvp = torch.empty((n, nq * hd), dtype=torch.float32, device=dev)
    rc = _lib.lib().dk_attn_bwd(_lib.ptr(qkv), _lib.ptr(out), _lib.ptr(lse), _lib.ptr(dout),
                                _lib.ptr(meta.cu), meta.cu.numel() - 1, _lib.ptr(meta.tab_bwd),
                                meta.n_bwd, n, nq, nkv, hd, _lib.ptr(delta), _lib.ptr(dq),
                                _lib.ptr(dkp), _lib.ptr(dvp), _lib.stream_handle(dev))
    _lib.check(rc, "dk_attn_bwd")
    return dq, dkp, dvp


def warmup_specs(nq, nkv, hd):
    """Nothing to warm up: the kernels are compiled ahead of time into libdk.so."""
    return []
