"""LM head over the vocabulary without full logits: loss, entropy, argmax accuracy, lse and
d(hidden) in one pass over vocabulary chunks.

Drop-in for the streamed head of the reference's solution/k_head.py (``ResidentEmbedding``,
``streamed_head``, ``STATE_W``: same names, arguments and results).  Per chunk of the embedding:
    logits_c = Y E_c^T          dk_h16_linear_fwd_lora (fp16 out, the 256-tile GEMM)
    dk_head_chunk               running (max, sum, entropy sum, argmax, target logit) per row;
                                P = p_scale e^(x - m) written in place for rows with a target
    acc += P E_c                dk_h16_linear_bwd_dx_lora with fp32 accumulation
then dk_head_finalize gives (loss, entropy, hit, lse) per row and d(hidden) in token order.  Only
[N, chunk] logits exist at a time.  The embedding stays resident in HBM (288 GB per GPU holds it
many times over): the reference's host-memory EmbeddingStream is not needed on this GPU.
"""

import torch

from . import _lib
from .w4linear import _h16_workspace

STATE_W = 8          # per-row running state: m, s, t, argmax, x_target, (pad)
CHUNK = 32768        # vocabulary rows per chunk (a multiple of 64): at 2048 tokens a 134 MB
                     # logits buffer; measured 2.81 / 2.49 / 2.45 ms per full-vocabulary call at
                     # 8192 / 16384 / 32768 (fewer split-K reduces and launches per call)


class ResidentEmbedding:
    """The embedding on the GPU: chunk c is a view of it (solution/k_head.py:180-199)."""

    def __init__(self, emb, chunk=CHUNK):
        if emb.dtype != torch.float16 or not emb.is_cuda or not emb.is_contiguous() or emb.dim() != 2:
            raise ValueError("the embedding must be a contiguous CUDA fp16 [vocab, hidden] tensor")
        if chunk % 64 or emb.shape[0] % 64 or emb.shape[1] % 64:
            raise ValueError("chunk, vocabulary and hidden size must be multiples of 64")
        self.emb, self.chunk = emb, int(chunk)
        self.vocab = emb.shape[0]
        self.n_chunks = -(-self.vocab // self.chunk)

    def start(self):
        pass

    def get(self, c):
        v0 = c * self.chunk
        return self.emb[v0:min(v0 + self.chunk, self.vocab)]

    def release(self, c):
        pass

    def rows(self, idx_dev, idx_cpu=None):
        return self.emb.index_select(0, idx_dev)


def _logits(ys, e_c, out):
    """out [N, vc] = fp16(ys e_c^T).  A chunk whose size is not a multiple of 256 (the
    vocabulary's last) runs as two GEMMs, the columns up to the last multiple of 256 on the
    256 x 256-tile kernel and the rest on their own: one GEMM over all of them would take the
    smaller tiles throughout (measured on MI355X, 2048 x 20,864 x 1536: 280 us)."""
    n, d = ys.shape
    vc = e_c.shape[0]
    split = vc - vc % 256 if vc > 256 else vc
    for c0, c1 in ((0, split), (split, vc)):
        if c1 == c0:
            continue
        ws, nbytes = _h16_workspace(n, c1 - c0, d, _lib.DK_OP_LINEAR_FWD, ys.device)
        rc = _lib.lib().dk_h16_linear_fwd_lora(_lib.ptr(ys), d, n, _lib.ptr(e_c[c0:]), c1 - c0, d,
                                               None, None, 0, 0, _lib.ptr(out[:, c0:]), vc,
                                               _lib.ptr(ws), nbytes, None,
                                               _lib.stream_handle(ys.device))
        _lib.check(rc, "dk_h16_linear_fwd_lora (logits)")


def _accumulate(acc, p16, e_c):
    """acc [n_lab, d] (fp32) += p16 [n_lab, vc] e_c [vc, d], fp16 inputs, fp32 accumulation in place
    (solution/k_head.py:164-175)."""
    m, vc = p16.shape
    d = e_c.shape[1]
    ws, nbytes = _h16_workspace(m, vc, d, _lib.DK_OP_LINEAR_BWD_DX, acc.device)
    rc = _lib.lib().dk_h16_linear_bwd_dx_lora(_lib.ptr(p16), p16.stride(0), m, _lib.ptr(e_c), vc, d,
                                              None, 0, 0, _lib.ptr(acc), d, _lib.DK_OUT_F32_ACCUM,
                                              _lib.ptr(ws), nbytes, None,
                                              _lib.stream_handle(acc.device))
    _lib.check(rc, "dk_h16_linear_bwd_dx_lora (head accumulate)")


def streamed_head(yf, source, tgt_sorted, perm, n_lab, e_target, grad_scale, dummy32=None):
    """LM head of the packed batch (solution/k_head.py:277-311).

    yf [N, D] fp16 final-norm output in token order; source: ResidentEmbedding; tgt_sorted [N]
    int32 targets (-1 = none) in the order `perm` (tokens with a target first, n_lab of them);
    e_target [n_lab, D] fp16 embedding rows of those targets.  Returns (loss_sum fp32 scalar,
    stats [N, 4] (loss, entropy, hit, lse) in sorted order, dY [N, D] fp16 = grad_scale *
    d(sum CE)/d(yf) in token order)."""
    n, d = yf.shape
    dev = yf.device
    if yf.dtype != torch.float16 or not yf.is_contiguous() or d % 64:
        raise ValueError("yf must be a contiguous fp16 [N, D] tensor, D a multiple of 64")
    for t, nm in ((tgt_sorted, "tgt_sorted"), (perm, "perm")):
        if t.dtype != torch.int32 or tuple(t.shape) != (n,) or not t.is_contiguous():
            raise ValueError(f"{nm} must be a contiguous int32 [{n}] tensor")
    if not 0 <= n_lab <= n:
        raise ValueError("n_lab must be within [0, N]")
    if n_lab > 0 and (e_target.dtype != torch.float16 or tuple(e_target.shape) != (n_lab, d)
                      or not e_target.is_contiguous()):
        raise ValueError(f"e_target must be a contiguous fp16 [{n_lab}, {d}] tensor")
    ys = yf.index_select(0, perm)
    state = torch.zeros((n, STATE_W), dtype=torch.float32, device=dev)
    state[:, 0] = float("-inf")
    acc = torch.zeros((max(n_lab, 1), d), dtype=torch.float32, device=dev)
    buf = torch.empty((n * source.chunk,), dtype=torch.float16, device=dev)
    lib = _lib.lib()
    for c in range(source.n_chunks):
        e_c = source.get(c)
        vc = e_c.shape[0]
        logits = buf[:n * vc].view(n, vc)
        _logits(ys, e_c, logits)
        rc = lib.dk_head_chunk(_lib.ptr(logits), _lib.ptr(tgt_sorted), _lib.ptr(state),
                               _lib.ptr(acc), n, n_lab, vc, c * source.chunk, float(grad_scale), d,
                               _lib.stream_handle(dev))
        _lib.check(rc, "dk_head_chunk")
        if n_lab > 0:
            _accumulate(acc[:n_lab], logits[:n_lab], e_c)
        source.release(c)
    del buf, ys
    stats = torch.empty((n, 4), dtype=torch.float32, device=dev)
    dy = torch.empty((n, d), dtype=torch.float16, device=dev)
    rc = lib.dk_head_finalize(_lib.ptr(state), _lib.ptr(tgt_sorted), _lib.ptr(perm), _lib.ptr(acc),
                              _lib.ptr(e_target) if n_lab > 0 else None, _lib.ptr(stats),
                              _lib.ptr(dy), n, n_lab, float(grad_scale), 1.0 / float(grad_scale),
                              d, _lib.stream_handle(dev))
    _lib.check(rc, "dk_head_finalize")
    return stats[:, 0].sum(), stats, dy


def warmup_specs(hidden=1536, chunk=CHUNK, impl="chunks"):
    """Nothing to warm up: the kernels are compiled ahead of time into libdk.so."""
    return []
