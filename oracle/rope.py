"""CPU restatement of the fused QKV epilogue: LoRA add + rotary embedding (forward), transposed
rotation + GQA partial sums (backward).  TEST INFRASTRUCTURE ONLY: imported by tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg, never by the product path.

Row layout [q heads (NQ) | k heads (NKV) | v heads (NKV)] x HD, fp16; c, s = cos/sin[pos, :HD/2]
(the tables hold the half-width angles twice, as Qwen2's rotary embedding builds them).
forward (solution/k_rope.py:23-61), every product and sum rounded to fp32 on its own:
    q = fp32(q16) + fp32(lq16) * scale;  k = fp32(k16);  v = fp32(v16) + fp32(lv16) * scale
    q, k <- [x1 * c - x2 * s | x2 * c + x1 * s]  (x1, x2 the two halves of a head); stored fp16
backward (solution/k_rope.py:64-104): dk / dv rows hold GIN partials per KV head, summed in order;
    dx1 = d1 * c + d2 * s,  dx2 = d2 * c - d1 * s;  stored fp16
"""

import numpy as np

F32, F16 = np.float32, np.float16


def rope_tables(positions, hd, theta=1e6):
    """cos/sin [positions, hd] fp32 as Qwen2 builds them: angles p * theta^(-2i/hd), twice."""
    inv = (1.0 / (theta ** (np.arange(0, hd, 2, dtype=F32) / hd))).astype(F32)
    fr = (np.arange(positions, dtype=F32)[:, None] * inv[None, :]).astype(F32)
    emb = np.concatenate([fr, fr], 1)
    return np.cos(emb).astype(F32), np.sin(emb).astype(F32)


def _rot(x1, x2, c, s):
    o1 = ((x1 * c).astype(F32) - (x2 * s).astype(F32)).astype(F32)
    o2 = ((x2 * c).astype(F32) + (x1 * s).astype(F32)).astype(F32)
    return o1, o2


def qkv_epilogue_fwd(qkv16, lq16, lv16, pos, cos, sin, scale, nq, nkv, hd):
    """Returns the new qkv buffer (fp16)."""
    qkv = np.asarray(qkv16, F16).astype(F32)
    n = qkv.shape[0]
    half = hd // 2
    p = np.asarray(pos).astype(np.int64)
    c = np.asarray(cos, F32)[p, :half][:, None, :]
    s = np.asarray(sin, F32)[p, :half][:, None, :]
    sc = F32(scale)
    q = qkv[:, :nq * hd].reshape(n, nq, hd)
    q = (q + (np.asarray(lq16, F16).astype(F32).reshape(n, nq, hd) * sc).astype(F32)).astype(F32)
    k = qkv[:, nq * hd:(nq + nkv) * hd].reshape(n, nkv, hd)
    v = qkv[:, (nq + nkv) * hd:]
    v = (v + (np.asarray(lv16, F16).astype(F32) * sc).astype(F32)).astype(F32)
    out = np.empty_like(qkv)
    for a, x in ((0, q), (nq * hd, k)):
        o1, o2 = _rot(x[..., :half], x[..., half:], c, s)
        heads = x.shape[1]
        out[:, a:a + heads * hd] = np.concatenate([o1, o2], -1).reshape(n, heads * hd)
    out[:, (nq + nkv) * hd:] = v
    return out.astype(F16)


def qkv_epilogue_bwd(dq, dk, dv, pos, cos, sin, nq, nkv, hd, gin):
    """dq [n, nq*hd], dk / dv [n, nkv*gin*hd] (fp32 or fp16) -> out [n, (nq + 2 nkv) hd] fp16."""
    dq = np.asarray(dq).astype(F32)
    n = dq.shape[0]
    half = hd // 2
    p = np.asarray(pos).astype(np.int64)
    c = np.asarray(cos, F32)[p, :half][:, None, :]
    s = np.asarray(sin, F32)[p, :half][:, None, :]
    out = np.empty((n, (nq + 2 * nkv) * hd), F32)

    def rot_t(d):
        d1, d2 = d[..., :half], d[..., half:]
        o1 = ((d1 * c).astype(F32) + (d2 * s).astype(F32)).astype(F32)
        o2 = ((d2 * c).astype(F32) - (d1 * s).astype(F32)).astype(F32)
        return np.concatenate([o1, o2], -1)

    out[:, :nq * hd] = rot_t(dq.reshape(n, nq, hd)).reshape(n, -1)
    parts_k = np.asarray(dk).astype(F32).reshape(n, nkv, gin, hd)
    parts_v = np.asarray(dv).astype(F32).reshape(n, nkv, gin, hd)
    ksum = np.zeros((n, nkv, hd), F32)
    vsum = np.zeros((n, nkv, hd), F32)
    for g in range(gin):
        ksum = (ksum + parts_k[:, :, g]).astype(F32)
        vsum = (vsum + parts_v[:, :, g]).astype(F32)
    out[:, nq * hd:(nq + nkv) * hd] = rot_t(ksum).reshape(n, -1)
    out[:, (nq + nkv) * hd:] = vsum.reshape(n, -1)
    return out.astype(F16)
