"""A whole Qwen2.5 QLoRA training step of the packed batch on this package's kernels.

The linear stack (stack.NF4LinearStack: NF4 weights, LoRA adapters and keep-masks, the dequant
slot and its dequant schedule) with everything around it, in the order of the reference's
FastQwen2.forward / backward (solution/fast_qwen.py:985-1390):
  forward   x_0 = E[ids] (fp32 residual stream)
            per layer: y = RMSNorm(x_i) (+ the previous MLP output added on the way, x_i kept),
            xq, xv = fp16(dropout(y)) of the fp32 y, z_q, z_v = LoRA-down(xq, xv), qkv = y W_qkv^T + b + LoRA-up, rotated (one GEMM),
            attention, o = out W_o^T, y2 = RMSNorm(x_i + o), act, gu = SwiGLU(y2 W_gu^T),
            d = act W_d^T
            y_f = RMSNorm(x_L + d), LM head over vocabulary chunks: loss, stats, d(y_f)
  backward  final norm, then per layer: down^T + SwiGLU', gate|up^T dX, norm 2 (residual in
            place), o^T, attention, QKV epilogue backward (rotation^T, GQA sums), q+v LoRA
            gradients, q|k|v^T with the masked LoRA input terms (fp32), norm 1 (layer 0 only its
            LoRA gradients, as the reference)
Every activation the backward needs is kept in HBM (about 120 MB per layer at 2048 tokens): the
reference's host arenas, recompute plans and offload options exist for a 16 GB card and are not
built.  Weights are random (W ~ N(0, 0.02) NF4, norm weights near 1, embedding ~ N(0, 0.02));
the tokens and targets are random ids, each sequence's targets its next token (-1 at its end).
"""

import torch

from . import k_attn, k_head, k_norm, k_rope
from .stack import D, KV, NF4LinearStack, layer_flops
from .w4linear import (down_swiglu_backward, gateup_swiglu_forward, linear_backward_dx,
                       linear_backward_dx_lora, linear_forward, linear_forward_rope,
                       lora_down_multi, lora_dz_multi, lora_grads_multi)

NQ, NKV, HD = 12, 2, 128
VOCAB = 151936


def rope_tables(positions, hd=HD, theta=1.0e6, device="cuda"):
    """cos/sin [positions, hd] fp32 as Qwen2's rotary embedding builds them (angles p theta^(-2i/hd),
    the half-width table repeated)."""
    inv = 1.0 / (theta ** (torch.arange(0, hd, 2, dtype=torch.float32, device=device) / hd))
    fr = torch.arange(positions, dtype=torch.float32, device=device)[:, None] * inv[None, :]
    emb = torch.cat((fr, fr), 1)
    return emb.cos().contiguous(), emb.sin().contiguous()


class QwenQLoRAStep(NF4LinearStack):
    """Random-init Qwen2.5-1.5B (n_layers decoder layers, the LM head over `vocab`) with rank-16
    LoRA on q and v, one packed batch of sequences of lengths `lens`."""

    def __init__(self, lens, n_layers=28, vocab=VOCAB, seed=0, device="cuda", eps=1e-6,
                 head_grad_scale=1024.0, head_chunk=k_head.CHUNK, ahead="layer"):
        m = int(sum(lens))
        super().__init__(n_layers, m, seed=seed, device=device, ahead=ahead)
        dev, f16, f32 = self.device, torch.float16, torch.float32
        self.lens, self.eps, self.head_grad_scale = list(lens), float(eps), float(head_grad_scale)
        gen = torch.Generator(device=dev)
        gen.manual_seed(seed + 1)

        def norm_w():
            return (1.0 + 0.1 * torch.randn(D, generator=gen, device=dev)).contiguous()
        self.w_in = [norm_w() for _ in range(n_layers)]
        self.w_post = [norm_w() for _ in range(n_layers)]
        self.w_final = norm_w()
        self.cos, self.sin = rope_tables(max(lens), device=dev)
        self.pos = torch.cat([torch.arange(n, dtype=torch.int32, device=dev) for n in lens])
        self.meta = k_attn.meta_for(lens, dev)
        # embedding, tokens and next-token targets (sorted: rows with a target first)
        self.emb = (torch.randn(vocab, D, generator=gen, device=dev) * 0.02).half()
        ids = torch.randint(0, vocab, (m,), generator=gen, device=dev)
        tgt = torch.cat([ids[1:], ids[:1]])
        ends = torch.cumsum(torch.tensor(lens, device=dev), 0) - 1
        tgt[ends] = -1
        self.source = k_head.ResidentEmbedding(self.emb, head_chunk)
        self.use_tokens(ids, tgt)
        # activations kept for the backward, per layer
        L = n_layers
        self.xin = [self.x0] + [torch.empty(m, D, dtype=f32, device=dev) for _ in range(L - 1)]
        self.y16 = [torch.empty(m, D, dtype=f16, device=dev) for _ in range(L)]
        # the LoRA inputs: fp16(dropout(y)) of the fp32 norm output, per adapter
        self.xq = [torch.empty(m, D, dtype=f16, device=dev) for _ in range(L)]
        self.xv = [torch.empty(m, D, dtype=f16, device=dev) for _ in range(L)]
        self.qkv_b = [torch.empty(m, (NQ + 2 * NKV) * HD, dtype=f16, device=dev) for _ in range(L)]
        self.att = [None] * L
        self.lse = [None] * L
        self.op = [torch.empty(m, D, dtype=f16, device=dev) for _ in range(L)]
        self.d16 = [torch.empty(m, D, dtype=f16, device=dev) for _ in range(L)]
        self.rstd1 = [torch.empty(m, dtype=f32, device=dev) for _ in range(L)]
        self.rstd2 = [torch.empty(m, dtype=f32, device=dev) for _ in range(L)]
        # per-step scratch
        self.y2 = torch.empty(m, D, dtype=f16, device=dev)
        self.h1 = torch.empty(m, D, dtype=f32, device=dev)
        self.hf = torch.empty(m, D, dtype=f32, device=dev)
        self.yf = torch.empty(m, D, dtype=f16, device=dev)
        self.rstd_f = torch.empty(m, dtype=f32, device=dev)
        self.dh = torch.empty(m, D, dtype=f32, device=dev)
        self.dh16 = torch.empty(m, D, dtype=f16, device=dev)
        self.dy2 = torch.empty(m, D, dtype=f16, device=dev)
        self.dout = torch.empty(m, NQ * HD, dtype=f16, device=dev)
        self.dx32 = torch.empty(m, D, dtype=f32, device=dev)
        self.one = torch.ones(1, dtype=f32, device=dev)

    @classmethod
    def for_batch(cls, batch, **kwargs):
        """The step on the tokens of a packed batch (trainer.pack): its rows' lengths, token ids
        and next-token targets; the weights are random-init as for any instance."""
        st = cls(batch.lens, **kwargs)
        st.use_tokens(batch.ids, batch.tgt)
        return st

    def use_tokens(self, ids, tgt):
        """Token ids [m] and next-token targets [m] (-1: none), in token order: the embedding rows
        the first layer reads, and the head's targets in sorted order (tokens with a target
        first, the order trainer.pack's perm gives)."""
        dev = self.device
        ids = torch.as_tensor(ids, device=dev).long()
        tgt = torch.as_tensor(tgt, device=dev).to(torch.int32)
        if ids.shape != (self.m,) or tgt.shape != (self.m,):
            raise ValueError(f"ids and targets must be [{self.m}] (the step's token count)")
        self.x0 = self.emb.index_select(0, ids).float()
        if hasattr(self, "xin"):
            self.xin[0] = self.x0
        has = tgt >= 0
        self.perm = torch.cat([torch.nonzero(has)[:, 0], torch.nonzero(~has)[:, 0]]).to(torch.int32)
        self.tgt_sorted = tgt.index_select(0, self.perm.long()).contiguous()
        self.n_lab = int(has.sum())
        self.e_target = self.emb.index_select(0, self.tgt_sorted[:self.n_lab].long()).contiguous()
        self.tgt = tgt

    @property
    def flops_per_step(self):
        """Algorithmic FLOPs: the linear layers, the causal attention (2 hd L(L+1) per sequence and
        head forward, 2.5 times that backward), the LM head (logits and P E, 2 M V D each)."""
        att = sum(2 * HD * n * (n + 1) for n in self.lens) * NQ * 3.5
        return self.n_layers * (layer_flops(self.m) + att) + 2 * 2 * self.m * self.emb.shape[0] * D

    def forward(self):
        """Returns (loss_sum, stats [N, 4] in sorted order, d(y_f) [N, D] fp16)."""
        self._pass = getattr(self, "_pass", 0) + 1
        self._forward = True
        w16, side, done = self._w16, self._side, self._done
        x, d_prev = self.x0, None
        for i in range(self.n_layers):
            Lw, lo, z = self.layers[i], self.lora[i], self.z[i]
            # norm 1 with the previous layer's MLP output added on the way (x_i materialised), and
            # the two LoRA inputs dropped out from its fp32 output (solution/k_norm.py:49-53)
            k_norm.rms_forward(x, self.w_in[i], self.y16[i], self.rstd1[i], self.eps, delta=d_prev,
                               xout=self.xin[i] if d_prev is not None else None,
                               xq=self.xq[i], xv=self.xv[i], mq=lo["mq"], mv=lo["mv"],
                               keep_scale=self.keep_scale)
            y = self.y16[i]
            self._lora_downs(i, lambda dq: lora_down_multi(
                None, [(lo["Aq"], None, 1.0, self.xq[i]), (lo["Av"], None, 1.0, self.xv[i])],
                outs=[z["q"], z["v"]], dequant=dq))
            linear_forward_rope(y, Lw["qkv"], lo["bias"], self.qkv_terms(i), self.pos, self.cos,
                                self.sin, (NQ + NKV) * HD, out=self.qkv_b[i], w16=w16("qkv", i),
                                side=side("qkv", i + 1))
            done("qkv", i + 1)
            self.att[i], self.lse[i] = k_attn.attention_forward(self.qkv_b[i], self.meta, NQ, NKV, HD)
            linear_forward(self.att[i], Lw["o"], out=self.op[i], w16=w16("o", i), side=side("o", i + 1))
            done("o", i + 1)
            k_norm.rms_forward(self.xin[i], self.w_post[i], self.y2, self.rstd2[i], self.eps,
                               delta=self.op[i], xout=self.h1)
            gateup_swiglu_forward(self.y2, Lw["gu"], act=self.act, gu=self.gu[i], w16=w16("gu", i),
                                  side=side("gu", i + 1))
            done("gu", i + 1)
            linear_forward(self.act, Lw["d"], out=self.d16[i], w16=w16("d", i), side=side("d", i + 1))
            done("d", i + 1)
            x, d_prev = self.h1, self.d16[i]
        k_norm.rms_forward(x, self.w_final, self.yf, self.rstd_f, self.eps, delta=d_prev,
                           xout=self.hf)
        return k_head.streamed_head(self.yf, self.source, self.tgt_sorted, self.perm, self.n_lab,
                                    self.e_target, self.head_grad_scale)

    def backward(self, dy_head, g_loss=1.0):
        """LoRA gradients of g_loss * loss_sum: self.grads[i] = (dA_q, dB_q, dA_v, dB_v) fp32."""
        self._pass = getattr(self, "_pass", 0) + 1
        self._forward = False
        w16, side, done = self._w16, self._side, self._done
        gscale = torch.full((1,), float(g_loss) / self.head_grad_scale, dtype=torch.float32,
                            device=self.device)
        dh, dh16 = self.dh, self.dh16
        k_norm.rms_backward(dy_head, gscale, self.hf, self.w_final, self.rstd_f, dh, out16=dh16)
        ks = self.keep_scale
        for i in reversed(range(self.n_layers)):
            Lw, lo, z = self.layers[i], self.lora[i], self.z[i]
            down_swiglu_backward(dh16, Lw["d"], self.gu[i], w16=w16("d", i), side=side("d", i - 1))
            done("d", i - 1)
            linear_backward_dx(self.gu[i], Lw["gu"], out=self.dy2, out_dtype=torch.float16,
                               w16=w16("gu", i), side=side("gu", i - 1))
            done("gu", i - 1)
            # norm 2: its input x_i + o rebuilt in registers; the residual gradient in place
            k_norm.rms_backward(self.dy2, self.one, self.xin[i], self.w_post[i], self.rstd2[i], dh,
                                dres=dh, out16=dh16, delta=self.op[i])
            linear_backward_dx(dh16, Lw["o"], out=self.dout, out_dtype=torch.float16,
                               w16=w16("o", i), side=side("o", i - 1))
            done("o", i - 1)
            dq, dkp, dvp = k_attn.attention_backward(self.qkv_b[i], self.att[i], self.lse[i],
                                                     self.dout, self.meta, NQ, NKV, HD)
            dqkv = self.qkv_b[i]      # the QKV epilogue backward writes d(qkv) over the forward's qkv
            k_rope.qkv_epilogue_backward(dq, dkp, dvp, self.pos, self.cos, self.sin, dqkv, NQ, NKV,
                                         HD, NQ // NKV)
            del dq, dkp, dvp
            terms = [(dqkv[:, :D], z["q"], lo["Bq"], self.s, None, 1.0, self.xq[i]),
                     (dqkv[:, D + KV:], z["v"], lo["Bv"], self.s, None, 1.0, self.xv[i])]
            w16q = w16("qkv", i) if i > 0 else None
            sums = None
            if w16q is not None:
                # dz now; the q|k|v dX launch carries the column sums (dA, dB) on its idle CUs
                sums = lora_dz_multi(None, terms)
                (daq, dbq, dzq), (dav, dbv, dzv) = sums.grads
            else:
                (daq, dbq, dzq), (dav, dbv, dzv) = lora_grads_multi(None, terms)
            if i > 0:
                # d(y) = dqkv W_qkv + the masked LoRA input terms, in fp32, into norm 1's backward
                linear_backward_dx_lora(dqkv, Lw["qkv"], [(dzq, lo["Aq"], lo["mq"], ks),
                                                          (dzv, lo["Av"], lo["mv"], ks)],
                                        out=self.dx32, w16=w16q, side=side("qkv", i - 1),
                                        sums=sums)
                done("qkv", i - 1)
                k_norm.rms_backward(self.dx32, self.one, self.xin[i], self.w_in[i], self.rstd1[i],
                                    dh, dres=dh, out16=dh16)
            self.grads[i] = (daq, dbq, dav, dbv)
        return self.grads

    def step(self):
        loss, stats, dy_head = self.forward()
        self.backward(dy_head)
        return loss
