"""The NF4 linear stack of Qwen2.5-1.5B (28 layers), forward + backward, on the fused kernels.

Per layer (shapes of solution/fast_qwen.py:53 QWEN15: D = 1536, I = 8960, KV = 256, r = 16),
with M packed tokens:

  forward   z_q = lora_down(X, A_q, mask_q)            z_v likewise, one launch (rank-16 inputs)
            qkv = X W_qkv^T + b_qkv, + s z_q B_q^T on the q columns, + s z_v B_v^T on the v
                  columns                               one GEMM over the q|k|v rows, as the
                                                        reference's addmm (fast_qwen.py:947)
            o = X W_o^T                                 (X stands in for the attention output)
            act, gu = SwiGLU(X W_gu^T)                  gate|up as one GEMM, gu kept
            y = act W_d^T
  backward  gu <- SwiGLU'(dY_d W_d, gu)                 down^T GEMM + SwiGLU backward fused
            dX_mlp = gu W_gu                            [M, 2I] x [2I, D]
            dX_o = dY_o W_o
            dA_q, dB_q, dz_q = lora_grads(dQKV[:, q], ...)    and v, in shared launches
            dX_qkv = dQKV W_qkv + mask_q ks dz_q A_q + mask_v ks dz_v A_v    one NN GEMM

The upstream gradients dY_* are fixed random tensors (the attention and norm backward that would
produce them are not part of the linear stack).  The step's algorithmic work is
``FLOP_PER_LAYER`` per layer (dequant counted as no FLOPs).

Weights of the kinds in ``ahead`` are dequantised to fp16 into one slot per kind and the GEMMs
read the slot (dk_h16_*); the other kinds read the NF4 sections directly (dk_w4_*).  This is the
reference's workspace schedule (solution/fast_qwen.py:694-756): right after layer i's GEMM reads
kind k's slot, the dequant of kind k for the next layer in step order (i + 1 forward, i - 1
backward) is issued, and a weight still resident is not dequantised again (the last layer at the
forward/backward turn, layer 0 between steps).  ``ahead="layer"`` keeps one slot
for the whole layer instead and dequantises all seven weights of a layer in one launch (the
reference's dequant_layer, solution/k_nf4.py:176-181): the small q|k|v and o dequants are
launch-bound on their own.  ``dq_stream="side"`` runs those dequants on a
stream of their own, overlapping the GEMMs in between; ``"main"`` (the default) issues them in
order on the compute stream.  Measured on MI355X (28 layers, M = 2048) the in-order form is
1.3 ms per step faster: each GEMM holds all of a CU's registers at two workgroups per CU, so a
concurrent dequant only takes workgroup slots from it.

``ahead="carried"`` keeps two whole-layer slots (layer i in slot i % 2) and has the GEMM launches
of layer i carry the dequant of the next layer in step order into the other slot
(k_nf4.side_dequant): each launch in ``CARRY`` takes its share of the next layer's second-level
blocks on extra workgroups, which the hardware dispatches after the tiles, onto the CUs the
GEMM's last round leaves idle.  A layer no launch carries is dequantised by a launch of its own
right before its first GEMM.  The dequant count per step is the reference's: every layer is
dequantised once in the forward (layer 0 excepted, resident from the previous backward) and once
in the backward (the last layer excepted, resident from the forward).

The default is ``ahead="layer"``.  Measured on MI355X (28 layers, M = 2048, the two stacks' steps
interleaved in one process on two boxes): 14.27-14.31 ms per step against 14.38-14.45 ms carried.
With the whole-layer dequant at about 19 us per launch, the CUs a GEMM's last round leaves idle
are not free: the carried blocks slow the GEMM's own tiles (the clock and the HBM-bound epilogues
are shared) by more than the launch they replace.
"""

import torch

from . import k_nf4, quant
from .schedule import DequantAhead
from .w4linear import (down_swiglu_backward, gateup_swiglu_forward, linear_backward_dx,
                       linear_backward_dx_lora, linear_forward, linear_forward_lora,
                       lora_down_multi, lora_dz_multi, lora_grads_multi)

D, I, KV, R = 1536, 8960, 256, 16
QKV = D + 2 * KV
SHAPES = {"q_proj": (D, D), "k_proj": (KV, D), "v_proj": (KV, D), "o_proj": (D, D),
          "gate_proj": (I, D), "up_proj": (I, D), "down_proj": (D, I)}


def layer_flops(m, d=D, inter=I, kv=KV, r=R):
    """Algorithmic FLOPs of one layer's forward + backward at M = m tokens (2 M N K per GEMM)."""
    fwd = 2 * m * d * (d + 2 * kv + d + 2 * inter) + 2 * m * inter * d
    lora_fwd = 2 * m * d * r * 2 + 2 * m * r * (d + kv)           # two downs, two ups
    bwd = fwd                                                        # dX of every projection
    lora_bwd = 4 * 2 * m * d * r + 2 * (2 * m * r * (d + kv))      # dA, dX_lora (x2); dB, dz
    return fwd + lora_fwd + bwd + lora_bwd


FLOP_PER_LAYER_M2048 = layer_flops(2048)


class _WholeLayer:
    """All seven weights of layer i as one dequant job into the whole-layer slot."""

    def __init__(self, stack, i):
        self.stack, self.i = stack, i
        self.rows, self.cols = stack.layers[i]["packed"].numel, 1

    def dequantize(self, out):
        st = self.stack
        k_nf4.dequant_layer(st.layers[self.i]["packed"], st.code2, st.nf4, out.view(-1))
        return out


class _WholeLayerWith(_WholeLayer):
    """_WholeLayer whose launch also runs layer i's LoRA downs: run(dequant) launches them with
    the layer's dequant (dk_lora_down_multi_dequant)."""

    def __init__(self, stack, i, run):
        super().__init__(stack, i)
        self.run = run

    def dequantize(self, out):
        st = self.stack
        pk = st.layers[self.i]["packed"]
        self.run(k_nf4.side_dequant(pk, st.code2, st.nf4, out.view(-1), 0, pk.n_qblocks // 256, -1))
        return out


class NF4LinearStack:
    """Random-init NF4 weights (W ~ N(0, 0.02), quantised on the GPU), rank-16 LoRA on q and v,
    and synthetic activations, all resident on `device`."""

    KINDS = ("qkv", "o", "gu", "d")
    # ahead="layer" on one stream: each forward layer's whole-layer dequant runs in the launch of
    # that layer's LoRA downs (dk_lora_down_multi_dequant) instead of a launch of its own
    LORA_WITH_DEQUANT = True
    # ahead="carried": the share of the next layer's dequant (fraction of its second-level blocks)
    # that each GEMM launch carries, in step order; the launches that leave CUs idle (a last round
    # of 128 x 128 tiles, split-K grids short of the CU count, 128 x 128 grids short of a round).
    # Backward only: measured on MI355X, the forward's idle windows are too short and the carried
    # stream slows the forward GEMMs' operand traffic by more than the launch it saves.  The
    # q|k|v dX launch carries the layer's LoRA column sums instead (lora_dz_multi).
    CARRY = {"fwd": (),
             "bwd": (("d", 0.60), ("gu", 0.20), ("o", 0.20))}

    def __init__(self, n_layers=28, m=2048, seed=0, device="cuda", p_drop=0.05, lora_scale=2.0,
                 save_gu=True, ahead="layer", dq_stream="main"):
        self.n_layers, self.m, self.device = n_layers, m, torch.device(device)
        self.s = float(lora_scale)
        self.keep_scale = 1.0 / float(torch.tensor(1.0 - p_drop, dtype=torch.float32))
        gen = torch.Generator(device=self.device)
        gen.manual_seed(seed)
        dev = self.device
        self.code2 = quant.code2_on(dev)
        self.nf4 = quant.nf4_table(dev)
        self.layers, self.lora = [], []
        for _ in range(n_layers):
            linears = {}
            for name in k_nf4.LAYER_WEIGHTS:
                w = (torch.randn(SHAPES[name], generator=gen, device=dev) * 0.02).half()
                linears[name] = quant.Linear4bit(quant.quantize_4bit(w, self.code2))
                del w
            packed, _ = k_nf4.repack_layer(linears, dev)
            self.layers.append(dict(
                packed=packed,
                qkv=packed.weights(("q_proj", "k_proj", "v_proj"), self.code2, self.nf4),
                o=packed.weight("o_proj", self.code2, self.nf4),
                gu=packed.weights(("gate_proj", "up_proj"), self.code2, self.nf4),
                d=packed.weight("down_proj", self.code2, self.nf4)))
            bound = 1.0 / D ** 0.5
            lo = {}
            for t, out in (("q", D), ("v", KV)):
                lo["A" + t] = ((torch.rand(R, D, generator=gen, device=dev) * 2 - 1) * bound).half()
                lo["B" + t] = (torch.randn(out, R, generator=gen, device=dev) * 0.02).half()
                lo["m" + t] = (torch.rand(m, D, generator=gen, device=dev) >= p_drop).to(torch.uint8)
            lo["bias"] = (torch.randn(QKV, generator=gen, device=dev) * 0.02).half()
            self.lora.append(lo)
        self.x = torch.randn(m, D, generator=gen, device=dev).half()
        self.dy = {k: (torch.randn(m, n, generator=gen, device=dev) * 1e-2).half()
                   for k, n in (("qkv", QKV), ("o", D), ("d", D))}
        self.save_gu = save_gu
        f16 = torch.float16
        self.out = {k: torch.empty(m, n, dtype=f16, device=dev)
                    for k, n in (("qkv", QKV), ("o", D), ("y", D))}
        self.act = torch.empty(m, I, dtype=f16, device=dev)
        self.gu = [torch.empty(m, 2 * I, dtype=f16, device=dev) for _ in range(n_layers)]
        self.z = [{t: torch.empty(m, R, dtype=f16, device=dev) for t in ("q", "v")}
                  for _ in range(n_layers)]
        self.dx_qkv = torch.empty(m, D, dtype=torch.float32, device=dev)
        self.dx_o = torch.empty(m, D, dtype=f16, device=dev)
        self.dx_mlp = torch.empty(m, D, dtype=f16, device=dev)
        self.grads = [None] * n_layers
        self.probe = None   # (operator name, [(start event, end event), ...]) or None
        self._deferred = None   # layer whose whole-layer dequant waits for its LoRA downs
        self._setup_schedule(ahead, dq_stream)

    def _setup_schedule(self, ahead, dq_stream):
        """The fp16 slots of the dequant-ahead schedule (see the module docstring)."""
        self.carried = ahead == "carried"
        self.whole_layer = ahead in ("layer", "carried")
        if self.carried:
            self.ahead = self.KINDS
            pk = self.layers[0]["packed"]
            first = {"qkv": "q_proj", "o": "o_proj", "gu": "gate_proj", "d": "down_proj"}
            self.views = {k: (pk.segments[first[k]][0], self.layers[0][k].rows * self.layers[0][k].cols)
                          for k in self.KINDS}
            self.slots = [torch.empty(pk.numel, dtype=torch.float16, device=self.device)
                          for _ in range(2)]
            self.slot_layer = [None, None]    # (layer, pass that dequantised it) per slot
            self._pass = 0
            self.dq = None
            n_sb = self.n_sb = pk.n_qblocks // 256
            self.carry = {}
            for way, shares in self.CARRY.items():
                acc, bounds = 0.0, {}
                for kind, frac in shares:
                    lo = round(acc * n_sb)
                    acc += frac
                    bounds[kind] = (lo, round(min(acc, 1.0) * n_sb))
                if shares:
                    bounds[shares[-1][0]] = (bounds[shares[-1][0]][0], n_sb)
                self.carry[way] = bounds
            return
        if self.whole_layer:
            self.ahead = self.KINDS
            pk = self.layers[0]["packed"]
            first = {"qkv": "q_proj", "o": "o_proj", "gu": "gate_proj", "d": "down_proj"}
            self.views = {k: (pk.segments[first[k]][0], self.layers[0][k].rows * self.layers[0][k].cols)
                          for k in self.KINDS}
            self.dq = DequantAhead(self.device, {"layer": pk.numel}, dq_stream)
        else:
            unknown = set(ahead) - set(self.KINDS)
            if unknown:
                raise ValueError(f"unknown weight kinds {sorted(unknown)}")
            self.ahead = tuple(ahead)
            self.dq = (DequantAhead(self.device, {k: self.layers[0][k].rows * self.layers[0][k].cols
                                                  for k in self.ahead}, dq_stream)
                       if self.ahead else None)

    @property
    def flops_per_step(self):
        return self.n_layers * layer_flops(self.m)

    def _w16(self, kind, i):
        """Layer i's fp16 weight of `kind` from its slot, or None for an NF4 read."""
        if kind not in self.ahead:
            return None
        if self.carried:
            # a layer's weights are dequantised in this pass (carried in by the previous layer's
            # launches, else by a launch of their own here), except the pass's first layer, which
            # may still hold them from the other pass (the reference's reuse at the turn and
            # between steps)
            slot = i % 2
            held = self.slot_layer[slot]
            first = 0 if self._forward else self.n_layers - 1
            if held != (i, self._pass) and not (i == first and held is not None and held[0] == i):
                k_nf4.dequant_layer(self.layers[i]["packed"], self.code2, self.nf4, self.slots[slot])
                self.slot_layer[slot] = (i, self._pass)
            start, n = self.views[kind]
            return self.slots[slot][start:start + n]
        if self.whole_layer:
            self.dq.issue("layer", i, _WholeLayer(self, i))     # no-op when already resident
            start, n = self.views[kind]
            return self.dq.take("layer", i)[start:start + n]
        key = (i, kind)
        self.dq.issue(kind, key, self.layers[i][kind])     # no-op when already resident
        return self.dq.take(kind, key)

    def _side(self, kind, nxt):
        """ahead="carried": the share of layer `nxt`'s dequant that this launch of `kind` carries
        into slot nxt % 2, or None."""
        if not self.carried or not 0 <= nxt < self.n_layers:
            return None
        bounds = self.carry["fwd" if self._forward else "bwd"]
        if kind not in bounds:
            return None
        sb0, sb1 = bounds[kind]
        slot = nxt % 2
        if sb1 == self.n_sb:    # the layer's last share: from here on the slot holds layer nxt
            self.slot_layer[slot] = (nxt, self._pass)
        return k_nf4.side_dequant(self.layers[nxt]["packed"], self.code2, self.nf4,
                                  self.slots[slot], sb0, sb1, -1)

    def _done(self, kind, nxt):
        """The slot of `kind` has had its last reader; dequantise layer `nxt`'s weight into it
        (whole-layer slot: after the last weight of the layer in step order)."""
        if kind not in self.ahead or self.carried:
            return
        if self.whole_layer:
            if kind != ("d" if self._forward else "qkv"):    # the layer's last weight
                return
            self.dq.release("layer")
            if 0 <= nxt < self.n_layers:
                if self._forward and self.dq.stream is None and self.LORA_WITH_DEQUANT:
                    self._deferred = nxt   # issued with layer nxt's LoRA downs (_lora_downs)
                else:
                    self.dq.issue("layer", nxt, _WholeLayer(self, nxt))
            return
        self.dq.release(kind)
        if 0 <= nxt < self.n_layers:
            self.dq.issue(kind, (nxt, kind), self.layers[nxt][kind])

    def op_name(self, kind, base):
        """Operator name as the kernel table and the timing probe use it."""
        return ("h16" if kind in self.ahead else "w4") + base

    def forward_layer(self, i):
        if i == 0 or not getattr(self, "_forward", False):
            self._pass = getattr(self, "_pass", 0) + 1
        self._forward = True
        L, lo, z, x, o = self.layers[i], self.lora[i], self.z[i], self.x, self.out
        op, nm, w16, done, side = self._op, self.op_name, self._w16, self._done, self._side
        self._lora_downs(i, lambda dq: op(
            "lora_down q+v", lora_down_multi, x,
            [(lo["Aq"], lo["mq"], self.keep_scale), (lo["Av"], lo["mv"], self.keep_scale)],
            outs=[z["q"], z["v"]], dequant=dq))
        op(nm("qkv", "_linear_fwd qkv+lora"), linear_forward_lora, x, L["qkv"], lo["bias"],
           self.qkv_terms(i), out=o["qkv"], w16=w16("qkv", i), side=side("qkv", i + 1))
        done("qkv", i + 1)
        op(nm("o", "_linear_fwd o"), linear_forward, x, L["o"], out=o["o"], w16=w16("o", i),
           side=side("o", i + 1))
        done("o", i + 1)
        op(nm("gu", "_gateup_swiglu_fwd"), gateup_swiglu_forward, x, L["gu"], act=self.act,
           gu=self.gu[i], w16=w16("gu", i), side=side("gu", i + 1))
        done("gu", i + 1)
        op(nm("d", "_linear_fwd down"), linear_forward, self.act, L["d"], out=o["y"],
           w16=w16("d", i), side=side("d", i + 1))
        done("d", i + 1)

    def _lora_downs(self, i, run):
        """Layer i's LoRA downs: run(dequant) launches them, in one launch with layer i's
        whole-layer dequant (a k_nf4.side_dequant description) when _done deferred that dequant
        to here, else with dequant None.  The downs are the layer's first operator that the
        dequant can share a launch with: they need the layer's input, and the dequant only has
        to precede the layer's first GEMM."""
        if getattr(self, "_deferred", None) == i and self.dq.holds["layer"] != i:
            self._deferred = None
            self.dq.issue("layer", i, _WholeLayerWith(self, i, run))
        else:
            run(None)

    def backward_layer(self, i):
        if i == self.n_layers - 1 or getattr(self, "_forward", True):
            self._pass = getattr(self, "_pass", 0) + 1
        self._forward = False
        L, lo, z, x, dy = self.layers[i], self.lora[i], self.z[i], self.x, self.dy
        gu = self.gu[i]
        op, nm, w16, done, side = self._op, self.op_name, self._w16, self._done, self._side
        op(nm("d", "_down_swiglu_bwd"), down_swiglu_backward, dy["d"], L["d"], gu, w16=w16("d", i),
           side=side("d", i - 1))
        done("d", i - 1)
        op(nm("gu", "_linear_bwd_dx gate|up"), linear_backward_dx, gu, L["gu"], out=self.dx_mlp,
           w16=w16("gu", i), side=side("gu", i - 1))
        done("gu", i - 1)
        op(nm("o", "_linear_bwd_dx o"), linear_backward_dx, dy["o"], L["o"], out=self.dx_o,
           w16=w16("o", i), side=side("o", i - 1))
        done("o", i - 1)
        dqkv = dy["qkv"]
        terms = [(dqkv[:, :D], z["q"], lo["Bq"], self.s, lo["mq"], self.keep_scale),
                 (dqkv[:, D + KV:], z["v"], lo["Bv"], self.s, lo["mv"], self.keep_scale)]
        w16q = w16("qkv", i)
        sums = None
        if w16q is not None:
            # dz now; the q|k|v dX launch carries the column sums (dA, dB) on its idle CUs
            sums = op("lora_grads q+v", lora_dz_multi, x, terms)
            (daq, dbq, dzq), (dav, dbv, dzv) = sums.grads
        else:
            (daq, dbq, dzq), (dav, dbv, dzv) = op("lora_grads q+v", lora_grads_multi, x, terms)
        op(nm("qkv", "_linear_bwd_dx qkv+lora"), linear_backward_dx_lora, dqkv, L["qkv"],
           [(dzq, lo["Aq"], lo["mq"], self.keep_scale), (dzv, lo["Av"], lo["mv"], self.keep_scale)],
           out=self.dx_qkv, w16=w16q, side=side("qkv", i - 1), sums=sums)
        done("qkv", i - 1)
        self.grads[i] = (daq, dbq, dav, dbv)

    def qkv_terms(self, i):
        """LoRA terms of layer i's fused QKV forward: q on columns [0, D), v on [D + KV, QKV)."""
        lo, z = self.lora[i], self.z[i]
        return [(z["q"], lo["Bq"], 0, D, self.s), (z["v"], lo["Bv"], D + KV, QKV, self.s)]

    def _op(self, name, fn, *args, **kwargs):
        """Run one operator; when ``self.probe`` is ``(name, events)`` for this operator, bracket
        it with a pair of timing events on the current stream (the stream it launches on)."""
        probe = self.probe
        if probe is None or probe[0] != name:
            return fn(*args, **kwargs)
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        result = fn(*args, **kwargs)
        e1.record()
        probe[1].append((e0, e1))
        return result

    def step(self):
        for i in range(self.n_layers):
            self.forward_layer(i)
        for i in reversed(range(self.n_layers)):
            self.backward_layer(i)
