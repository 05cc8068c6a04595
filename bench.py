"""Benchmark of the NF4 QLoRA linear path on one MI355X.

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-cpu] [--layers 28]

Workload: the 28-layer NF4 linear stack of Qwen2.5-1.5B, forward + backward,
M = 2048 packed tokens, LoRA r = 16 (alpha 32) with dropout 0.05 on q_proj and v_proj, random-init
weights W ~ N(0, 0.02) quantised to NF4 with double quantisation on the GPU, synthetic fp16
activations ~ N(0, 1) and upstream gradients ~ N(0, 1e-2), all resident in HBM before timing.
One step = every layer's forward then every layer's backward (dX of all seven projections plus
the LoRA gradients).  value = algorithmic TFLOP/s of the step (2 M N K per GEMM; dequant counts
no FLOPs).

Also measured, with HIP events: each operator of the step in isolation and the NF4 dequant of all
28 layers (3.30 GB of algorithmic traffic, far above the 256 MB Infinity Cache), both as CUDA-graph
replays so the host's launch overhead is not in the figure; BASELINE configs 0-3 on layer 0 of
the stack (GPU time and roofline fraction, the CPU oracle's time on this host's cores, and the
parity of the GPU result with the oracle).  The CPU baseline of the metric times the CPU oracle
(numpy dequant + fp32 torch GEMMs) on a sample of config 4's layers, on this host's cores.
"""

import argparse
import json
import math
import os
import sys
import time

HBM_PEAK_GBS = 8000.0
EAGER = False   # --eager: time operators by plain back-to-back launches (counter runs count dispatches)
FP16_PEAK_TFLOPS = 2516.6   # 256 CU x 2.4 GHz x 4096 FLOP/clk (dense fp16 MFMA)
# the operator whose launches the last timed step times (the largest per-layer share of the step):
# the gate|up forward, h16_ or w4_ by the schedule
DOMINANT = "_gateup_swiglu_fwd"


def _events(torch):
    return torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)


def time_op(torch, fn, reps):
    """Average duration (ms) of fn over `reps` back-to-back launches, HIP events on the current
    stream (the stream every operator launches on)."""
    fn()
    torch.cuda.synchronize()
    e0, e1 = _events(torch)
    e0.record()
    for _ in range(reps):
        fn()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / reps


def time_graph(torch, fn, iters=10, reps=3):
    """Average GPU time (ms) of one call of fn: `iters` calls captured in one CUDA graph and the
    graph replayed `reps` times, timed with HIP events.  This is the kernels' time plus the GPU-side
    gaps between them, without the host's launch overhead (which exceeds the kernel time of the
    small operators when they are launched back to back from Python)."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()                       # lazy allocations (workspaces, outputs) outside the capture
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(iters):
            fn()
    g.replay()
    torch.cuda.synchronize()
    e0, e1 = _events(torch)
    e0.record()
    for _ in range(reps):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / (reps * iters)
    del g
    return ms


def _median_s(fn, reps=5):
    """Median wall time (s) of fn on the CPU over `reps` runs after one warm-up run."""
    fn()
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return sorted(ts)[len(ts) // 2]


def _scaled_err(got, want, absolute=False):
    """Whether every element is within rtol 1e-2 / atol 2e-2 (the tolerance BASELINE.json's
    north_star states for GEMM outputs and LoRA gradients), and the largest error.  absolute: on
    the values themselves (forward outputs, of order 1); otherwise relative to the output's scale
    max |want| (gradients, which dY ~ N(0, 1e-2) makes small), reported as max |err| / scale."""
    import numpy as np
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    scale = 1.0 if absolute else (float(np.abs(want).max()) or 1.0)
    err = np.abs(got - want) / scale
    ok = bool(np.all(err <= 2e-2 + 1e-2 * np.abs(want) / scale))
    return float(err.max()), ok


def config_rows(torch, st, cpu=True):
    """BASELINE.json configs 0-3 on layer 0 of the bench's stack (its NF4 weights, LoRA factors,
    keep-masks, X and dY, generated as configs 0-4 prescribe): per config the GPU time of the
    NF4-reading kernels (CUDA-graph replay), its roofline fraction, the CPU oracle's time on this
    host's cores (NF4 dequant + fp32 GEMMs, median of 5) and the parity of the GPU result with the
    oracle (dequant bit-exact; GEMM outputs and LoRA gradients at rtol 1e-2 / atol 2e-2)."""
    import numpy as np
    from decentrik_prime_amd import k_nf4
    from decentrik_prime_amd import w4linear as W
    from oracle import linear, mlp, nf4
    torch.set_num_threads(os.cpu_count())
    m, D, I, KV, r = st.m, 1536, 8960, 256, 16
    L, lo, x, dev = st.layers[0], st.lora[0], st.x, st.x.device
    pk = L["packed"]
    ks, s = st.keep_scale, st.s
    f16 = torch.float16
    host = lambda t: t.detach().cpu().numpy()  # noqa: E731
    ws = {n: pk.weight(n, st.code2, st.nf4) for n in ("q_proj", "v_proj", "gate_proj", "down_proj")}
    wgu = pk.weights(("gate_proj", "up_proj"), st.code2, st.nf4)
    c2 = host(st.code2)

    def sections(w):
        return tuple(host(t) for t in (w.packed, w.qabs, w.scale2, w.offset2))

    def cpu_deq(w):
        return nf4.dequant(*sections(w), c2).reshape(w.rows, w.cols)

    g = lambda mm, n, k: 2.0 * mm * n * k  # noqa: E731
    rows = []
    cores = torch.get_num_threads()

    def row(cfg, what, ms, work, unit, cpu_s, parity, alt=None):
        if unit == "GB/s":
            rate = work / (ms * 1e-3) / 1e9
            gpu = {"us": round(ms * 1e3, 2), "bytes": int(work), "gbps": round(rate, 1),
                   "frac": round(rate / HBM_PEAK_GBS, 4)}
        else:
            rate = work / (ms * 1e-3) / 1e12
            gpu = {"us": round(ms * 1e3, 2), "gflop": round(work / 1e9, 3), "tflops": round(rate, 1),
                   "frac": round(rate / FP16_PEAK_TFLOPS, 4)}
        out = {"config": cfg, "what": what, "gpu": gpu}
        if alt:
            out["gpu_fp16_slot_form"] = alt
        if cpu_s is not None:
            out["cpu"] = {"s": round(cpu_s, 4), "cores": cores, "kind": "port",
                          "gpu_speedup": round(cpu_s / (ms * 1e-3), 1)}
        out["parity"] = parity
        rows.append(out)
        print(f"[bench] config {cfg}: {what}: {gpu} cpu {out.get('cpu')} parity {parity}",
              file=sys.stderr, flush=True)

    def check(label, pairs, absolute):
        worst, ok = 0.0, True
        for got, want in pairs:
            e, good = _scaled_err(got, want, absolute)
            worst, ok = max(worst, e), ok and good
        if not ok:
            raise RuntimeError(f"{label}: GPU result outside rtol 1e-2 / atol 2e-2 of the oracle")
        if absolute:
            return f"rtol 1e-2 / atol 2e-2: pass (max |err| {worst:.2e})"
        return f"rtol 1e-2 / atol 2e-2 of scale: pass (max |err| / scale {worst:.2e})"

    # config 0: dequant of one q_proj weight [1536, 1536]
    wq = ws["q_proj"]
    out0 = torch.empty(D * D, dtype=f16, device=dev)
    dq0 = lambda: k_nf4.dequant_tensors(wq.packed, wq.qabs, wq.scale2, wq.offset2, D * D // 64,  # noqa: E731
                                        st.code2, st.nf4, out0)
    ms0 = time_graph(torch, dq0)
    dq0()
    torch.cuda.synchronize()
    want0 = cpu_deq(wq).reshape(-1)
    exact = bool(np.array_equal(host(out0).view(np.uint16), want0.view(np.uint16)))
    if not exact:
        raise RuntimeError("config 0: GPU dequant not bit-exact with the oracle")
    row(0, "NF4 dequant of q_proj [1536,1536] (latency-bound at this size; the bandwidth figure is "
           "the 28-layer dequant)", ms0, D * D * (0.5 + 1 / 64 + 8 / 16384 + 2), "GB/s",
        _median_s(lambda: cpu_deq(wq)) if cpu else None, "bit-exact")

    # config 1: q_proj forward with the rank-16 LoRA term and dropout (no bias)
    wq16 = out0.view(D, D)
    aq, bq, mq = lo["Aq"], lo["Bq"], lo["mq"]
    y1 = torch.empty(m, D, dtype=f16, device=dev)
    z1 = torch.empty(m, r, dtype=f16, device=dev)

    def fwd1(w16=None):
        W.lora_down_multi(x, [(aq, mq, ks)], outs=[z1])
        return W.linear_forward(x, wq, z=z1, lora_B=bq, lora_scale=s, out=y1, w16=w16)
    f1 = g(m, D, D) + g(m, r, D) + g(m, D, r)
    ms1 = time_graph(torch, fwd1)
    ms1h = time_graph(torch, lambda: (dq0(), fwd1(wq16)))
    fwd1()
    torch.cuda.synchronize()
    xn, aqn, bqn, mqn = host(x), host(aq), host(bq), host(mq)
    ref1 = {}

    def cpu1():
        ref1["y"], ref1["z"] = linear.linear_fwd(xn, cpu_deq(wq), None, mqn, ks, aqn, bqn, s)
    cpu1_s = _median_s(cpu1) if cpu else (cpu1() or None)
    par1 = check("config 1", [(host(y1), ref1["y"]), (host(z1), ref1["z"])], True)
    row(1, "q_proj forward + LoRA r=16 with dropout, M=2048 (lora_down + dk_w4_linear_fwd: the NF4 "
           "weight dequantised into the workspace, then the 256-tile fp16 GEMM with the LoRA "
           "epilogue)", ms1,
        f1, "TFLOP/s", cpu1_s, par1,
        alt={"us": round(ms1h * 1e3, 2), "what": "dequant to fp16 + fp16 GEMM"})

    # config 2: MLP forward, no LoRA (gate|up + SwiGLU, down)
    act2 = torch.empty(m, I, dtype=f16, device=dev)
    gu2 = torch.empty(m, 2 * I, dtype=f16, device=dev)
    y2 = torch.empty(m, D, dtype=f16, device=dev)

    def fwd2():
        W.gateup_swiglu_forward(x, wgu, act=act2, gu=gu2)
        W.linear_forward(act2, ws["down_proj"], out=y2)
    f2 = g(m, 2 * I, D) + g(m, D, I)
    ms2 = time_graph(torch, fwd2, iters=3)
    fwd2()
    torch.cuda.synchronize()
    ref2 = {}

    def cpu2():
        ref2["gu"], ref2["h"], ref2["y"] = mlp.mlp_fwd(xn, cpu_deq(wgu), cpu_deq(ws["down_proj"]))
    cpu2_s = _median_s(cpu2, 3) if cpu else (cpu2() or None)
    par2 = check("config 2", [(host(act2), ref2["h"]), (host(y2), ref2["y"])], True)
    row(2, "MLP forward: gate|up + SwiGLU, down, M=2048 (NF4 weights, dequantised once to fp16 "
           "then the 256-tile GEMMs)", ms2, f2, "TFLOP/s", cpu2_s, par2)

    # config 3: backward of q_proj and v_proj (dX through the NF4 weight + LoRA dX, dA, dB)
    wv = ws["v_proj"]
    av, bv, mv = lo["Av"], lo["Bv"], lo["mv"]
    zv = W.lora_down_multi(x, [(av, mv, ks)])[0]
    dyq, dyv = st.dy["qkv"][:, :D], st.dy["qkv"][:, D + KV:]
    dxq = torch.empty(m, D, dtype=torch.float32, device=dev)
    dxv = torch.empty(m, D, dtype=torch.float32, device=dev)
    res3 = {}

    def bwd3():
        (daq, dbq, dzq), (dav, dbv, dzv) = W.lora_grads_multi(
            x, [(dyq, z1, bq, s, mq, ks), (dyv, zv, bv, s, mv, ks)])
        W.linear_backward_dx_lora(dyq, wq, [(dzq, aq, mq, ks)], out=dxq)
        W.linear_backward_dx_lora(dyv, wv, [(dzv, av, mv, ks)], out=dxv)
        res3.update(daq=daq, dbq=dbq, dav=dav, dbv=dbv)
    # q: dX + (dB, dz, dA, dX_lora) = 10.066 GFLOP; v: dX + the same four = 1.845 GFLOP
    f3 = g(m, D, D) + 4 * g(m, r, D) + g(m, D, KV) + 2 * g(m, KV, r) + 2 * g(m, r, D)
    ms3 = time_graph(torch, bwd3)
    bwd3()
    torch.cuda.synchronize()
    dyqn, dyvn, zqn, zvn = host(dyq), host(dyv), host(z1), host(zv)
    avn, bvn, mvn = host(av), host(bv), host(mv)
    ref3 = {}

    def cpu3():
        ref3["q"] = linear.linear_bwd(dyqn, cpu_deq(wq), zqn, xn, mqn, ks, aqn, bqn, s)
        ref3["v"] = linear.linear_bwd(dyvn, cpu_deq(wv), zvn, xn, mvn, ks, avn, bvn, s)
    cpu3_s = _median_s(cpu3) if cpu else (cpu3() or None)
    par3 = check("config 3", [(host(dxq), ref3["q"]["dx"]), (host(dxv), ref3["v"]["dx"]),
                              (host(res3["daq"]), ref3["q"]["dA"]), (host(res3["dbq"]), ref3["q"]["dB"]),
                              (host(res3["dav"]), ref3["v"]["dA"]), (host(res3["dbv"]), ref3["v"]["dB"])],
                  False)
    row(3, "q_proj + v_proj backward: dX through the NF4 weights with the masked LoRA dX, dA, dB, "
           "M=2048", ms3, f3, "TFLOP/s", cpu3_s, par3)
    return rows


def kernel_table(torch, st, reps, only=None):
    """Each operator of one layer's step in isolation (layer 0), with its algorithmic work.
    `only`: a set of operator names to restrict the table to."""
    from decentrik_prime_amd import w4linear as W
    m, D, I, KV, r = st.m, 1536, 8960, 256, 16
    QKV = D + 2 * KV
    L, lo, z, x, dy, o = st.layers[0], st.lora[0], st.z[0], st.x, st.dy, st.out
    ks, s = st.keep_scale, st.s
    gu = st.gu[0]
    gu_save = gu.clone()
    dzq = (torch.randn(m, r, device=x.device) * 1e-2).half()
    dzv = (torch.randn(m, r, device=x.device) * 1e-2).half()
    lora_terms = [(dy["qkv"][:, :D], z["q"], lo["Bq"], s, lo["mq"], ks),
                  (dy["qkv"][:, D + KV:], z["v"], lo["Bv"], s, lo["mv"], ks)]
    g = lambda mm, n, k: 2.0 * mm * n * k  # noqa: E731
    # fp16 copies of layer 0's weights: the operand of the dk_h16_* entry points, as the
    # side-stream dequant leaves it
    h = {k: L[k].dequantize() for k in st.KINDS}
    dq_bytes = lambda w: w.rows * w.cols * (0.5 + 1 / 64 + 8 / 16384 + 2)  # noqa: E731
    gemms = [
        # kind, name suffix, fn(w16), flops
        ("gu", "_gateup_swiglu_fwd",
         lambda w16: W.gateup_swiglu_forward(x, L["gu"], act=st.act, gu=gu, w16=w16), g(m, 2 * I, D)),
        ("d", "_linear_fwd down", lambda w16: W.linear_forward(st.act, L["d"], out=o["y"], w16=w16),
         g(m, D, I)),
        ("qkv", "_linear_fwd qkv+lora", lambda w16: W.linear_forward_lora(
            x, L["qkv"], lo["bias"], st.qkv_terms(0), out=o["qkv"], w16=w16),
         g(m, QKV, D) + g(m, D, r) + g(m, KV, r)),
        ("o", "_linear_fwd o", lambda w16: W.linear_forward(x, L["o"], out=o["o"], w16=w16), g(m, D, D)),
        ("d", "_down_swiglu_bwd", lambda w16: W.down_swiglu_backward(dy["d"], L["d"], gu, w16=w16),
         g(m, I, D)),
        ("gu", "_linear_bwd_dx gate|up",
         lambda w16: W.linear_backward_dx(gu, L["gu"], out=st.dx_mlp, w16=w16), g(m, D, 2 * I)),
        ("o", "_linear_bwd_dx o",
         lambda w16: W.linear_backward_dx(dy["o"], L["o"], out=st.dx_o, w16=w16), g(m, D, D)),
        ("qkv", "_linear_bwd_dx qkv+lora", lambda w16: W.linear_backward_dx_lora(
            dy["qkv"], L["qkv"], [(dzq, lo["Aq"], lo["mq"], ks), (dzv, lo["Av"], lo["mv"], ks)],
            out=st.dx_qkv, w16=w16), g(m, D, QKV) + 2 * g(m, D, r)),
    ]
    # the fused QKV projection with the rotary epilogue (the QKV epilogue's forward folded in; not
    # part of the linear stack's step): compare with h16_linear_fwd qkv+lora + qkv_epilogue_fwd
    rot = torch.arange(4096, device=x.device, dtype=torch.float32)[:, None] * (
        1.0 / (1e6 ** (torch.arange(0, 128, 2, device=x.device, dtype=torch.float32) / 128)))[None, :]
    rcos = torch.cat((rot, rot), 1).cos().contiguous()
    rsin = torch.cat((rot, rot), 1).sin().contiguous()
    rpos = (torch.arange(m, device=x.device, dtype=torch.int32) % 4096).contiguous()
    rope_row = ("h16_linear_fwd qkv+lora+rope", lambda: W.linear_forward_rope(
        x, L["qkv"], lo["bias"], st.qkv_terms(0), rpos, rcos, rsin, D + KV, out=o["qkv"],
        w16=h["qkv"]), g(m, QKV, D) + g(m, D, r) + g(m, KV, r), None, 0)
    rows = [rope_row]
    # k_proj alone (the step runs it inside the fused q|k|v GEMM): 2048 x 256 x 1536 does ~200
    # FLOP per byte of its operands, under the ~315 of the MFMA / HBM ridge, so the row gives both
    # TFLOP/s and GB/s.  Its NF4 weight is rows [D, D + KV) of the fused one (whole second-level
    # blocks).
    wk = W.W4.from_sections(L["qkv"].packed, L["qkv"].qabs, L["qkv"].scale2, L["qkv"].offset2,
                            D * D, KV, D, st.code2, st.nf4)
    ok = torch.empty(m, KV, dtype=torch.float16, device=x.device)
    k_bytes = lambda wb: m * D * 2 + wb + m * KV * 2  # noqa: E731
    rows.append(("w4_linear_fwd k alone", lambda: W.linear_forward(x, wk, out=ok), g(m, KV, D),
                 k_bytes(KV * D * (0.5 + 1 / 64 + 8 / 16384)), 0))
    rows.append(("h16_linear_fwd k alone",
                 lambda: W.linear_forward(x, wk, out=ok, w16=h["qkv"][D:D + KV]), g(m, KV, D),
                 k_bytes(KV * D * 2), 0))
    for kind, suffix, fn, flops in gemms:
        # both forms; the one the step runs counts once per layer, the other is reported only
        used = "h16" if kind in st.ahead else "w4"
        rows.append(("w4" + suffix, (lambda f: lambda: f(None))(fn), flops, None,
                     int(used == "w4")))
        rows.append(("h16" + suffix, (lambda f, k: lambda: f(h[k]))(fn, kind), flops, None,
                     int(used == "h16")))
    for kind in st.KINDS:
        # the dequant of one weight into its fp16 slot (HBM-bound)
        rows.append((f"dequant {kind}", (lambda k: lambda: L[k].dequantize(out=h[k]))(kind), 0.0,
                     dq_bytes(L[kind]), 0 if st.whole_layer else 2))
    # the whole layer in one launch (forward and backward of every layer; with the carried
    # schedule the forward's only: the backward's rides on the GEMM launches, whose in-step times
    # include it)
    from decentrik_prime_amd import k_nf4
    hl = torch.empty(L["packed"].numel, dtype=torch.float16, device=x.device)
    per_layer = (1 if getattr(st, "carried", False) else 2) if st.whole_layer else 0
    rows.append(("dequant layer", lambda: k_nf4.dequant_layer(L["packed"], st.code2, st.nf4, hl), 0.0,
                 L["packed"].numel * (0.5 + 1 / 64 + 8 / 16384 + 2), per_layer))
    rows += [
        ("lora_down q+v", lambda: W.lora_down_multi(
            x, [(lo["Aq"], lo["mq"], ks), (lo["Av"], lo["mv"], ks)], outs=[z["q"], z["v"]]),
         2 * g(m, r, D), m * D * 2 + 2 * m * D + 2 * r * D * 2 + 2 * m * r * 2, 1),
        ("lora_grads q+v", lambda: W.lora_grads_multi(x, lora_terms),
         g(m, r, D) * 3 + g(m, r, KV) * 2 + g(m, r, D), None, 1),
    ]
    # the step's form when the q|k|v dX reads the fp16 slot: dz alone, then the dX GEMM carrying
    # the column sums (dB, dA of both adapters) on its idle CUs
    carried_sums = "qkv" in st.ahead
    # the carried sums of dz = (dzq, dzv), set up without a launch of their own
    arr, mm, kk, rr, _, keep, res = W._lora_grads_args(
        x, lora_terms, [(torch.empty(r, D, device=x.device), torch.empty(n, r, device=x.device), dz_)
                        for n, dz_ in ((D, dzq), (KV, dzv))])
    pre = W.LoraSums(x, arr, mm, kk, rr, 2, keep, res)
    pzq, pzv = dzq, dzv
    rows += [
        ("lora_dz q+v", lambda: W.lora_dz_multi(x, lora_terms), g(m, r, D) + g(m, r, KV), None,
         int(carried_sums)),
        ("h16_linear_bwd_dx qkv+lora+sums", lambda: W.linear_backward_dx_lora(
            dy["qkv"], L["qkv"], [(pzq, lo["Aq"], lo["mq"], ks), (pzv, lo["Av"], lo["mv"], ks)],
            out=st.dx_qkv, w16=h["qkv"], sums=pre),
         g(m, D, QKV) + 2 * g(m, D, r) + 3 * g(m, r, D) + g(m, r, KV), None, int(carried_sums)),
    ]
    if carried_sums:   # the two launches these replace in the step
        rows = [(n, f, fl, nb, 0 if n in ("lora_grads q+v", "h16_linear_bwd_dx qkv+lora") else pl)
                for n, f, fl, nb, pl in rows]
    out = []
    for name, fn, flops, nbytes, per_layer in rows:
        if only is not None and name not in only:
            continue
        ms = time_op(torch, fn, reps) if EAGER else time_graph(torch, fn, iters=max(3, reps // 2))
        row = {"kernel": name, "avg_us": round(ms * 1e3, 2), "launches_per_layer": per_layer,
               "gflop": round(flops / 1e9, 3)}
        if flops:
            row["tflops"] = round(flops / (ms * 1e-3) / 1e12, 1)
            row["frac_fp16_peak"] = round(flops / (ms * 1e-3) / 1e12 / FP16_PEAK_TFLOPS, 4)
        if nbytes:
            row["gbps"] = round(nbytes / (ms * 1e-3) / 1e9, 1)
            row["frac_hbm_peak"] = round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)
        out.append(row)
    gu.copy_(gu_save)
    del h, hl
    return out


def neighbour_table(torch, reps, m=2048, d=1536, nq=12, nkv=2, hd=128, only=None):
    """The kernels on either side of the LoRA'd q/v linear (RMSNorm + dropout forward, its
    backward with the LoRA input grads, the QKV epilogue forward and backward, and the causal GQA
    attention that consumes the QKV buffer, on four sequences of M / 4 tokens), each in isolation
    at config 4's shapes (M tokens, hidden 1536, 12 query / 2 KV heads of 128), with their
    algorithmic HBM bytes (or, for the attention, FLOPs).  They are not part of the linear stack's
    step."""
    from decentrik_prime_amd import k_attn, k_head, k_norm, k_rope
    dev = "cuda"
    g = torch.Generator(device=dev)
    g.manual_seed(7)
    f16, f32 = torch.float16, torch.float32
    x = torch.randn(m, d, device=dev, generator=g)
    delta = torch.randn(m, d, device=dev, generator=g).half()
    w = torch.rand(d, device=dev, generator=g) + 0.5
    mq = (torch.rand(m, d, device=dev, generator=g) >= 0.05).to(torch.uint8)
    mv = (torch.rand(m, d, device=dev, generator=g) >= 0.05).to(torch.uint8)
    y, xq, xv = (torch.empty(m, d, dtype=f16, device=dev) for _ in range(3))
    xout, out = torch.empty(m, d, device=dev), torch.empty(m, d, device=dev)
    rstd = torch.empty(m, device=dev)
    dy16, lq, lv = (torch.randn(m, d, device=dev, generator=g).half() for _ in range(3))
    out16 = torch.empty(m, d, dtype=f16, device=dev)
    gs = torch.ones(1, device=dev)
    row = (nq + 2 * nkv) * hd
    qkv = torch.randn(m, row, device=dev, generator=g).half()
    lqq = torch.randn(m, nq * hd, device=dev, generator=g).half()
    lvv = torch.randn(m, nkv * hd, device=dev, generator=g).half()
    pos = torch.randint(0, 4096, (m,), device=dev, dtype=torch.int32, generator=g)
    ang = torch.arange(4096, device=dev, dtype=f32)[:, None] * (
        1.0 / (1e6 ** (torch.arange(0, hd, 2, device=dev, dtype=f32) / hd)))[None, :]
    cos, sin = torch.cat((ang, ang), 1).cos().contiguous(), torch.cat((ang, ang), 1).sin().contiguous()
    gin = nq // nkv
    dq = torch.randn(m, nq * hd, device=dev, generator=g)
    dk, dv = (torch.randn(m, nkv * gin * hd, device=dev, generator=g) for _ in range(2))
    qkv_out = torch.empty(m, row, dtype=f16, device=dev)
    lens = [m // 4] * 4
    meta = k_attn.meta_for(lens, dev)
    aqkv = (torch.randn(m, row, device=dev, generator=g) * 0.8).half()
    aout, alse = k_attn.attention_forward(aqkv, meta, nq, nkv, hd)
    adout = torch.randn(m, nq * hd, device=dev, generator=g).half()
    # causal: hd L (L + 1) FLOP per (sequence, head) for each of Q K^T and P V; the backward's
    # S, dP, dV, dK, dQ are 2.5 times that
    att_fwd = sum(2 * hd * L * (L + 1) for L in lens) * nq
    # LM head over Qwen2.5's 151,936-token vocabulary, every row with a target: the logits GEMM
    # and the P E accumulation, 2 M V D FLOP each
    vocab = 151936
    emb = (torch.randn(vocab, d, device=dev, generator=g) * 0.02).half()
    yh = torch.randn(m, d, device=dev, generator=g).half()
    tg = torch.randint(0, vocab, (m,), device=dev, dtype=torch.int32, generator=g)
    ident = torch.arange(m, device=dev, dtype=torch.int32)
    et = emb.index_select(0, tg.long()).contiguous()
    src = k_head.ResidentEmbedding(emb)
    head_flops = 2 * 2 * m * vocab * d
    e = m * d
    rows = [
        ("rms_fwd norm+dropout", lambda: k_norm.rms_forward(
            x, w, y, rstd, 1e-6, delta=delta, xout=xout, xq=xq, xv=xv, mq=mq, mv=mv,
            keep_scale=1 / 0.95), e * (4 + 2 + 1 + 1 + 4 + 2 + 2 + 2) + m * 4),
        ("rms_bwd norm+lora grads", lambda: k_norm.rms_backward(
            dy16, gs, x, w, rstd, out, dres=out, lq=lq, lv=lv, mq=mq, mv=mv, keep_scale=1 / 0.95,
            out16=out16, delta=delta), e * (2 + 4 + 2 + 2 + 2 + 1 + 1 + 4 + 4 + 2) + m * 4),
        ("qkv_epilogue_fwd lora+rope", lambda: k_rope.qkv_epilogue_forward(
            qkv, lqq, lvv, pos, cos, sin, 2.0, nq, nkv, hd),
         m * (row * 2 * 2 + (nq + nkv) * hd * 2 + hd * 4)),
        ("qkv_epilogue_bwd rope^T+gqa", lambda: k_rope.qkv_epilogue_backward(
            dq, dk, dv, pos, cos, sin, qkv_out, nq, nkv, hd, gin),
         m * (nq * hd * 4 + 2 * nkv * gin * hd * 4 + row * 2 + hd * 4)),
        ("attention_fwd causal gqa", lambda: k_attn.attention_forward(aqkv, meta, nq, nkv, hd),
         None, att_fwd),
        ("attention_bwd causal gqa", lambda: k_attn.attention_backward(
            aqkv, aout, alse, adout, meta, nq, nkv, hd), None, 2.5 * att_fwd),
        ("lm_head streamed loss+grad", lambda: k_head.streamed_head(
            yh, src, tg, ident, m, et, 1.0), None, head_flops),
    ]
    res = []
    for name, fn, nbytes, *flops in rows:
        if only is not None and name not in only:
            continue
        ms = time_op(torch, fn, reps) if EAGER else time_graph(torch, fn, iters=3, reps=max(2, reps // 4))
        if nbytes is None:
            tf = flops[0] / (ms * 1e-3) / 1e12
            res.append({"kernel": name, "avg_us": round(ms * 1e3, 2),
                        "gflop": round(flops[0] / 1e9, 3), "tflops": round(tf, 1),
                        "frac_fp16_peak": round(tf / FP16_PEAK_TFLOPS, 4)})
            continue
        gbps = nbytes / (ms * 1e-3) / 1e9
        res.append({"kernel": name, "avg_us": round(ms * 1e3, 2), "bytes": int(nbytes),
                    "gbps": round(gbps, 1), "frac_hbm_peak": round(gbps / HBM_PEAK_GBS, 4)})
    return res


def model_step(torch, layers, m, steps, warmup):
    """The whole Qwen2.5 QLoRA step around the linear stack (decentrik_prime_amd.model: norms,
    rotary q|k|v GEMM, causal GQA attention, SwiGLU MLP, the LM head over the 151,936-token
    vocabulary, and the backward to the LoRA gradients) on four sequences of m / 4 tokens: time
    per step, tokens per second, and algorithmic TFLOP/s (linear layers, attention, LM head)."""
    from decentrik_prime_amd.model import QwenQLoRAStep
    lens = [m // 4] * 4
    st = QwenQLoRAStep(lens, n_layers=layers, seed=0)
    for _ in range(warmup):
        st.step()
    torch.cuda.synchronize()
    e0, e1 = _events(torch)
    e0.record()
    for _ in range(steps):
        st.step()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    tf = st.flops_per_step / (ms * 1e-3) / 1e12
    loss = float(st.step())
    finite = math.isfinite(loss) and all(bool(torch.isfinite(g).all()) for gs in st.grads for g in gs)
    if not finite:
        raise RuntimeError(f"whole QLoRA step: non-finite loss or LoRA gradients (loss {loss})")
    res = {"workload": "Qwen2.5-1.5B QLoRA training step (embedding rows, 28 decoder layers, "
                       "final norm, LM head + cross-entropy, backward to the LoRA gradients)",
           "layers": layers, "lens": lens, "ms_per_step": round(ms, 3),
           "tokens_per_s": round(m / (ms * 1e-3), 1), "flop_per_step": st.flops_per_step,
           "tflops": round(tf, 1), "frac_fp16_peak": round(tf / FP16_PEAK_TFLOPS, 4),
           "loss_per_token": round(loss / st.n_lab, 4)}
    del st
    torch.cuda.empty_cache()
    return res


def dequant_bandwidth(torch, st, reps):
    """NF4 dequant of every layer into its own fp16 output (the working set, 3.30 GB of
    algorithmic traffic for 28 layers, does not fit the 256 MB Infinity Cache)."""
    from decentrik_prime_amd import k_nf4
    outs = [torch.empty(L["packed"].numel, dtype=torch.float16, device=st.device) for L in st.layers]

    def run():
        for L, out in zip(st.layers, outs):
            k_nf4.dequant_layer(L["packed"], st.code2, st.nf4, out)
    ms = time_op(torch, run, reps) if EAGER else time_graph(torch, run, iters=2, reps=max(2, reps // 2))
    n_weights = st.layers[0]["packed"].numel
    bytes_per_weight = 0.5 + 1 / 64 + 8 / 16384 + 2
    per_launch_bytes = n_weights * bytes_per_weight
    avg_launch_ms = ms / len(st.layers)
    gbps = per_launch_bytes / (avg_launch_ms * 1e-3) / 1e9
    del outs
    torch.cuda.empty_cache()
    return {"kernel": "nf4_dequant_kernel (dequant_layer)", "weights_per_launch": n_weights,
            "bytes_per_weight": bytes_per_weight, "bytes_per_launch": int(per_launch_bytes),
            "avg_us": round(avg_launch_ms * 1e3, 2), "gbps": round(gbps, 1),
            "frac_hbm_peak": round(gbps / HBM_PEAK_GBS, 4)}


def gemm_calibration(torch, m, reps, n=2 * 8960, k=1536):
    """torch.mm (hipBLASLt) of fp16 [m, k] x [k, n] (the gate|up forward's shape, no dequant, no
    epilogue), launched back to back (each call is ~140 us, far above the launch overhead; a
    library call is kept out of graph capture): the box's GEMM rate in this run, beside the
    step."""
    a = torch.randn(m, k, device="cuda").half()
    b = torch.randn(n, k, device="cuda").half()
    out = torch.empty(m, n, dtype=torch.float16, device="cuda")
    us = time_op(torch, lambda: torch.mm(a, b.t(), out=out), 10 * reps) * 1e3
    return {"kernel": f"torch.mm fp16 [{m}, {k}] x [{k}, {n}]", "avg_us": round(us, 2),
            "tflops": round(2 * m * n * k / (us * 1e-6) / 1e12, 1)}


def copy_calibration(torch, reps, nbytes=512 << 20):
    """A plain device copy of known size (read nbytes + write nbytes per launch): the reference
    against which rocprofv3's FETCH_SIZE / WRITE_SIZE counters are scaled."""
    a = torch.empty(nbytes, dtype=torch.uint8, device="cuda").fill_(1)
    b = torch.empty_like(a)
    ms = time_op(torch, lambda: b.copy_(a), reps)
    del a, b
    return {"kernel": "copy (torch)", "bytes_read": nbytes, "bytes_written": nbytes,
            "avg_us": round(ms * 1e3, 2), "gbps": round(2 * nbytes / (ms * 1e-3) / 1e9, 1)}


def cpu_baseline(layers=1, m=2048):
    """The CPU oracle on `layers` layer(s) of the same workload: numpy NF4 dequant of the seven
    weights + fp32 torch GEMMs of the forward and backward with the LoRA terms."""
    import numpy as np
    import torch
    from oracle import linear, mlp, nf4
    torch.set_num_threads(os.cpu_count())
    rng = np.random.default_rng(0)
    D, I, KV, r = 1536, 8960, 256, 16
    shapes = {"q": (D, D), "k": (KV, D), "v": (KV, D), "o": (D, D), "g": (2 * I, D), "d": (D, I)}
    qs = {}
    for name, shp in shapes.items():
        w = (rng.standard_normal(shp, dtype=np.float32) * 0.02).astype(np.float16)
        qs[name] = nf4.quantize(w)
    x = rng.standard_normal((m, D), dtype=np.float32).astype(np.float16)
    a = (rng.uniform(-1, 1, (r, D)) / np.sqrt(D)).astype(np.float16)
    bq = (rng.standard_normal((D, r)) * 0.02).astype(np.float16)
    bv = (rng.standard_normal((KV, r)) * 0.02).astype(np.float16)
    mask = (rng.random((m, D)) >= 0.05).astype(np.uint8)
    dys = {k: (rng.standard_normal((m, n), dtype=np.float32) * 1e-2).astype(np.float16)
           for k, n in (("q", D), ("k", KV), ("v", KV), ("o", D), ("d", D))}
    ks = linear.keep_scale(0.05)
    t0 = time.perf_counter()
    for _ in range(layers):
        wd = {k: nf4.dequant(q["packed"], q["qabs"], q["scale2"], q["offset2"], q["code2"]).reshape(shapes[k])
              for k, q in qs.items()}
        _, zq = linear.linear_fwd(x, wd["q"], None, mask, ks, a, bq, 2.0)
        linear.linear_fwd(x, wd["k"])
        _, zv = linear.linear_fwd(x, wd["v"], None, mask, ks, a, bv, 2.0)
        linear.linear_fwd(x, wd["o"])
        gu, h, _ = mlp.mlp_fwd(x, wd["g"], wd["d"])
        mlp.mlp_bwd(dys["d"], gu, wd["g"], wd["d"])
        linear.linear_bwd(dys["o"], wd["o"])
        linear.linear_bwd(dys["q"], wd["q"], zq, x, mask, ks, a, bq, 2.0)
        linear.linear_bwd(dys["k"], wd["k"])
        linear.linear_bwd(dys["v"], wd["v"], zv, x, mask, ks, a, bv, 2.0)
    dt = time.perf_counter() - t0
    from decentrik_prime_amd.stack import layer_flops
    flops = layers * layer_flops(m)
    return {"value": round(flops / dt / 1e12, 4), "unit": "TFLOP/s", "cores": torch.get_num_threads(),
            "kind": "port",
            "sample": f"{layers} layer(s) of config 4 fwd+bwd at M={m} (NF4 dequant + fp32 GEMMs), "
                      f"{dt:.2f} s; full 28-layer step extrapolated = {dt * 28 / layers:.1f} s",
            "cpu_model": _cpu_model(), "os_cpu_count": os.cpu_count()}


def _cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


# ---------------------------------------------------------------------------------------------
# rocprofv3 summaries (rocpd SQLite databases written by `rocprofv3 -d DIR -o run ...`)

def _short(name):
    """Kernel name without 'void', anonymous namespaces and the argument list (an Itanium-mangled
    name of this library's kernels is reduced to its identifier and integer/bool template
    arguments)."""
    import re
    if name.startswith("_Z"):
        m = re.search(r"(\d+)([A-Za-z_]\w*)", name[name.find("N_1") + 3:] if "N_1" in name else name[2:])
        if m:
            ident = m.group(2)[:int(m.group(1))]
            rest = m.group(2)[int(m.group(1)):]
            targs = re.findall(r"L([ib])(\d+)E", rest.split("EEv")[0]) if rest.startswith("I") else []
            vals = [("true" if v == "1" else "false") if t == "b" else v for t, v in targs]
            return ident + (f"<{', '.join(vals)}>" if vals else "")
        return name[:100]
    name = name.replace("(anonymous namespace)::", "")
    if name.startswith("void "):
        name = name[5:]
    depth, cut = 0, len(name)
    for i, ch in enumerate(name):   # cut at the '(' of the argument list (outside template <>)
        if ch == "<":
            depth += 1
        elif ch == ">":
            depth -= 1
        elif ch == "(" and depth == 0:
            cut = i
            break
    return re.sub(r"\s+", " ", name[:cut])[:100]


def summarize_trace(db, top=40, ops=()):
    """Per-kernel dispatch statistics of a kernel trace: calls, average and total duration,
    grouped by kernel name and grid (a kernel instance launched at several shapes is split).
    ops: [(operator, kernel-name substring, grid, (first, end[, step]) or None)] for which an
    'OPAVG' line is added (what bench.py reads back as the profile's average duration of that
    operator's kernel): the average over that kernel's dispatches at that grid, or over
    dispatches first, first + step, ... below end of them in launch order (bench.py's timed
    steps: warmup x 28 .. (warmup + steps) x 28 for a kernel launched once per layer; step 2 and
    an odd first pick the second of two operators that launch the same kernel at the same grid
    in each layer)."""
    import collections
    import sqlite3
    cur = sqlite3.connect(db).cursor()
    agg = collections.defaultdict(list)
    for name, dur, gx, gy, gz, wx, wy, wz in cur.execute(
            "select name, duration, grid_x, grid_y, grid_z, workgroup_x, workgroup_y, workgroup_z "
            "from kernels order by start"):
        wgs = (gx // max(wx, 1)) * (gy // max(wy, 1)) * (gz // max(wz, 1))
        agg[(_short(name), wgs, wx * wy * wz)].append(dur)
    total = sum(sum(v) for v in agg.values())
    lines = [f"SOURCES {source_digest()}",
             f"{'kernel':78s} {'wgs':>7s} {'wg':>4s} {'calls':>6s} {'avg_us':>9s} "
             f"{'total_ms':>9s} {'pct':>6s}"]
    for (k, wgs, wx), v in sorted(agg.items(), key=lambda kv: -sum(kv[1]))[:top]:
        lines.append(f"{k:78s} {wgs:7d} {wx:4d} {len(v):6d} {sum(v) / len(v) / 1e3:9.2f} "
                     f"{sum(v) / 1e6:9.3f} {100 * sum(v) / total:6.2f}")
    for op, pattern, grid, span in ops:
        sel = [(k, v) for k, v in agg.items() if pattern in k[0] and k[1] == grid]
        if sel:
            durs = [d for _, v in sel for d in v]
            if span is not None:
                durs = durs[span[0]:span[1]:span[2] if len(span) > 2 else 1]
            lines.append(f"OPAVG {op} | {sel[0][0][0]} | {grid} | {sum(durs) / len(durs) / 1e3:.2f} | "
                         f"{len(durs)}")
    return "\n".join(lines)


def _counter_by_dispatch(db, counter):
    import sqlite3
    cur = sqlite3.connect(db).cursor()
    rows = {}
    for did, name, grid, wg, val in cur.execute(
            "select dispatch_id, kernel_name, grid_size, workgroup_size, value "
            "from counters_collection where counter_name = ?", (counter,)):
        key = (did, _short(name), grid // max(wg, 1), wg)
        rows[key] = rows.get(key, 0.0) + val
    return rows


def _grid_sel(spec):
    """'substring#grid[,grid][first:end]' -> (substring, set of grids or None, (first, end) or
    None): the dispatch range picks, in launch order, among the matching dispatches (two
    operators that launch one kernel at one grid, run one after the other)."""
    span = None
    if spec.endswith("]"):
        spec, rng = spec[:-1].rsplit("[", 1)
        span = tuple(int(v) for v in rng.split(":"))
    wgs = None
    if "#" in spec:
        spec, w = spec.rsplit("#", 1)
        wgs = {int(v) for v in w.split(",")}
    return spec, wgs, span


def _pick(rows, pattern, wgs, span):
    """The dispatches (keyed by (dispatch id, kernel, grid, ...)) of `rows` that match, in
    dispatch order, cut to `span`."""
    sel = sorted((k, v) for k, v in rows.items()
                 if pattern in k[1] and (wgs is None or k[2] in wgs))
    return sel[span[0]:span[1]] if span is not None else sel


def summarize_pmc(fetch_db, write_db, groups, copy_bytes=512 << 20):
    """HBM traffic per operator call from a FETCH_SIZE run and a WRITE_SIZE run (KiB per
    dispatch), each scaled by what the same counter reads for the calibration copy of
    `copy_bytes` read + `copy_bytes` written (the __amd_rocclr_copyBuffer dispatches within a
    factor of two of the largest one: nothing else in the run copies a quarter as much).
    groups: [(operator name, kernel-name substring, operator calls in the run, set of grid sizes in
    workgroups or None for any, (first, end) dispatch range among the matching ones or None)]."""
    out = []
    scaled = {}
    for label, db, counter in (("fetch", fetch_db, "FETCH_SIZE"), ("write", write_db, "WRITE_SIZE")):
        rows = _counter_by_dispatch(db, counter)
        copies = [v for k, v in rows.items() if k[1].startswith("__amd_rocclr_copyBuffer")]
        if not copies:
            raise SystemExit(f"{db}: no {counter} value of a copy dispatch")
        kib = [v for v in copies if v >= 0.5 * max(copies)]
        kib_avg = sum(kib) / len(kib)
        factor = copy_bytes / (kib_avg * 1024.0)
        out.append(f"{counter}: calibration copy {copy_bytes} B -> {kib_avg:.0f} KiB per dispatch "
                   f"(n={len(kib)}), scale factor {factor:.4f}")
        for op, pattern, calls, wgs_only, span in groups:
            sel = dict(_pick(rows, pattern, wgs_only, span))
            per_kernel = {}
            for k, v in sel.items():
                per_kernel.setdefault((k[1], k[2]), []).append(v)
            for (name, wgs), vals in sorted(per_kernel.items()):
                out.append(f"  {op} | {name} wgs={wgs}: {len(vals)} dispatches, "
                           f"{sum(vals) / len(vals):.0f} KiB each (raw)")
            per_call = sum(sel.values()) * 1024.0 * factor / calls
            scaled[(op, label)] = per_call
            out.append(f"  {op}: {label} {per_call:.4g} B per operator call (scaled, {calls} calls)")
    for op, _, _, _, _ in groups:
        f, w = scaled[(op, "fetch")], scaled[(op, "write")]
        out.append(f"TRAFFIC {op} | fetch {f:.0f} | write {w:.0f} | total {f + w:.0f}")
    return "\n".join(out)


def _counters_by_dispatch(db):
    """{(dispatch id, kernel, grid in workgroups, workgroup size): {counter: (sum, max, n)}} over
    the counter's instances (SEs / XCDs) of each dispatch, and each dispatch's duration (ns) when
    the run also traced kernels."""
    import sqlite3
    cur = sqlite3.connect(db).cursor()
    out = {}
    for did, name, grid, wg, cname, val in cur.execute(
            "select dispatch_id, kernel_name, grid_size, workgroup_size, counter_name, value "
            "from counters_collection"):
        key = (did, _short(name), grid // max(wg, 1), wg)
        agg = out.setdefault(key, {})
        s_, m_, n_ = agg.get(cname, (0.0, float("-inf"), 0))
        agg[cname] = (s_ + val, max(m_, val), n_ + 1)
    dur = {}
    try:
        for did, start, end in cur.execute("select dispatch_id, start, end from kernels"):
            dur[did] = end - start
    except sqlite3.Error:
        pass
    return out, dur


def summarize_counters(db, groups, simds=1024, xcds=8, cus=256):
    """Counters per operator from one `rocprofv3 --pmc ... --kernel-trace` pass.

    Every counter the pass collected is listed per operator (mean over its dispatches of the sum
    over the counter's instances), then what follows from them where the pass has the inputs:
    - mfma_busy = SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE per XCD x SIMDs) (rocprofv3's
      MfmaUtil), mfma_GFLOP = SQ_INSTS_VALU_MFMA_MOPS_F16 x 512 (the FLOPs the hardware counted);
    - clock_GHz = GRBM_GUI_ACTIVE per XCD / kernel duration (GRBM_GUI_ACTIVE is stored summed over
      the XCDs, 8 on MI355X; its window also covers the dispatch's start and drain, which for
      kernels of ~20 us inflates the clock and deflates the busy fractions);
    - lds_read_B_per_clk_cu, lds_write_B_per_clk_cu: bytes moved by LDS instructions
      (SQ_INSTS_LDS_LOAD_BANDWIDTH / _STORE_BANDWIDTH, units of 64 bytes) per busy clock per CU;
    - lds_active = SQ_LDS_IDX_ACTIVE / (GRBM_GUI_ACTIVE per XCD x CUs): the fraction of clocks a
      CU's LDS works on indexed (ds_*) instructions; lds_conflict = SQ_LDS_BANK_CONFLICT over
      SQ_LDS_IDX_ACTIVE;
    - lds_wait = SQ_WAIT_INST_LDS / SQ_WAVE_CYCLES (both in quad-cycles per wave), any_wait =
      SQ_WAIT_INST_ANY / SQ_WAVE_CYCLES: the fraction of a wave's life spent waiting to issue an
      LDS instruction / any instruction;
    - ta_busy = TA_TA_BUSY_sum / (GRBM_GUI_ACTIVE per XCD x CUs): the texture-addresser (vector
      memory, LDS DMA included) busy fraction; dma_waves = TA_FLAT_READ_LDS_WAVEFRONTS_sum, the
      LDS-DMA load instructions.
    groups: [(operator name, kernel-name substring, grid in workgroups or None, algorithmic
    FLOP, (first, end) dispatch range among the matching ones or None)]."""
    rows, dur = _counters_by_dispatch(db)
    lines = []
    mean = lambda xs: sum(xs) / len(xs) if xs else float("nan")  # noqa: E731
    for op, pattern, wgs_only, algo, span in groups:
        sel = _pick(rows, pattern, None if wgs_only is None else {wgs_only}, span)
        if not sel:
            lines.append(f"{op}: (no dispatch of {pattern})")
            continue
        name, wgs = sel[0][0][1], sel[0][0][2]
        cnt = {}
        for _, v in sel:
            for c, (tot, _, _) in v.items():
                cnt.setdefault(c, []).append(tot)
        c = {k: mean(v) for k, v in cnt.items()}
        us = mean([dur[k[0]] / 1e3 for k, _ in sel if k[0] in dur and dur[k[0]] > 0])
        gui = c.get("GRBM_GUI_ACTIVE", 0.0) / xcds
        lines.append(f"{op} | {name} | {wgs} workgroups | {len(sel)} dispatches | "
                     f"{us:.2f} us | {(algo or 0) / 1e9:.2f} GFLOP algorithmic")
        for k in sorted(c):
            lines.append(f"    {k:36s} {c[k]:16.0f}")
        der = {}
        if gui > 0:
            if us == us:
                der["clock_ghz"] = gui / (us * 1e3)
            if "SQ_VALU_MFMA_BUSY_CYCLES" in c:
                der["mfma_busy"] = c["SQ_VALU_MFMA_BUSY_CYCLES"] / (gui * simds)
            if "SQ_INSTS_LDS_LOAD_BANDWIDTH" in c:
                der["lds_read_B_per_clk_cu"] = c["SQ_INSTS_LDS_LOAD_BANDWIDTH"] * 64 / (gui * cus)
            if "SQ_INSTS_LDS_STORE_BANDWIDTH" in c:
                der["lds_write_B_per_clk_cu"] = c["SQ_INSTS_LDS_STORE_BANDWIDTH"] * 64 / (gui * cus)
            if "SQ_LDS_IDX_ACTIVE" in c:
                der["lds_active"] = c["SQ_LDS_IDX_ACTIVE"] / (gui * cus)
            if "TA_TA_BUSY_sum" in c:
                der["ta_busy"] = c["TA_TA_BUSY_sum"] / (gui * cus)
        if c.get("SQ_LDS_IDX_ACTIVE"):
            der["lds_conflict"] = c.get("SQ_LDS_BANK_CONFLICT", 0.0) / c["SQ_LDS_IDX_ACTIVE"]
        if c.get("SQ_WAVE_CYCLES"):
            for cn, dn in (("SQ_WAIT_INST_LDS", "lds_wait"), ("SQ_WAIT_INST_ANY", "any_wait")):
                if cn in c:
                    der[dn] = c[cn] / c["SQ_WAVE_CYCLES"]
        if "SQ_INSTS_VALU_MFMA_MOPS_F16" in c:
            der["mfma_gflop"] = c["SQ_INSTS_VALU_MFMA_MOPS_F16"] * 512 / 1e9
        if "TA_FLAT_READ_LDS_WAVEFRONTS_sum" in c:
            der["dma_waves"] = c["TA_FLAT_READ_LDS_WAVEFRONTS_sum"]
        if der:
            lines.append("COUNTERS " + op + " | " + " | ".join(
                f"{k} {v:.4g}" for k, v in der.items()))
        if "mfma_busy" in der:   # the line the MFMA summary has always had
            lines.append(f"MFMA {op} | busy {der['mfma_busy']:.4f} | clock_ghz "
                         f"{der.get('clock_ghz', float('nan')):.3f} | avg_us {us:.2f}")
    return "\n".join(lines)


def source_digest():
    """Digest of the kernel sources (csrc/*.hip, csrc/*.h, include/dk.h): a profile summary carries
    the digest of the sources it was taken on, so a figure read back from it is labelled stale
    once the kernels change."""
    import glob
    import hashlib
    here = os.path.dirname(os.path.abspath(__file__))
    h = hashlib.sha256()
    files = sorted(glob.glob(os.path.join(here, "decentrik_prime_amd", "csrc", "*.hip")) +
                   glob.glob(os.path.join(here, "decentrik_prime_amd", "csrc", "*.h")) +
                   [os.path.join(here, "include", "dk.h")])
    for f in files:
        h.update(os.path.basename(f).encode())
        h.update(open(f, "rb").read())
    return h.hexdigest()[:16]


def committed_kernel_avg(op):
    """Average duration (us) of operator `op`'s kernel in the committed rocprof kernel-trace summary
    (an 'OPAVG op | kernel | wgs | avg_us | calls' line), the summary's path, the source digest it
    records ('SOURCES <digest>' line) and whether that is the digest of the sources now, or
    None."""
    import glob
    here = os.path.dirname(os.path.abspath(__file__))
    for path in sorted(glob.glob(os.path.join(here, "profiles", "*.txt"))):
        lines = open(path).read().splitlines()
        digest = next((l.split()[1] for l in lines if l.startswith("SOURCES ")), None)
        for line in lines:
            if line.startswith("OPAVG ") and line[6:].split(" | ")[0] == op:
                parts = [x.strip() for x in line[6:].split(" | ")]
                return {"avg_us": float(parts[3]), "kernel": parts[1], "wgs": int(parts[2]),
                        "calls": int(parts[4]), "source": os.path.relpath(path, here),
                        "sources_digest": digest, "sources_match": digest == source_digest()}
    return None


def committed_traffic(op):
    """HBM bytes per call of `op` from the TRAFFIC lines of the committed profile summaries."""
    import glob
    here = os.path.dirname(os.path.abspath(__file__))
    for path in sorted(glob.glob(os.path.join(here, "profiles", "*.txt"))):
        for line in open(path):
            if line.startswith("TRAFFIC ") and line[8:].split(" | ")[0] == op:
                parts = line.strip().split(" | ")
                return {"bytes": int(parts[3].split()[1]), "fetch": int(parts[1].split()[1]),
                        "write": int(parts[2].split()[1]),
                        "source": os.path.relpath(path, here)}
    return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--layers", type=int, default=28)
    ap.add_argument("--m", type=int, default=2048)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-layers", type=int, default=6,
                    help="layers of the CPU-oracle sample (about 10-30 s of CPU work)")
    ap.add_argument("--no-kernels", action="store_true")
    ap.add_argument("--no-model", action="store_true",
                    help="skip the whole-model step (norms, attention, LM head around the stack)")
    ap.add_argument("--reps", type=int, default=20)
    ap.add_argument("--eager", action="store_true",
                    help="time operators by plain back-to-back launches instead of CUDA-graph replays "
                         "(rocprofv3 counter runs: each operator call is then one dispatch per kernel)")
    ap.add_argument("--no-configs", action="store_true",
                    help="skip the BASELINE configs 0-3 rows (GPU, CPU oracle, parity)")
    ap.add_argument("--kernels-only", action="store_true",
                    help="skip the step timing: per-kernel table, dequant and a copy of known size "
                         "(the calibration of rocprofv3 FETCH_SIZE / WRITE_SIZE)")
    ap.add_argument("--op", default=None,
                    help="with --kernels-only: comma-separated operator names to run "
                         "('dequant' for the dequant) instead of the whole table")
    ap.add_argument("--summarize-trace", metavar="DB",
                    help="print the per-kernel table of a rocprofv3 kernel-trace database")
    ap.add_argument("--summarize-pmc", nargs=2, metavar=("FETCH_DB", "WRITE_DB"),
                    help="print HBM traffic per operator call from FETCH_SIZE / WRITE_SIZE runs")
    ap.add_argument("--op-avg", action="append", default=[],
                    help="with --summarize-trace: 'operator=kernel-name substring#grid"
                         "[first:end[:step]]' for an OPAVG line (the dispatch range is optional)")
    ap.add_argument("--summarize-counters", metavar="DB",
                    help="print MFMA busy, clock and MFMA FLOPs per operator from a PMC run")
    ap.add_argument("--group", action="append", default=[],
                    help="with --summarize-pmc / --summarize-counters: 'operator=kernel-name "
                         "substring[#grid[,grid]][[first:end]]@calls' (or @GFLOP; grid: only "
                         "dispatches of that many workgroups; [first:end]: those of the matching "
                         "dispatches, in launch order)")
    args = ap.parse_args()
    global EAGER
    EAGER = args.eager
    if args.summarize_trace:
        ops = []
        for o in args.op_avg:   # 'operator=kernel substring#grid[first:end[:step]]'
            op, rest = o.split("=", 1)
            pattern, grid = rest.rsplit("#", 1)
            span = None
            if "[" in grid:
                grid, rng = grid.rstrip("]").split("[")
                span = tuple(int(v) for v in rng.split(":"))
            ops.append((op, pattern, int(grid), span))
        print(summarize_trace(args.summarize_trace, ops=ops))
        return
    if args.summarize_counters:
        groups = []
        for g in args.group:   # 'operator=kernel substring[#grid][[first:end]]@GFLOP'
            op, rest = g.split("=", 1)
            pattern, gflop = rest.rsplit("@", 1)
            pattern, wgs, span = _grid_sel(pattern)
            groups.append((op, pattern, None if wgs is None else min(wgs), float(gflop) * 1e9,
                           span))
        print(summarize_counters(args.summarize_counters, groups))
        return
    if args.summarize_pmc:
        groups = []
        for g in args.group:   # one grid, or several: '#240,3072'; a range: '#192[0:3]'
            op, rest = g.split("=", 1)
            pattern, calls = rest.rsplit("@", 1)
            pattern, wgs, span = _grid_sel(pattern)
            groups.append((op, pattern, int(calls), wgs, span))
        print(summarize_pmc(*args.summarize_pmc, groups))
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: the NF4 linear path has no multi-GPU leg in this build "
              "(it would shard data-parallel over packed tokens with one LoRA-gradient all-reduce)",
              file=sys.stderr)
        sys.exit(2)

    import torch
    from decentrik_prime_amd.stack import NF4LinearStack
    torch.cuda.set_device(0)
    print(f"[bench] building {args.layers}-layer NF4 stack, M={args.m}", file=sys.stderr, flush=True)
    st = NF4LinearStack(args.layers, args.m, seed=0, device="cuda")
    torch.cuda.synchronize()
    if args.kernels_only:
        only = set(args.op.split(",")) if args.op else None
        res = {"kernels": kernel_table(torch, st, args.reps, only),
               "neighbours": neighbour_table(torch, args.reps, args.m, only=only)}
        if only is None or "dequant" in only:
            res["dequant"] = dequant_bandwidth(torch, st, args.reps)
        res["copy"] = copy_calibration(torch, args.reps)
        res["calls_per_operator"] = args.reps + 1
        print(json.dumps(res), flush=True)
        return
    for _ in range(args.warmup):
        st.step()
    torch.cuda.synchronize()
    print("[bench] warmup done", file=sys.stderr, flush=True)
    # the timed steps right after the warmup, so that in a kernel trace of this run they are
    # dispatches [warmup x 28, (warmup + steps) x 28) of each once-per-layer kernel.  The
    # dominant operator's launches are timed inside the last one (events in every step would cost
    # the step about 3%): the gate|up forward, which the per-operator table run afterwards
    # confirms (another dominant operator gets a probe step of its own after the timed ones)
    probe = (st.op_name("gu", DOMINANT), []) if not args.no_kernels else None
    torch.cuda.synchronize()
    e0, e1 = _events(torch)
    t0 = time.perf_counter()
    e0.record()
    for k in range(args.steps):
        if probe is not None and k == args.steps - 1:
            st.probe = probe
        st.step()
    e1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    st.probe = None
    kernels = None
    if not args.no_kernels:
        kernels = kernel_table(torch, st, args.reps)
        dom = max(kernels, key=lambda r: r["avg_us"] * r["launches_per_layer"])
        print(f"[bench] kernel table done; dominant operator {dom['kernel']}", file=sys.stderr,
              flush=True)
        if dom["kernel"] != probe[0]:
            probe = (dom["kernel"], [])
            st.probe = probe
            st.step()
            torch.cuda.synchronize()
            st.probe = None
    ms_per_step = e0.elapsed_time(e1) / args.steps
    value = st.flops_per_step / (ms_per_step * 1e-3) / 1e12
    # the last step's outputs and every layer's LoRA gradients must be finite
    checked = [st.out[k] for k in ("qkv", "o", "y")] + [st.dx_qkv, st.dx_o, st.dx_mlp]
    checked += [g for gs in st.grads for g in gs]
    if not all(bool(torch.isfinite(t.float()).all()) for t in checked):
        raise RuntimeError("linear stack: non-finite outputs or LoRA gradients")
    print(f"[bench] {ms_per_step:.3f} ms/step, {value:.1f} TFLOP/s (wall {wall:.2f} s)",
          file=sys.stderr, flush=True)

    result = {
        "metric": "NF4 QLoRA linear fwd+bwd TFLOP/s (M=2048, Qwen2.5-1.5B); dequant GB/s",
        "value": round(value, 2), "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_per_step, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "fp16", "data": "synthetic",
        "config": {"workload": "config 4: Qwen2.5-1.5B NF4 linear stack fwd+bwd",
                   "layers": args.layers, "m_tokens": args.m, "lora_rank": 16, "lora_alpha": 32,
                   "lora_dropout": 0.05, "lora_on": ["q_proj", "v_proj"],
                   "flop_per_step": st.flops_per_step},
    }
    if kernels is not None:
        name, events = probe
        live_ms = sum(a.elapsed_time(b) for a, b in events) / len(events)
        achieved = dom["gflop"] * 1e9 / (live_ms * 1e-3) / 1e12
        traffic = committed_traffic(name)
        prof = committed_kernel_avg(name)
        result["roofline"] = {
            "kernel": name, "bound": "mfma", "achieved": round(achieved, 1),
            "peak": FP16_PEAK_TFLOPS, "unit": "TFLOP/s", "frac": round(achieved / FP16_PEAK_TFLOPS, 4),
            "traffic": traffic["bytes"] if traffic else None,
            "per_launch": f"{dom['gflop']} GFLOP algorithmic / {live_ms * 1e3:.2f} us average over "
                          f"{len(events)} launches inside the last timed step (HIP events on the "
                          f"launch stream); {dom['avg_us']} us in isolation",
            "traffic_source": (f"{traffic['source']}: FETCH_SIZE {traffic['fetch']} B + WRITE_SIZE "
                               f"{traffic['write']} B per call, scaled by a copy of known size")
                              if traffic else None}
        if prof:
            # the committed trace's figure, labelled with whether it was taken on these sources
            a_prof = dom["gflop"] * 1e9 / (prof["avg_us"] * 1e-6) / 1e12
            result["roofline"]["committed_profile"] = {
                **prof, "frac": round(a_prof / FP16_PEAK_TFLOPS, 4),
                "note": f"{prof['kernel']} ({prof['wgs']} workgroups) average {prof['avg_us']} us "
                        f"over {prof['calls']} dispatches of the traced bench run -> "
                        f"{a_prof:.1f} TFLOP/s"}
            if prof["sources_match"]:
                result["roofline"]["frac_rocprof"] = round(a_prof / FP16_PEAK_TFLOPS, 4)
        # the box's GEMM clock in this run: hipBLASLt (torch.mm, fp16) at the gate|up shape, so a
        # step time can be compared across boxes whose power-limited clocks differ
        mm = gemm_calibration(torch, args.m, max(3, args.reps // 4))
        mm["step_tflops_over_mm"] = round(value / mm["tflops"], 4)
        result["gemm_clock"] = mm
        print(f"[bench] torch.mm gate|up shape {mm['avg_us']} us, {mm['tflops']} TFLOP/s",
              file=sys.stderr, flush=True)
        dq = dequant_bandwidth(torch, st, max(3, args.reps // 4))
        print(f"[bench] dequant {dq['gbps']} GB/s", file=sys.stderr, flush=True)
        dq_traffic = committed_traffic("dequant layer")
        result["dequant"] = {**dq, "roofline": {"bound": "hbm", "achieved": dq["gbps"],
                                                "peak": HBM_PEAK_GBS, "unit": "GB/s",
                                                "frac": dq["frac_hbm_peak"],
                                                "traffic": dq_traffic["bytes"] if dq_traffic else None}}
        # beside the graph-replayed figure (which includes the gaps between the 28 launches): the
        # kernel's own average duration in the committed trace of the default bench command
        # the practical ceiling beside it: a plain 512 MiB device copy (read + write) on this box
        cp = copy_calibration(torch, max(3, args.reps // 4))
        result["dequant"]["copy_gbps"] = cp["gbps"]
        result["dequant"]["frac_of_copy"] = round(dq["gbps"] / cp["gbps"], 4)
        dq_prof = committed_kernel_avg("dequant layer")
        if dq_prof:
            g_prof = dq["bytes_per_launch"] / (dq_prof["avg_us"] * 1e-6) / 1e9
            result["dequant"]["roofline"]["committed_profile"] = {
                **dq_prof, "frac": round(g_prof / HBM_PEAK_GBS, 4),
                "note": f"{dq_prof['kernel']} ({dq_prof['wgs']} workgroups) average "
                        f"{dq_prof['avg_us']} us over {dq_prof['calls']} dispatches -> "
                        f"{g_prof:.1f} GB/s"}
            if dq_prof["sources_match"]:
                result["dequant"]["roofline"]["frac_rocprof"] = round(g_prof / HBM_PEAK_GBS, 4)
        result["kernels"] = kernels
        result["neighbours"] = neighbour_table(torch, args.reps, args.m)
        print("[bench] " + ", ".join(
            f"{r['kernel']} {r['avg_us']} us " + (f"{r['gbps']} GB/s" if "gbps" in r
                                                  else f"{r['tflops']} TFLOP/s")
            for r in result["neighbours"]), file=sys.stderr, flush=True)
    if not args.no_configs:
        result["configs"] = config_rows(torch, st, cpu=not args.no_cpu)
    if not args.no_model:
        del st
        torch.cuda.empty_cache()
        result["model_step"] = model_step(torch, args.layers, args.m, args.steps, args.warmup)
        ms = result["model_step"]
        print(f"[bench] whole QLoRA step {ms['ms_per_step']} ms, {ms['tokens_per_s']} tokens/s, "
              f"{ms['tflops']} TFLOP/s", file=sys.stderr, flush=True)
    if not args.no_cpu:
        print(f"[bench] CPU baseline (oracle, {args.cpu_layers} layers)", file=sys.stderr, flush=True)
        result["cpu_baseline"] = cpu_baseline(args.cpu_layers, args.m)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
