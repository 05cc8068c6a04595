"""Config 4 at its real size: the bench's 28-layer NF4 linear stack (M = 2048, whole-layer dequant
launches, the default schedule), two steps.

Every layer's forward outputs, backward dX, saved/overwritten gate|up buffer and LoRA gradients
are checked bit-identical
  * to the same stack run with the carried schedule (``ahead="carried"``), which moves the
    backward's dequant into the GEMM launches and alternates two slots, so a wrong slot, a wrong
    layer or an ordering error in it changes a result here (every layer has different weights);
  * between the two steps (the slots then hold other layers at the start of each pass).
Layers 0, 13 and 27 are also checked against the CPU oracle (solution/fast_qwen.py:943-947,
1037, 1080-1112, 1310-1383 restated in oracle/linear.py and oracle/mlp.py) on the GPU-dequantised
weights (bit-exact with the oracle's dequant, which layer 13's whole packed buffer re-checks
here): forward outputs at rtol 1e-2 / atol 2e-2 on the values, gradients at rtol 1e-2 / atol 2e-2
of each gradient's scale.
"""

import numpy as np
import pytest

from tests.helpers import assert_close, host, log

pytestmark = pytest.mark.gpu
N_LAYERS, M = 28, 2048
D, I, KV = 1536, 8960, 256
QKV = D + 2 * KV
ORACLE_LAYERS = (0, 13, 27)


@pytest.fixture(scope="module")
def torch():
    import torch as t
    return t


def _run(torch, ahead, steps=2):
    """Two steps of the bench's stack, layer by layer as NF4LinearStack.step does, with every
    layer's results copied out.  Returns (stack, [per step: {name: tensor}])."""
    from decentrik_prime_amd.stack import NF4LinearStack
    st = NF4LinearStack(N_LAYERS, M, seed=0, device="cuda", ahead=ahead)
    runs = []
    for _ in range(steps):
        res = {}
        for i in range(N_LAYERS):
            st.forward_layer(i)
            for k in ("qkv", "o", "y"):
                res[f"L{i}.{k}"] = st.out[k].clone()
            res[f"L{i}.act"] = st.act.clone()
            res[f"L{i}.gu"] = st.gu[i].clone()
            res[f"L{i}.zq"] = st.z[i]["q"].clone()
            res[f"L{i}.zv"] = st.z[i]["v"].clone()
        for i in reversed(range(N_LAYERS)):
            st.backward_layer(i)
            res[f"L{i}.dgu"] = st.gu[i].clone()
            res[f"L{i}.dx_mlp"] = st.dx_mlp.clone()
            res[f"L{i}.dx_o"] = st.dx_o.clone()
            res[f"L{i}.dx_qkv"] = st.dx_qkv.clone()
            for name, g in zip(("dAq", "dBq", "dAv", "dBv"), st.grads[i]):
                res[f"L{i}.{name}"] = g.clone()
        torch.cuda.synchronize()
        runs.append(res)
    return st, runs


def _same(a, b, what):
    assert a.shape == b.shape and a.dtype == b.dtype, what
    if not bool(torch_equal_bits(a, b)):
        diff = (a.float() != b.float()).sum().item()
        raise AssertionError(f"{what}: {diff} of {a.numel()} elements differ")


def torch_equal_bits(a, b):
    import torch
    return torch.equal(a.contiguous().view(torch.uint8), b.contiguous().view(torch.uint8))


def _close(got, want, what):
    """Gradients: rtol 1e-2 / atol 2e-2 of the output's scale (dY ~ N(0, 1e-2) makes them
    small-valued, so an absolute 2e-2 would accept anything)."""
    want = np.asarray(want, np.float64)
    s = float(np.abs(want).max()) or 1.0
    assert_close(np.asarray(got, np.float64) / s, want / s, 1e-2, 2e-2, what)


def _abs(got, want, what):
    """Forward outputs (of order 1): rtol 1e-2 / atol 2e-2 on the values themselves."""
    assert_close(np.asarray(got, np.float64), np.asarray(want, np.float64), 1e-2, 2e-2, what)


@pytest.fixture(scope="module")
def runs(torch):
    log(f"config 4: {N_LAYERS}-layer stack, M={M}, whole-layer vs carried schedule, 2 steps")
    st, base = _run(torch, "layer")
    carried = _run(torch, "carried")[1]
    return st, base, carried


def test_config4_carried_matches_whole_layer_schedule(runs):
    st, base, carried = runs
    for step in range(2):
        assert carried[step].keys() == base[step].keys()
        for name, t in carried[step].items():
            _same(t, base[step][name], f"step {step} {name} (carried vs layer)")
    for name, t in base[1].items():
        _same(t, base[0][name], f"{name} (step 1 vs step 0)")


def test_config4_finite(runs, torch):
    st, base, _ = runs
    for name, t in base[1].items():
        assert bool(torch.isfinite(t.float()).all()), f"{name}: non-finite values"


@pytest.mark.parametrize("layer", ORACLE_LAYERS)
def test_config4_layer_vs_oracle(runs, torch, layer):
    """One layer of the bench's stack against the CPU oracle on the same weights and inputs."""
    from decentrik_prime_amd import k_nf4
    from oracle import linear, mlp, nf4
    st, base, _ = runs
    log(f"config 4: layer {layer} vs oracle")
    res = base[0]
    pk = st.layers[layer]["packed"]
    w_all = torch.empty(pk.numel, dtype=torch.float16, device="cuda")
    k_nf4.dequant_layer(pk, st.code2, st.nf4, w_all)
    w_all = host(w_all)
    if layer == 13:
        # the whole packed layer through the oracle's dequant: bit-exact
        p, q, s2, o2 = (host(t) for t in (pk.packed, pk.qabs, pk.scale2, pk.offset2))
        want = nf4.dequant(p, q, s2, o2, host(st.code2))
        assert np.array_equal(w_all.view(np.uint16), want.view(np.uint16)), "layer dequant"
    seg = pk.segments

    def wmat(name, rows, cols):
        e0 = seg[name][0]
        return w_all[e0:e0 + rows * cols].reshape(rows, cols)

    wqkv = np.concatenate([wmat("q_proj", D, D), wmat("k_proj", KV, D), wmat("v_proj", KV, D)])
    wo = wmat("o_proj", D, D)
    wgu = np.concatenate([wmat("gate_proj", I, D), wmat("up_proj", I, D)])
    wd = wmat("down_proj", D, I)
    lo = {k: host(v) for k, v in st.lora[layer].items()}
    x = host(st.x)
    ks, s = st.keep_scale, st.s
    dy = {k: host(v) for k, v in st.dy.items()}

    # forward: q|k|v with the q and v LoRA terms on their column ranges, o, gate|up + SwiGLU, down
    yq, zq = linear.linear_fwd(x, wqkv[:D], lo["bias"][:D], lo["mq"], ks, lo["Aq"], lo["Bq"], s)
    yk, _ = linear.linear_fwd(x, wqkv[D:D + KV], lo["bias"][D:D + KV])
    yv, zv = linear.linear_fwd(x, wqkv[D + KV:], lo["bias"][D + KV:], lo["mv"], ks, lo["Av"],
                               lo["Bv"], s)
    _abs(host(res[f"L{layer}.zq"]), zq, f"L{layer} z_q")
    _abs(host(res[f"L{layer}.zv"]), zv, f"L{layer} z_v")
    _abs(host(res[f"L{layer}.qkv"]), np.concatenate([yq, yk, yv], 1), f"L{layer} qkv")
    _abs(host(res[f"L{layer}.o"]), linear.linear_fwd(x, wo)[0], f"L{layer} o")
    gu, h, y = mlp.mlp_fwd(x, wgu, wd)
    _abs(host(res[f"L{layer}.gu"]), gu, f"L{layer} gu")
    _abs(host(res[f"L{layer}.act"]), h, f"L{layer} act")
    _abs(host(res[f"L{layer}.y"]), y, f"L{layer} y")

    # backward: down^T + SwiGLU', gate|up dX, o dX, the q and v LoRA gradients, q|k|v dX with both
    # masked LoRA input terms (the GPU's saved gu is the forward input of the SwiGLU backward)
    dgu, dx_mlp = mlp.mlp_bwd(dy["d"], host(res[f"L{layer}.gu"]), wgu, wd)
    _close(host(res[f"L{layer}.dgu"]), dgu, f"L{layer} dgu")
    _close(host(res[f"L{layer}.dx_mlp"]), dx_mlp, f"L{layer} dx_mlp")
    _close(host(res[f"L{layer}.dx_o"]), linear.linear_bwd(dy["o"], wo)["dx"], f"L{layer} dx_o")
    zq_gpu, zv_gpu = host(res[f"L{layer}.zq"]), host(res[f"L{layer}.zv"])
    gq = linear.linear_bwd(dy["qkv"][:, :D], wqkv[:D], zq_gpu, x, lo["mq"], ks, lo["Aq"], lo["Bq"], s)
    gv = linear.linear_bwd(dy["qkv"][:, D + KV:], wqkv[D + KV:], zv_gpu, x, lo["mv"], ks, lo["Av"],
                           lo["Bv"], s)
    for name, want in (("dAq", gq["dA"]), ("dBq", gq["dB"]), ("dAv", gv["dA"]), ("dBv", gv["dB"])):
        _close(host(res[f"L{layer}.{name}"]), want, f"L{layer} {name}")
    f32 = np.float32
    dxb = linear.mm16(dy["qkv"], wqkv).astype(f32)
    tq = np.where(lo["mq"] != 0, (gq["lx"].astype(f32) * f32(ks)).astype(f32), f32(0))
    tv = np.where(lo["mv"] != 0, (gv["lx"].astype(f32) * f32(ks)).astype(f32), f32(0))
    _close(host(res[f"L{layer}.dx_qkv"]), (dxb + tq + tv).astype(f32), f"L{layer} dx_qkv")
